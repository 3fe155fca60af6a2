"""Second, independent restatement of the Q4 formats in numpy / pure Python.

TEST INFRASTRUCTURE ONLY (checks the C oracle in q4_oracle.c).  Written from
the format specification in the reference's DESIGN.md:322-380 (Q4_0) and
DESIGN.md:436-520 (Q4_K_M) rather than from the C code, so that a shared
mistake is unlikely.  numpy float16 provides the IEEE binary16 conversions;
float32 arithmetic is done with numpy float32 scalars/arrays (one rounding
per operation, no fused multiply-add).
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


# ---- scales: get_scale_min_k4 written as a 96-bit field extraction ---------
def scale_min_k4(scales: np.ndarray, j: int) -> tuple[int, int]:
    """(sc, m) of sub-block j from the 12-byte scales field.

    Layout (DESIGN.md:456-470): bytes 0..3 hold sc[0..3] in their low 6 bits
    and the high 2 bits of sc[4..7]; bytes 4..7 hold m[0..3] in their low 6
    bits and the high 2 bits of m[4..7]; bytes 8..11 hold the low nibble of
    sc[4..7] (bits 0-3) and of m[4..7] (bits 4-7).
    """
    s = [int(v) for v in scales]
    if j < 4:
        return s[j] & 0x3F, s[4 + j] & 0x3F
    i = j - 4
    sc = (s[8 + i] & 0x0F) + 16 * (s[i] >> 6)
    m = (s[8 + i] >> 4) + 16 * (s[4 + i] >> 6)
    return sc, m


def scale_min_table(q4k_sb: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Vectorised (sc, m) for every superblock (rows of 144 bytes) and j."""
    s = q4k_sb[:, 4:16].astype(np.int64)
    sc = np.empty((s.shape[0], 8), dtype=np.int64)
    m = np.empty_like(sc)
    sc[:, 0:4] = s[:, 0:4] & 0x3F
    m[:, 0:4] = s[:, 4:8] & 0x3F
    sc[:, 4:8] = (s[:, 8:12] & 0x0F) + 16 * (s[:, 0:4] >> 6)
    m[:, 4:8] = (s[:, 8:12] >> 4) + 16 * (s[:, 4:8] >> 6)
    return sc, m


# ---- dequantisation ---------------------------------------------------------
def q4k_dequant(q: np.ndarray) -> np.ndarray:
    """Q4_K_M superblocks (n*144 bytes) -> n*256 float32 weights."""
    sbs = np.asarray(q, dtype=np.uint8).reshape(-1, 144)
    d = sbs[:, 0:2].copy().view("<f2").astype(F32).reshape(-1)
    dmin = sbs[:, 2:4].copy().view("<f2").astype(F32).reshape(-1)
    sc, m = scale_min_table(sbs)
    qs = sbs[:, 16:144].reshape(-1, 4, 32)           # chunk c, byte l
    lo = (qs & 0x0F).astype(F32)                       # sub-block 2c
    hi = (qs >> 4).astype(F32)                         # sub-block 2c+1
    out = np.empty((sbs.shape[0], 4, 2, 32), dtype=F32)
    for c in range(4):
        d1 = d * sc[:, 2 * c].astype(F32)
        m1 = dmin * m[:, 2 * c].astype(F32)
        d2 = d * sc[:, 2 * c + 1].astype(F32)
        m2 = dmin * m[:, 2 * c + 1].astype(F32)
        out[:, c, 0, :] = d1[:, None] * lo[:, c, :] - m1[:, None]
        out[:, c, 1, :] = d2[:, None] * hi[:, c, :] - m2[:, None]
    return out.reshape(-1)


# ---- Q5_K / Q6_K (ggml k-quants), from each weight's point of view -----------
# Element e of a superblock is traced to the byte, nibble and bit it comes
# from (ggml block_q5_K / block_q6_K layouts), instead of looping over the
# packed bytes as the C oracle does.
def _q6k_sources():
    e = np.arange(256)
    n, r = e // 128, e % 128
    part, l = r // 32, r % 32               # part 0..3: q1..q4 of ggml's loop
    ql_byte = 64 * n + l + 32 * (part % 2)  # parts 1 and 3 read ql[l + 32]
    ql_shift = 4 * (part // 2)              # parts 2 and 3 take the high nibble
    qh_byte = 128 + 32 * n + l
    qh_shift = 2 * part
    sc_byte = 192 + 8 * n + l // 16 + 2 * part
    return ql_byte, ql_shift, qh_byte, qh_shift, sc_byte


def q6k_dequant(q: np.ndarray) -> np.ndarray:
    """Q6_K, 210-byte superblocks: w = d * sc * (q6 - 32); every product is exact."""
    b = np.asarray(q, dtype=np.uint8).reshape(-1, 210).astype(np.int64)
    ql_b, ql_s, qh_b, qh_s, sc_b = _q6k_sources()
    q6 = ((b[:, ql_b] >> ql_s) & 0xF) | (((b[:, qh_b] >> qh_s) & 3) << 4)
    sc = b[:, sc_b]
    sc = np.where(sc >= 128, sc - 256, sc)  # int8
    d = b[:, 208:210].astype(np.uint8).copy().view(np.float16).astype(np.float64)
    w = d * sc * (q6 - 32)  # exact in f64, and representable in f32
    return w.astype(np.float32).reshape(-1)


def q5k_dequant(q: np.ndarray) -> np.ndarray:
    """Q5_K, 176-byte superblocks: w = RN_f32(d*sc*q5 - dmin*m), q5 = nibble + 16*qh bit."""
    b = np.asarray(q, dtype=np.uint8).reshape(-1, 176)
    e = np.arange(256)
    j, hi, l = e // 64, (e % 64) // 32, e % 32
    bi = b.astype(np.int64)
    nib = (bi[:, 48 + 32 * j + l] >> (4 * hi)) & 0xF
    bit = (bi[:, 16 + l] >> (2 * j + hi)) & 1
    q5 = nib + 16 * bit
    header = np.concatenate([b[:, :16], np.zeros((b.shape[0], 128), np.uint8)], axis=1)
    sc_t, m_t = scale_min_table(header)       # same 12-byte scales field as Q4_K
    sub = 2 * j + hi
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)
    d1 = d * sc_t[:, sub].astype(np.float32)          # exact
    m1 = dmin * m_t[:, sub].astype(np.float32)        # exact
    prod = (d1.astype(np.float64) * q5).astype(np.float32)  # exact
    return (prod - m1).astype(np.float32).reshape(-1)  # one f32 rounding


def q4_0_dequant(q: np.ndarray) -> np.ndarray:
    """Q4_0 blocks (n*18 bytes) -> n*32 float32 weights."""
    blk = np.asarray(q, dtype=np.uint8).reshape(-1, 18)
    d = blk[:, 0:2].copy().view("<f2").astype(F32).reshape(-1)
    qs = blk[:, 2:18]
    lo = (qs & 0x0F).astype(F32) - F32(8)
    hi = (qs >> 4).astype(F32) - F32(8)
    out = np.concatenate([lo * d[:, None], hi * d[:, None]], axis=1)
    return out.reshape(-1)


# ---- dot products in the reference order (pure Python, small inputs) --------
def q4k_dot_loop(q: np.ndarray, x: np.ndarray) -> np.float32:
    """sum over sb, chunk, l of lo_f*x[..l] then hi_f*x[..32+l], float32."""
    w = q4k_dequant(q)
    xs = np.asarray(x, dtype=F32)
    acc = F32(0.0)
    n_sb = w.size // 256
    for sb in range(n_sb):
        for c in range(4):
            base = sb * 256 + 64 * c
            for l in range(32):
                acc = F32(acc + F32(w[base + l] * xs[base + l]))
                acc = F32(acc + F32(w[base + 32 + l] * xs[base + 32 + l]))
    return acc


def q4_0_dot_loop(q: np.ndarray, x: np.ndarray) -> np.float32:
    """sum over block, k of w[k]*x[k] then w[k+16]*x[k+16], float32."""
    w = q4_0_dequant(q)
    xs = np.asarray(x, dtype=F32)
    acc = F32(0.0)
    for b in range(w.size // 32):
        for k in range(16):
            i = 32 * b + k
            acc = F32(acc + F32(w[i] * xs[i]))
            acc = F32(acc + F32(w[i + 16] * xs[i + 16]))
    return acc


# ---- the reference's LCG generator, in Python integers ----------------------
MASK64 = (1 << 64) - 1


def u64_to_f32(v: int) -> np.float32:
    """Round-to-nearest-even u64 -> binary32 in integer arithmetic (Rust `as f32`)."""
    if v == 0:
        return F32(0.0)
    shift = max(0, v.bit_length() - 24)
    q, rem = v >> shift, v & ((1 << shift) - 1)
    if shift:
        half = 1 << (shift - 1)
        if rem > half or (rem == half and (q & 1)):
            q += 1
    return F32(float(q) * 2.0 ** shift)  # exact: q < 2^25 and a power-of-two scale


def generate_q4km_test_data(n_superblocks: int, seed: int):
    """generate_q4km_test_data (tests/common_helpers.rs:476-519)."""
    state = (seed ^ 0x9E3779B97F4A7C15) & MASK64
    umax = u64_to_f32(MASK64)  # u64::MAX as f32 rounds to 2^64

    def nxt() -> int:
        nonlocal state
        state = (state * 6364136223846793005 + 1442695040888963407) & MASK64
        return state

    def u01() -> np.float32:
        return F32(u64_to_f32(nxt()) / umax)

    q = bytearray()
    for _ in range(n_superblocks):
        d = F32(F32(0.1) + F32(u01() * F32(1.9)))
        q += np.array([d], dtype=F32).astype("<f2").tobytes()
        dmin = F32(u01() * F32(0.5))
        q += np.array([dmin], dtype=F32).astype("<f2").tobytes()
        for _ in range(140):
            q.append(nxt() & 0xFF)
    x = np.empty(n_superblocks * 256, dtype=F32)
    for i in range(x.size):
        x[i] = F32(F32(u01() * F32(2.0)) - F32(1.0))
    return np.frombuffer(bytes(q), dtype=np.uint8), x
