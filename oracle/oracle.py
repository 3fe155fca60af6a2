"""ctypes wrapper of the C oracle (oracle/liboracle.so) with numpy arrays.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker; never by the product library.
Each function restates the reference CPU path; see q4_oracle.c for the
file:line of each and the tests that pin it.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# AXH_ORACLE_LIBRARY selects another build (e.g. the sanitizer build).
LIB_PATH = (Path(os.environ["AXH_ORACLE_LIBRARY"]) if os.environ.get("AXH_ORACLE_LIBRARY")
            else HERE / "liboracle.so")

Q4_0_BLOCK_BYTES, Q4_0_BLOCK_ELEMS = 18, 32
Q4K_SB_BYTES, Q4K_SB_ELEMS = 144, 256
# ggml type ids (GGUF) and superblock bytes of the k-quants next to Q4_K.
GGML_Q5_K, GGML_Q6_K = 13, 14
KQ_SB_BYTES = {GGML_Q5_K: 176, GGML_Q6_K: 210}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(str(LIB_PATH))
        c = ctypes
        vp, sz, u64, u32, i32 = c.c_void_p, c.c_size_t, c.c_uint64, c.c_uint32, c.c_int
        sigs = {
            "axo_f16_bits_to_f32": (c.c_float, [c.c_uint16]),
            "axo_f32_to_f16_bits": (c.c_uint16, [c.c_float]),
            "axo_unpack_scale_min_k4": (None, [vp, i32, vp, vp]),
            "axo_q4_0_dot": (c.c_float, [vp, vp, sz]),
            "axo_q4k_dot": (c.c_float, [vp, vp, sz]),
            "axo_q4_0_matvec": (None, [vp, vp, vp, sz, sz]),
            "axo_q4k_matvec": (None, [vp, vp, vp, sz, sz]),
            "axo_q4k_matvec_mt": (None, [vp, vp, vp, sz, sz, i32]),
            "axo_q4_0_matvec_mt": (None, [vp, vp, vp, sz, sz, i32]),
            "axo_q4_0_dequant": (None, [vp, vp, sz]),
            "axo_q4k_dequant": (None, [vp, vp, sz]),
            "axo_q4k_matvec_f64": (None, [vp, vp, vp, vp, sz, sz]),
            "axo_q4_0_matvec_f64": (None, [vp, vp, vp, vp, sz, sz]),
            "axo_q4k_matmul_f16x": (None, [vp, vp, vp, sz, sz, sz, i32]),
            "axo_generate_q4km_test_data": (None, [u32, u64, vp, vp]),
            "axo_gen_q4k_weights": (None, [u64, vp, sz]),
            "axo_gen_q4_0_weights": (None, [u64, vp, sz]),
            "axo_gen_normal_f32": (None, [u64, vp, sz, c.c_double]),
            "axo_q5k_dequant": (None, [vp, vp, sz]),
            "axo_q6k_dequant": (None, [vp, vp, sz]),
            "axo_kq_dot": (c.c_float, [i32, vp, vp, sz]),
            "axo_kq_matvec": (None, [i32, vp, vp, vp, sz, sz, i32]),
            "axo_kq_matvec_f64": (None, [i32, vp, vp, vp, vp, sz, sz]),
            "axo_gen_q5k_weights": (None, [u64, vp, sz]),
            "axo_gen_q6k_weights": (None, [u64, vp, sz]),
        }
        for name, (res, args) in sigs.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def default_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


# ---- scalar pieces ---------------------------------------------------------
def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    f = lib().axo_f16_bits_to_f32
    flat, of = bits.ravel(), out.ravel()
    for i in range(flat.size):
        of[i] = f(int(flat[i]))
    return out


def f32_to_f16_bits(x: float) -> int:
    return int(lib().axo_f32_to_f16_bits(float(np.float32(x))))


def unpack_scale_min_k4(scales: bytes, j: int) -> tuple[int, int]:
    s = np.frombuffer(bytes(scales), dtype=np.uint8).copy()
    assert s.size == 12
    sc, m = ctypes.c_uint8(), ctypes.c_uint8()
    lib().axo_unpack_scale_min_k4(_p(s), j, ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


# ---- single-output dots (the reference kernels' y[0]) -----------------------
def q4_0_dot(q: np.ndarray, x: np.ndarray, n_blocks: int) -> np.float32:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    if q.size != n_blocks * Q4_0_BLOCK_BYTES or x.size != n_blocks * Q4_0_BLOCK_ELEMS:
        raise ValueError("q4_0_dequant_matvec_cpu: length mismatch")  # common.rs:218-222
    return np.float32(lib().axo_q4_0_dot(_p(q), _p(x), n_blocks))


def q4k_dot(q: np.ndarray, x: np.ndarray, n_superblocks: int) -> np.float32:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    if q.size != n_superblocks * Q4K_SB_BYTES or x.size < n_superblocks * Q4K_SB_ELEMS:
        raise ValueError("q4km_dequant_matvec_cpu: length mismatch")  # common_helpers.rs:412-421
    return np.float32(lib().axo_q4k_dot(_p(q), _p(x), n_superblocks))


# ---- matrices --------------------------------------------------------------
def q4k_matvec(q, x, n_rows: int, sb_per_row: int, threads: int = 0) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert q.size == n_rows * sb_per_row * Q4K_SB_BYTES and x.size >= sb_per_row * Q4K_SB_ELEMS
    y = np.empty(n_rows, dtype=np.float32)
    lib().axo_q4k_matvec_mt(_p(q), _p(x), _p(y), n_rows, sb_per_row, threads or default_threads())
    return y


def q4k_matvec_single(q, x, n_rows: int, sb_per_row: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(n_rows, dtype=np.float32)
    lib().axo_q4k_matvec(_p(q), _p(x), _p(y), n_rows, sb_per_row)
    return y


def q4_0_matvec(q, x, n_rows: int, blocks_per_row: int, threads: int = 0) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert q.size == n_rows * blocks_per_row * Q4_0_BLOCK_BYTES
    assert x.size >= blocks_per_row * Q4_0_BLOCK_ELEMS
    y = np.empty(n_rows, dtype=np.float32)
    lib().axo_q4_0_matvec_mt(_p(q), _p(x), _p(y), n_rows, blocks_per_row,
                             threads or default_threads())
    return y


def q4k_dequant(q, n_superblocks: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    w = np.empty(n_superblocks * Q4K_SB_ELEMS, dtype=np.float32)
    lib().axo_q4k_dequant(_p(q), _p(w), n_superblocks)
    return w


def q4_0_dequant(q, n_blocks: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    w = np.empty(n_blocks * Q4_0_BLOCK_ELEMS, dtype=np.float32)
    lib().axo_q4_0_dequant(_p(q), _p(w), n_blocks)
    return w


def q4k_matvec_f64(q, x, n_rows: int, sb_per_row: int):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(n_rows, dtype=np.float64)
    a = np.empty(n_rows, dtype=np.float64)
    lib().axo_q4k_matvec_f64(_p(q), _p(x), _p(y), _p(a), n_rows, sb_per_row)
    return y, a


def q4_0_matvec_f64(q, x, n_rows: int, blocks_per_row: int):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(n_rows, dtype=np.float64)
    a = np.empty(n_rows, dtype=np.float64)
    lib().axo_q4_0_matvec_f64(_p(q), _p(x), _p(y), _p(a), n_rows, blocks_per_row)
    return y, a


def q4k_matmul_f16x(q, x_f16_bits, n_rows: int, sb_per_row: int, batch: int,
                    threads: int = 0) -> np.ndarray:
    """Y[r, b] = q4k dot of row r with f32(X[:, b]); X given as B vectors of f16 bits."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    xb = np.ascontiguousarray(x_f16_bits, dtype=np.uint16)
    assert xb.size == batch * sb_per_row * Q4K_SB_ELEMS
    y = np.empty((n_rows, batch), dtype=np.float32)
    lib().axo_q4k_matmul_f16x(_p(q), _p(xb), _p(y), n_rows, sb_per_row, batch,
                              threads or default_threads())
    return y


# ---- Q5_K / Q6_K (ggml k-quants; restated in kq_oracle.c) ---------------------
def kq_dequant(kind: int, q, n_superblocks: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    assert q.size >= n_superblocks * KQ_SB_BYTES[kind]
    w = np.empty(n_superblocks * 256, dtype=np.float32)
    fn = lib().axo_q5k_dequant if kind == GGML_Q5_K else lib().axo_q6k_dequant
    fn(_p(q), _p(w), n_superblocks)
    return w


def kq_matvec(kind: int, q, x, n_rows: int, sb_per_row: int, threads: int = 0) -> np.ndarray:
    """Row r: sequential f32 dot of row r's superblocks with x (element order)."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert q.size >= n_rows * sb_per_row * KQ_SB_BYTES[kind] and x.size >= sb_per_row * 256
    y = np.empty(n_rows, dtype=np.float32)
    lib().axo_kq_matvec(kind, _p(q), _p(x), _p(y), n_rows, sb_per_row,
                        threads or default_threads())
    return y


def kq_matvec_f64(kind: int, q, x, n_rows: int, sb_per_row: int):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(n_rows, dtype=np.float64)
    a = np.empty(n_rows, dtype=np.float64)
    lib().axo_kq_matvec_f64(kind, _p(q), _p(x), _p(y), _p(a), n_rows, sb_per_row)
    return y, a


def gen_kq_weights(kind: int, seed: int, n_superblocks: int) -> np.ndarray:
    q = np.empty(n_superblocks * KQ_SB_BYTES[kind], dtype=np.uint8)
    fn = lib().axo_gen_q5k_weights if kind == GGML_Q5_K else lib().axo_gen_q6k_weights
    fn(seed, _p(q), n_superblocks)
    return q


# ---- SwiGLU gate/up (no reference counterpart) -------------------------------
def silu(g) -> np.ndarray:
    """silu(g) = g * sigmoid(g) = g / (1 + exp(-g)) in f64 (the SwiGLU gate of
    a decode step's feed-forward block; the reference stops at one matvec,
    ROADMAP.md:54-72).  Pinned against scipy.special.expit, the identity
    silu(g) - silu(-g) = g and closed-form values."""
    g = np.asarray(g, dtype=np.float64)
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-g))


def q4k_gate_up_f64(q_gate, q_up, x, n_rows: int, sb_per_row: int):
    """h = silu(Wg x) * (Wu x) from the f64 row dots; also returns the dots
    (g, |g| terms, u, |u| terms) for the tolerance criterion."""
    g, ag = q4k_matvec_f64(q_gate, x, n_rows, sb_per_row)
    u, au = q4k_matvec_f64(q_up, x, n_rows, sb_per_row)
    return silu(g) * u, g, ag, u, au


def q4_0_gate_up_f64(q_gate, q_up, x, n_rows: int, blocks_per_row: int):
    """The same for two Q4_0 matrices (q4_0_matvec_f64 row dots)."""
    g, ag = q4_0_matvec_f64(q_gate, x, n_rows, blocks_per_row)
    u, au = q4_0_matvec_f64(q_up, x, n_rows, blocks_per_row)
    return silu(g) * u, g, ag, u, au


def kq_gate_up_f64(kind: int, q_gate, q_up, x, n_rows: int, sb_per_row: int):
    """The same for two Q5_K / Q6_K matrices (kq_matvec_f64 row dots)."""
    g, ag = kq_matvec_f64(kind, q_gate, x, n_rows, sb_per_row)
    u, au = kq_matvec_f64(kind, q_up, x, n_rows, sb_per_row)
    return silu(g) * u, g, ag, u, au


def gate_up_tolerance_report(h_gpu, g, ag, u, au, n_cols: int, rel_tol: float = 1e-3,
                             cancel_frac: float = 0.1) -> dict:
    """Acceptance for h = silu(g) * u when each dot product may carry the
    matvec criterion's error e = rel_tol * (|c| if |c| >= cancel_frac * s
    else s), s = sum|w x| / sqrt(n): per row
      |h - h_ref| <= L * e_g * (|u| + e_u) + |silu(g)| * e_u + 8 ulp(h_ref)
    with L = 1.1 >= max |silu'|, and ||h - h_ref|| <= rel_tol * ||h_ref||."""
    h = np.asarray(h_gpu, dtype=np.float64)
    g, u = np.asarray(g, np.float64), np.asarray(u, np.float64)

    def allowed(c, a):
        s = np.asarray(a, np.float64) / np.sqrt(max(1, n_cols))
        return rel_tol * np.where(np.abs(c) < cancel_frac * s, s, np.abs(c))

    ref = silu(g) * u
    e_g, e_u = allowed(g, ag), allowed(u, au)
    bound = 1.1 * e_g * (np.abs(u) + e_u) + np.abs(silu(g)) * e_u + 8 * 2.0 ** -24 * np.abs(ref)
    diff = np.abs(h - ref)
    row_ok = (diff <= bound) & np.isfinite(h)
    norm_err = float(np.linalg.norm(h - ref) / max(np.linalg.norm(ref), 1e-30))
    return {
        "rows": int(h.size),
        "rows_failed": int((~row_ok).sum()),
        "worst_over_bound": float((diff / np.maximum(bound, 1e-300)).max()) if h.size else 0.0,
        "norm_rel_err": norm_err,
        "ok": bool(row_ok.all() and norm_err <= rel_tol),
    }


# ---- generators ------------------------------------------------------------
def generate_q4km_test_data(n_superblocks: int, seed: int):
    """generate_q4km_test_data (tests/common_helpers.rs:476-519)."""
    q = np.empty(n_superblocks * Q4K_SB_BYTES, dtype=np.uint8)
    x = np.empty(n_superblocks * Q4K_SB_ELEMS, dtype=np.float32)
    lib().axo_generate_q4km_test_data(n_superblocks, seed & 0xFFFFFFFFFFFFFFFF, _p(q), _p(x))
    return q, x


def gen_q4k_weights(seed: int, n_superblocks: int) -> np.ndarray:
    q = np.empty(n_superblocks * Q4K_SB_BYTES, dtype=np.uint8)
    lib().axo_gen_q4k_weights(seed, _p(q), n_superblocks)
    return q


def gen_q4_0_weights(seed: int, n_blocks: int) -> np.ndarray:
    q = np.empty(n_blocks * Q4_0_BLOCK_BYTES, dtype=np.uint8)
    lib().axo_gen_q4_0_weights(seed, _p(q), n_blocks)
    return q


def gen_normal_f32(seed: int, n: int, sigma: float = 1.0) -> np.ndarray:
    x = np.empty(n, dtype=np.float32)
    lib().axo_gen_normal_f32(seed, _p(x), n, sigma)
    return x


# ---- acceptance ------------------------------------------------------------
def reference_rel_err(gpu: float, cpu: float) -> float:
    """The reference's check (compile_q4km_dequant_matvec.rs:946-956, DESIGN.md:508-513):
    |g-c|/|c| if |c| > 1e-10 else |g-c|, computed in f32."""
    g, c = np.float32(gpu), np.float32(cpu)
    d = np.float32(abs(g - c))
    return float(d / np.float32(abs(c))) if abs(c) > np.float32(1e-10) else float(d)


def matvec_tolerance_report(y_gpu, y_cpu, y_f64, absdot, n_cols: int, rel_tol: float = 1e-3,
                            cancel_frac: float = 0.1) -> dict:
    """Row-wise acceptance criterion for multi-row matvec.

    With s = sum|w x| / sqrt(n) (the size of a sum of n random-sign terms),
    a row is well conditioned when |c| >= cancel_frac * s and must satisfy
    |g - c| <= rel_tol * |c|; a row that cancels below that level must satisfy
    the condition-scaled bound |g - c| <= rel_tol * s.  In addition the
    norm-wise error ||g - c||_2 / ||c||_2 must be <= rel_tol.
    """
    g = np.asarray(y_gpu, dtype=np.float64)
    c = np.asarray(y_cpu, dtype=np.float64)
    a = np.asarray(absdot, dtype=np.float64)
    diff = np.abs(g - c)
    scale = a / np.sqrt(max(1, n_cols))
    cancel = np.abs(c) < cancel_frac * scale
    rel_ok = diff <= rel_tol * np.abs(c)
    cond_ok = diff <= rel_tol * scale
    row_ok = np.where(cancel, cond_ok, rel_ok)
    norm_err = float(np.linalg.norm(g - c) / max(np.linalg.norm(c), 1e-30))
    return {
        "rows": int(g.size),
        "rows_failed": int((~row_ok).sum()),
        "cancelling_rows": int(cancel.sum()),
        "max_rel_err_wellcond": float((diff / np.maximum(np.abs(c), 1e-30))[~cancel].max())
        if (~cancel).any() else 0.0,
        "norm_rel_err": norm_err,
        "gpu_err_vs_f64_norm": float(np.linalg.norm(g - y_f64) / max(np.linalg.norm(y_f64), 1e-30)),
        "cpu_err_vs_f64_norm": float(np.linalg.norm(c - y_f64) / max(np.linalg.norm(y_f64), 1e-30)),
        "ok": bool(row_ok.all() and norm_err <= rel_tol),
    }
