"""Pins of the CPU oracle (CPU only).

The oracle (oracle/q4_oracle.c) is the checker for the HIP path, so each of
its functions is pinned here by something other than its own formula:
  - the reference's own known-answer tests, transcribed with their expected
    values (AT-1312 get_scale_min_k4 pairs, the Q4_0 layout KATs, AT-1323);
  - closed forms (exactly representable sums, one-rounding dequantisation,
    IEEE binary16 widening over all 65,536 patterns);
  - an independent restatement (oracle/q4_numpy.py, written from the
    reference's format specification) agreeing bit for bit;
  - planted mistakes (the q[j-4] bit-spread, the interleaved Q4_0 layout,
    swapped nibble halves) that the pins must reject.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as O
from oracle import q4_numpy as N


# ---- a3: binary16 decode ------------------------------------------------------
def test_f16_decode_exhaustive_matches_ieee():
    bits = np.arange(65536, dtype=np.uint16)
    ours = O.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(ours.view(np.uint32)[~nan], ref.view(np.uint32)[~nan])
    # NaNs: same class and sign, quiet bit set (half::f16::to_f32 behaviour)
    assert np.isnan(ours[nan]).all()
    qn = ours.view(np.uint32)[nan]
    assert ((qn & 0x00400000) != 0).all()
    assert np.array_equal(qn >> 31, (bits[nan] >> 15).astype(np.uint32))


def test_f16_decode_subnormals_and_one():
    # 0x3C00 -> 1.0 is the value the reference's own tests rely on
    # (common_helpers.rs:255-263); 0x0001 is the smallest f16 subnormal.
    assert O.f16_bits_to_f32(np.array([0x3C00], np.uint16))[0] == np.float32(1.0)
    assert O.f16_bits_to_f32(np.array([0x0001], np.uint16))[0] == np.float32(2.0 ** -24)
    assert O.f16_bits_to_f32(np.array([0x03FF], np.uint16))[0] == np.float32(1023 * 2.0 ** -24)
    assert O.f16_bits_to_f32(np.array([0x8000], np.uint16)).view(np.uint32)[0] == 0x80000000


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32),
        rng.uniform(0.0, 0.05, 20000).astype(np.float32),
        (rng.uniform(0, 1, 5000) * 2.0 ** -20).astype(np.float32),   # f16 subnormal range
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 1e9, -1e9, 2.0 ** -25,
                  2.0 ** -25 * 1.0000001, 2.0 ** -24 * 1.5, 2.0 ** -24 * 2.5,
                  np.inf, -np.inf], dtype=np.float32),
    ])
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    ours = np.array([O.f32_to_f16_bits(v) for v in vals], dtype=np.uint16)
    assert np.array_equal(ours, ref)


# ---- a4: get_scale_min_k4 --------------------------------------------------------
def _sc(scales, j):
    return O.unpack_scale_min_k4(bytes(scales), j)


def test_at_1312_get_scale_min_k4_hand_verified_pairs():
    """The assertions of AT-1312 (compile_q4km_dequant_matvec.rs:485-584)."""
    for j in range(8):
        assert _sc([0] * 12, j) == (0, 0)
    s = [0] * 12; s[0] = 0xFF; s[4] = 0xC0
    assert _sc(s, 0) == (63, 0)
    s = [0] * 12; s[3] = 0x3F; s[7] = 0x3F
    assert _sc(s, 3) == (63, 63)
    s = [0] * 12; s[8] = 0xAB; s[0] = 0xC0; s[4] = 0xD0
    assert _sc(s, 4) == (59, 58)
    s = [0] * 12; s[9] = 0xCD; s[1] = 0x80; s[5] = 0x40
    assert _sc(s, 5) == ((0xCD & 0x0F) | (2 << 4), (0xCD >> 4) | (1 << 4))
    s = [0] * 12; s[10] = 0x12; s[2] = 0x55; s[6] = 0xAA
    assert _sc(s, 6) == ((0x12 & 0x0F) | (1 << 4), (0x12 >> 4) | (2 << 4))
    s = [0] * 12; s[11] = 0xFF; s[3] = 0xFF; s[7] = 0xFF
    assert _sc(s, 7) == (63, 63)
    # discriminator: m-high comes from scales[j] (=0x80 -> 33), not scales[j-4] (-> 17)
    s = [0] * 12; s[8] = 0x10; s[4] = 0x80; s[0] = 0x40
    assert _sc(s, 4)[1] == 33


def _planted_j_minus_4(s, j):
    """The mistake AT-1312 guards against: m-high from scales[j-4]."""
    if j < 4:
        return s[j] & 63, s[j + 4] & 63
    return (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4), (s[j + 4] >> 4) | ((s[j - 4] >> 6) << 4)


def test_get_scale_min_k4_all_byte_values_vs_field_layout():
    """Every value of every byte that feeds each j, against the field layout."""
    rng = np.random.default_rng(7)
    planted_differs = 0
    for j in range(8):
        for pos in range(12):
            for v in range(256):
                s = rng.integers(0, 256, 12).astype(np.uint8)
                s[pos] = v
                assert _sc(s, j) == N.scale_min_k4(s, j), (j, pos, v)
                planted_differs += _planted_j_minus_4([int(t) for t in s], j) != N.scale_min_k4(s, j)
    assert planted_differs > 0  # the pin rejects the q[j-4] mistake


# ---- a1/a5: dequantisation ---------------------------------------------------------
def test_q4k_dequant_matches_independent_restatement():
    q = O.gen_q4k_weights(5, 4000)
    assert np.array_equal(O.q4k_dequant(q, 4000).view(np.uint32),
                          N.q4k_dequant(q).view(np.uint32))
    q2, _ = O.generate_q4km_test_data(512, 0xCAFEBABE)
    assert np.array_equal(O.q4k_dequant(q2, 512).view(np.uint32),
                          N.q4k_dequant(q2).view(np.uint32))


def test_q4k_dequant_is_one_rounding_of_exact_value():
    """w = RN_f32(d*sc*q - dmin*m) computed exactly with fractions."""
    q = O.gen_q4k_weights(9, 24)
    w = O.q4k_dequant(q, 24)
    sbs = q.reshape(-1, 144)
    for i in range(24):
        d = Fraction(float(sbs[i, 0:2].view("<f2")[0]))
        dmin = Fraction(float(sbs[i, 2:4].view("<f2")[0]))
        for c in range(4):
            sc0, m0 = N.scale_min_k4(sbs[i, 4:16], 2 * c)
            sc1, m1 = N.scale_min_k4(sbs[i, 4:16], 2 * c + 1)
            for l in range(32):
                b = int(sbs[i, 16 + 32 * c + l])
                lo = d * sc0 * (b & 15) - dmin * m0
                hi = d * sc1 * (b >> 4) - dmin * m1
                # both values span < 53 bits, so float() is exact and the f32
                # cast is the single rounding the reference performs
                assert Fraction(float(lo)) == lo and Fraction(float(hi)) == hi
                assert w[i * 256 + 64 * c + l] == np.float32(float(lo))
                assert w[i * 256 + 64 * c + 32 + l] == np.float32(float(hi))


def test_q4_0_dequant_closed_form_and_layout():
    q = O.gen_q4_0_weights(3, 3000)
    w = O.q4_0_dequant(q, 3000)
    assert np.array_equal(w.view(np.uint32), N.q4_0_dequant(q).view(np.uint32))
    blk = q.reshape(-1, 18)
    d = blk[:, 0:2].copy().view("<f2").astype(np.float64).reshape(-1)
    lo = (blk[:, 2:] & 15).astype(np.float64) - 8
    hi = (blk[:, 2:] >> 4).astype(np.float64) - 8
    exact = np.concatenate([lo * d[:, None], hi * d[:, None]], axis=1).reshape(-1)
    assert np.array_equal(w.astype(np.float64), exact)  # no rounding at all


# ---- a2: Q4_0 dot -------------------------------------------------------------------
def test_q4_0_layout_kat_minus_128():
    """common_helpers.rs:270-296: scale 1.0, bytes 0x80, x = 1 -> -128.0."""
    q = np.array([0x00, 0x3C] + [0x80] * 16, dtype=np.uint8)
    x = np.ones(32, dtype=np.float32)
    assert O.q4_0_dot(q, x, 1) == np.float32(-128.0)


def test_q4_0_layout_discriminating_kat_minus_96():
    """common_helpers.rs:315-333: bytes 0x12, x[0..16]=1 -> -96 (interleaved layout: -104)."""
    q = np.array([0x00, 0x3C] + [0x12] * 16, dtype=np.uint8)
    x = np.zeros(32, dtype=np.float32)
    x[:16] = 1.0
    assert O.q4_0_dot(q, x, 1) == np.float32(-96.0)
    w = O.q4_0_dequant(q, 1)
    interleaved = sum(float(w[k]) * float(x[2 * k]) for k in range(16))  # planted mistake
    assert interleaved != -96.0


def test_q4_0_dot_matches_reference_order_loop():
    for nb, seed in ((1, 1), (7, 2), (64, 3)):
        q = O.gen_q4_0_weights(seed, nb)
        x = O.gen_normal_f32(seed + 100, nb * 32)
        assert O.q4_0_dot(q, x, nb).view(np.uint32) == N.q4_0_dot_loop(q, x).view(np.uint32)


def test_q4_0_dot_rejects_length_mismatch():
    with pytest.raises(ValueError):
        O.q4_0_dot(np.zeros(18, np.uint8), np.zeros(31, np.float32), 1)


# ---- a6: Q4_K dot -------------------------------------------------------------------
def test_at_1323_q4km_cpu_reference_finite_reproducible_and_zero():
    q, x = O.generate_q4km_test_data(16, 0xDEADBEEF)
    r1, r2 = O.q4k_dot(q, x, 16), O.q4k_dot(q, x, 16)
    assert np.isfinite(r1) and r1.view(np.uint32) == r2.view(np.uint32)
    q0, x0 = O.generate_q4km_test_data(0, 0xDEADBEEF)
    assert O.q4k_dot(q0, x0, 0).view(np.uint32) == 0  # +0.0 bits


def test_q4k_dot_matches_reference_order_loop():
    for n, seed in ((1, 0xDEADBEEF), (3, 0xCAFEBABE), (16, 0xDEADBEEF)):
        q, x = O.generate_q4km_test_data(n, seed)
        assert O.q4k_dot(q, x, n).view(np.uint32) == N.q4k_dot_loop(q, x).view(np.uint32)


def test_q4k_dot_closed_form_uniform_superblock():
    """d = 1, all sc = 1, m = 0, every nibble = v, x = 1 -> 256 * v exactly."""
    for v in (0, 1, 7, 15):
        sb = np.zeros(144, dtype=np.uint8)
        sb[0:2] = np.array([1.0], np.float16).view(np.uint8)
        sb[4:8] = 1                     # sc[0..3] = 1, m[0..3] = 0
        sb[8:12] = 0
        sb[12:16] = 0x01                # sc[4..7] low nibble 1, m[4..7] = 0
        sb[16:] = v | (v << 4)
        x = np.ones(256, dtype=np.float32)
        assert O.q4k_dot(sb, x, 1) == np.float32(256 * v)


def test_q4k_dot_closed_form_mins_only():
    """nibbles 0, dmin = 0.5, m[j] = j + 1, x = 1 -> -(0.5 * 32 * sum(1..8)) = -576."""
    sb = np.zeros(144, dtype=np.uint8)
    sb[0:2] = np.array([1.0], np.float16).view(np.uint8)
    sb[2:4] = np.array([0.5], np.float16).view(np.uint8)
    for j in range(4):
        sb[8 + j] = j + 1                       # m[j] = j+1 (low 6 bits of scales[4+j])
        sb[12 + j] = (j + 5) << 4               # m[4+j] low nibble = j+5
    assert [N.scale_min_k4(sb[4:16], j)[1] for j in range(8)] == list(range(1, 9))
    x = np.ones(256, dtype=np.float32)
    assert O.q4k_dot(sb, x, 1) == np.float32(-576.0)


def test_q4k_dot_rejects_length_mismatch():
    with pytest.raises(ValueError):
        O.q4k_dot(np.zeros(143, np.uint8), np.zeros(256, np.float32), 1)


def test_q4k_swapped_nibble_halves_is_detected():
    """Planted mistake: hi nibble paired with x[..l] instead of x[..32+l]."""
    q, x = O.generate_q4km_test_data(2, 0xDEADBEEF)
    w = N.q4k_dequant(q).reshape(-1, 4, 2, 32)
    wrong = w[:, :, ::-1, :].reshape(-1)
    good = float(O.q4k_dot(q, x, 2))
    bad = float(np.dot(wrong.astype(np.float64), x.astype(np.float64)))
    assert abs(good - bad) > 1e-3 * abs(good)


# ---- a8: generators ------------------------------------------------------------------
@pytest.mark.parametrize("n,seed", [(16, 0xDEADBEEF), (128, 0xDEADBEEF), (128, 0xCAFEBABE), (512, 0xCAFEBABE)])
def test_generate_q4km_test_data_matches_integer_lcg(n, seed):
    q1, x1 = O.generate_q4km_test_data(n, seed)
    q2, x2 = N.generate_q4km_test_data(n, seed)
    assert np.array_equal(q1, q2)
    assert np.array_equal(x1.view(np.uint32), x2.view(np.uint32))
    assert (x1 >= -1.0).all() and (x1 <= 1.0).all()


def test_generator_determinism_and_seed_sensitivity():
    a = O.gen_q4k_weights(1, 64)
    assert np.array_equal(a, O.gen_q4k_weights(1, 64))
    assert not np.array_equal(a, O.gen_q4k_weights(2, 64))
    x = O.gen_normal_f32(3, 100000, 0.5)
    assert abs(float(x.std()) - 0.5) < 0.01 and abs(float(x.mean())) < 0.01


def test_benchmark_weight_distributions():
    q = O.gen_q4k_weights(11, 20000).reshape(-1, 144)
    d = q[:, 0:2].copy().view("<f2").astype(np.float32).reshape(-1)
    dmin = q[:, 2:4].copy().view("<f2").astype(np.float32).reshape(-1)
    assert d.min() >= np.float32(0.001) * 0.999 and d.max() <= 0.05 * 1.001
    assert dmin.min() >= 0.0 and dmin.max() <= 0.02 * 1.001
    # f16 subnormals occur in dmin (below 2^-14)
    assert (dmin < 2.0 ** -14).any() and (dmin > 0).any()


# ---- multi-row extension and baselines --------------------------------------------
def test_multirow_is_rowwise_reference_dot_and_threads_are_bit_identical():
    rows, sb = 37, 9
    q = O.gen_q4k_weights(21, rows * sb)
    x = O.gen_normal_f32(22, sb * 256)
    y1 = O.q4k_matvec_single(q, x, rows, sb)
    for t in (2, 8):
        assert np.array_equal(y1.view(np.uint32), O.q4k_matvec(q, x, rows, sb, t).view(np.uint32))
    rb = sb * 144
    for r in (0, 17, 36):
        assert y1[r].view(np.uint32) == O.q4k_dot(q[r * rb:(r + 1) * rb], x, sb).view(np.uint32)
    q0 = O.gen_q4_0_weights(23, rows * sb)
    x0 = O.gen_normal_f32(24, sb * 32)
    z = O.q4_0_matvec(q0, x0, rows, sb, 4)
    assert z[5].view(np.uint32) == O.q4_0_dot(q0[5 * sb * 18:6 * sb * 18], x0, sb).view(np.uint32)


def test_f64_reference_bounds_the_f32_oracle():
    rows, sb = 64, 56
    q = O.gen_q4k_weights(31, rows * sb)
    x = O.gen_normal_f32(32, sb * 256, 0.5)
    y = O.q4k_matvec(q, x, rows, sb)
    yf, absdot = O.q4k_matvec_f64(q, x, rows, sb)
    # sequential f32 summation error <= n * eps * sum|w x| (loose a-priori bound)
    assert (np.abs(y - yf) <= sb * 256 * 2.0 ** -24 * absdot).all()
    rep = O.matvec_tolerance_report(y, y, yf, absdot, sb * 256)
    assert rep["ok"] and rep["rows_failed"] == 0


def test_tolerance_report_rejects_planted_error():
    rows, sb = 64, 16
    q = O.gen_q4k_weights(41, rows * sb)
    x = O.gen_normal_f32(42, sb * 256)
    y = O.q4k_matvec(q, x, rows, sb)
    yf, absdot = O.q4k_matvec_f64(q, x, rows, sb)
    bad = y.copy()
    bad[3] *= np.float32(1.01)
    assert not O.matvec_tolerance_report(bad, y, yf, absdot, sb * 256)["ok"]


def test_batched_oracle_is_per_column_dot():
    rows, sb, batch = 5, 3, 4
    q = O.gen_q4k_weights(51, rows * sb)
    xh = O.gen_normal_f32(52, sb * 256 * batch).astype(np.float16)
    Y = O.q4k_matmul_f16x(q, xh.view(np.uint16), rows, sb, batch)
    xf = xh.astype(np.float32).reshape(batch, sb * 256)
    for b in range(batch):
        assert np.array_equal(Y[:, b].view(np.uint32),
                              O.q4k_matvec_single(q, xf[b], rows, sb).view(np.uint32))


# ---- f3: SwiGLU gate/up ----------------------------------------------------------
def test_silu_matches_scipy_expit_and_closed_forms():
    from scipy.special import expit

    g = np.concatenate([np.linspace(-60, 60, 2001), [0.0, 1e-30, -1e-30, 700.0, -700.0]])
    s = O.silu(g)
    assert np.allclose(s, g * expit(g), rtol=1e-14, atol=1e-300)
    assert O.silu(0.0) == 0.0
    assert O.silu(1.0) == pytest.approx(1.0 / (1.0 + np.exp(-1.0)), rel=1e-15)
    assert O.silu(800.0) == 800.0 and O.silu(-800.0) == 0.0  # exp overflow handled
    # silu(g) - silu(-g) = g * (sigmoid(g) + sigmoid(-g)) = g
    assert np.allclose(O.silu(g) - O.silu(-g), g, rtol=1e-13, atol=1e-12)


def test_gate_up_oracle_is_silu_of_rowwise_dots():
    rows, sb = 9, 2
    qg, qu = O.gen_q4k_weights(61, rows * sb), O.gen_q4k_weights(62, rows * sb)
    x = O.gen_normal_f32(63, sb * 256, 0.5)
    h, g, ag, u, au = O.q4k_gate_up_f64(qg, qu, x, rows, sb)
    wg = O.q4k_dequant(qg, rows * sb).reshape(rows, -1).astype(np.float64)
    wu = O.q4k_dequant(qu, rows * sb).reshape(rows, -1).astype(np.float64)
    xd = x.astype(np.float64)
    assert np.allclose(g, wg @ xd, rtol=1e-12) and np.allclose(u, wu @ xd, rtol=1e-12)
    assert np.allclose(ag, np.abs(wg) @ np.abs(xd), rtol=1e-12)
    assert np.allclose(h, (wg @ xd) / (1 + np.exp(-(wg @ xd))) * (wu @ xd), rtol=1e-12)


def test_gate_up_tolerance_rejects_swapped_and_perturbed_rows():
    rows, sb = 64, 16
    qg, qu = O.gen_q4k_weights(64, rows * sb), O.gen_q4k_weights(65, rows * sb)
    x = O.gen_normal_f32(66, sb * 256, 0.5)
    h, g, ag, u, au = O.q4k_gate_up_f64(qg, qu, x, rows, sb)
    assert O.gate_up_tolerance_report(h.astype(np.float32), g, ag, u, au, sb * 256)["ok"]
    swapped = O.silu(u) * g  # gate and up exchanged
    assert not O.gate_up_tolerance_report(swapped, g, ag, u, au, sb * 256)["ok"]
    shifted = np.roll(h, 1)  # row r paired with row r-1
    assert not O.gate_up_tolerance_report(shifted, g, ag, u, au, sb * 256)["ok"]
    bad = h.copy()
    bad[5] *= 1.01
    assert not O.gate_up_tolerance_report(bad, g, ag, u, au, sb * 256)["ok"]


# ---- f2: Q5_K / Q6_K (ggml k-quants; no reference counterpart) ------------------
@pytest.mark.parametrize("kind", [O.GGML_Q5_K, O.GGML_Q6_K])
def test_kq_dequant_matches_independent_restatement(kind):
    q = O.gen_kq_weights(kind, 77, 500)
    # include extreme header values: f16 subnormal and large d / dmin
    nb = O.KQ_SB_BYTES[kind]
    blocks = q.reshape(-1, nb)
    d_off = 208 if kind == O.GGML_Q6_K else 0
    blocks[0, d_off:d_off + 2] = np.array([0x0001], np.uint16).view(np.uint8)
    blocks[1, d_off:d_off + 2] = np.array([0x7BFF], np.uint16).view(np.uint8)
    w = O.kq_dequant(kind, q, 500)
    ref = (N.q5k_dequant if kind == O.GGML_Q5_K else N.q6k_dequant)(q)
    assert np.array_equal(w.view(np.uint32), ref.view(np.uint32))


def _q6k_block(d=1.0, scales=1, ql=0, qh=0):
    b = np.zeros(210, np.uint8)
    b[0:128] = ql
    b[128:192] = qh
    b[192:208] = np.asarray(scales, np.int8).view(np.uint8) if np.ndim(scales) else np.uint8(
        np.int8(scales).view(np.uint8))
    b[208:210] = np.array([d], np.float16).view(np.uint8)
    return b


def test_q6k_closed_forms_and_bit_sources():
    assert np.all(O.kq_dequant(O.GGML_Q6_K, _q6k_block(0.5), 1) == -16.0)  # q = 0 -> -32
    assert np.all(O.kq_dequant(O.GGML_Q6_K, _q6k_block(0.5, 1, 0xFF, 0xFF), 1) == 15.5)
    # scale s of sub-block t (16 weights) multiplies exactly weights 16t..16t+15
    sc = np.arange(-8, 8, dtype=np.int8) * 3
    w = O.kq_dequant(O.GGML_Q6_K, _q6k_block(0.25, sc, 0, 0), 1).reshape(2, 4, 2, 16)
    for n in range(2):
        for part in range(4):
            for half in range(2):
                s = int(sc[8 * n + half + 2 * part])
                assert np.all(w[n, part, half] == 0.25 * s * -32), (n, part, half)
    # one qh bit pair / one ql nibble at a time: exactly one weight moves
    for byte, shift, elem, q6 in [(128 + 5, 2, 32 + 5, 16), (128 + 32 + 7, 6, 128 + 96 + 7, 16),
                                  (128 + 0, 0, 0, 16), (40, 4, 96 + 8, 1), (64 + 3, 0, 128 + 3, 1)]:
        b = _q6k_block(1.0)
        b[byte] = np.uint8(1 << shift)
        w = O.kq_dequant(O.GGML_Q6_K, b, 1)
        moved = np.flatnonzero(w != -32.0)
        assert moved.tolist() == [elem] and w[elem] == q6 - 32, (byte, shift)


def test_q6k_planted_mistakes_are_rejected():
    """A restatement with the qh bit pairs of parts 1 and 2 swapped, or with
    ql halves exchanged, disagrees with the pinned oracle."""
    q = O.gen_kq_weights(O.GGML_Q6_K, 78, 8)
    w = O.kq_dequant(O.GGML_Q6_K, q, 8)
    b = q.reshape(-1, 210).astype(np.int64)
    e = np.arange(256)
    n, r = e // 128, e % 128
    part, l = r // 32, r % 32
    bad_shift = 2 * np.array([0, 2, 1, 3])[part]
    q6 = ((b[:, 64 * n + l + 32 * (part % 2)] >> (4 * (part // 2))) & 0xF) | \
        (((b[:, 128 + 32 * n + l] >> bad_shift) & 3) << 4)
    sc = b[:, 192 + 8 * n + l // 16 + 2 * part]
    sc = np.where(sc >= 128, sc - 256, sc)
    d = q.reshape(-1, 210)[:, 208:210].copy().view(np.float16).astype(np.float64)
    assert not np.array_equal((d * sc * (q6 - 32)).astype(np.float32).reshape(-1), w)


def test_q5k_with_zero_high_bits_is_q4k_and_high_bit_adds_sixteen():
    """Q5_K = Q4_K's header and nibbles plus one high bit per weight: with qh = 0
    it decodes exactly as the (pinned) Q4_K oracle, and with qh = 0xFF every
    weight is RN_f32(d*sc*(q+16) - dmin*m)."""
    q4 = O.gen_q4k_weights(79, 64).reshape(-1, 144)
    q5 = np.zeros((64, 176), np.uint8)
    q5[:, :16] = q4[:, :16]
    q5[:, 48:] = q4[:, 16:]
    w4 = O.q4k_dequant(q4.reshape(-1), 64)
    assert np.array_equal(O.kq_dequant(O.GGML_Q5_K, q5, 64).view(np.uint32), w4.view(np.uint32))
    q5[:, 16:48] = 0xFF
    w5 = O.kq_dequant(O.GGML_Q5_K, q5, 64).reshape(64, 256)
    for sb in range(3):
        d = float(q4[sb, 0:2].copy().view(np.float16)[0])
        dmin = float(q4[sb, 2:4].copy().view(np.float16)[0])
        for e in (0, 31, 32, 100, 255):
            j, hi, l = e // 64, (e % 64) // 32, e % 32
            sc, m = N.scale_min_k4(q4[sb, 4:16], 2 * j + hi)
            nib = (int(q4[sb, 16 + 32 * j + l]) >> (4 * hi)) & 0xF
            exact = Fraction(d) * sc * (nib + 16) - Fraction(dmin) * m
            assert w5[sb, e] == np.float32(float(exact)), (sb, e)


def test_q5k_high_bit_sources():
    for l, j, hi in [(0, 0, 0), (5, 0, 1), (31, 3, 1), (17, 2, 0)]:
        b = np.zeros(176, np.uint8)
        b[0:2] = np.array([1.0], np.float16).view(np.uint8)
        b[4:8] = 1  # sc = 1 for sub-blocks 0..3
        b[12:16] = 1  # low nibble of sc[4..7] = 1, m[4..7] = 0
        b[16 + l] = np.uint8(1 << (2 * j + hi))
        w = O.kq_dequant(O.GGML_Q5_K, b, 1)
        assert np.flatnonzero(w).tolist() == [64 * j + 32 * hi + l] and w.max() == 16.0


@pytest.mark.parametrize("kind", [O.GGML_Q5_K, O.GGML_Q6_K])
def test_kq_dot_is_sequential_f32_in_element_order(kind):
    q = O.gen_kq_weights(kind, 80, 2)
    x = O.gen_normal_f32(81, 512)
    w = O.kq_dequant(kind, q, 2)
    s = np.float32(0)
    for i in range(512):
        s = np.float32(s + np.float32(w[i] * x[i]))
    y = O.kq_matvec(kind, q, x, 1, 2, threads=1)
    assert y[0].view(np.uint32) == s.view(np.uint32)
    yf, ad = O.kq_matvec_f64(kind, q, x, 1, 2)
    exact = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(w, x))
    assert abs(yf[0] - float(exact)) <= 1e-12 * ad[0]


@pytest.mark.parametrize("kind", [O.GGML_Q5_K, O.GGML_Q6_K])
def test_kq_matvec_threads_bit_identical(kind):
    rows, sb = 37, 3
    q = O.gen_kq_weights(kind, 82, rows * sb)
    x = O.gen_normal_f32(83, sb * 256)
    a = O.kq_matvec(kind, q, x, rows, sb, threads=1)
    b = O.kq_matvec(kind, q, x, rows, sb, threads=5)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
