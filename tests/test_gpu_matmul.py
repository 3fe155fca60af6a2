"""Batched Q4_K_M matmul on MFMA (marked `gpu`): y_b = RN_f16(W) x_b for f16
activation vectors x_b.  The reference has no batched kernel; per column it
is the reference dot product (q4km_dequant_matvec_cpu,
crates/axc-driver/tests/common_helpers.rs:411-461) with x widened from f16.

Three checks, from tight to loose:
  * one-hot activations pick single weights: y = RN_f16(w32) bit for bit
    (pins the f16 weights against numpy's float16 rounding of the oracle's
    bit-exact f32 dequantisation);
  * against an f64 product of the same f16 weights: only f32 accumulation
    error remains (norm-wise <= 1e-5);
  * against the f32-weight oracle (the reference's arithmetic per column):
    per row |dy| <= 2^-11 * sum|w*x| (f16 weight rounding) + 1e-5 * sum|w*x|,
    and norm-wise <= 1e-3.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _dev(ctx, arr):
    b = ctx.alloc(max(arr.nbytes, 16))
    ctx.upload(b, arr)
    return b


def _run(ctx, q, xh, rows, sb, batch, variant=None):
    dq, dx, dy = _dev(ctx, q), _dev(ctx, xh), ctx.alloc(batch * rows * 4)
    ctx.q4k_matmul(dq, dx, dy, rows, sb, batch, variant)
    ctx.synchronize()
    y = np.frombuffer(ctx.download(dy, batch * rows * 4), dtype=np.float32).reshape(batch, rows)
    for b in (dq, dx, dy):
        b.close()
    return y.copy()


def _inputs(seed, rows, sb, batch):
    q = O.gen_q4k_weights(seed, rows * sb)
    xh = O.gen_normal_f32(seed + 1, sb * 256 * batch).astype(np.float16)
    return q, xh


def _w32(q, rows, sb):
    return O.q4k_dequant(q, rows * sb).reshape(rows, sb * 256)


def _check(y, q, xh, rows, sb, batch, what, oracle_f32=True):
    w32 = _w32(q, rows, sb)
    w16 = w32.astype(np.float16).astype(np.float64)
    xf = xh.astype(np.float64).reshape(batch, sb * 256)
    ref16 = xf @ w16.T                              # batch x rows, f64
    abs16 = np.abs(xf) @ np.abs(w16).T
    err16 = np.linalg.norm(y - ref16) / max(np.linalg.norm(ref16), 1e-30)
    worst = float(np.max(np.abs(y - ref16) / np.maximum(abs16, 1e-30)))
    _say(f"{what}: vs f16-weight f64 ref norm {err16:.2e}, worst/sum|wx| {worst:.2e}")
    assert err16 <= 1e-5, what
    assert np.all(np.abs(y - ref16) <= 1e-5 * abs16 + 1e-30), what
    # f32-weight reference (the reference's per-column arithmetic)
    if oracle_f32:
        ref = O.q4k_matmul_f16x(q, xh.view(np.uint16), rows, sb, batch).T  # batch x rows
    else:
        ref = xf @ w32.astype(np.float64).T
    abs32 = np.abs(xf) @ np.abs(w32.astype(np.float64)).T
    d = np.abs(y.astype(np.float64) - ref)
    bound = (2.0 ** -11 + 1e-5) * abs32
    norm = np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-30)
    _say(f"{what}: vs f32-weight ref norm {norm:.2e}, max d/bound {float(np.max(d / bound)):.3f}")
    assert np.all(d <= bound), what
    assert norm <= 1e-3, what


def test_one_hot_activations_give_rn_f16_weights_bit_exact(ctx):
    rows, sb = 64, 1
    batch = sb * 256
    q = O.gen_q4k_weights(71, rows * sb)
    xh = np.eye(batch, dtype=np.float16)  # x_b = e_b
    y = _run(ctx, q, xh, rows, sb, batch)
    w16 = _w32(q, rows, sb).astype(np.float16).astype(np.float32)
    assert np.array_equal(y.view(np.uint32), w16.T.copy().view(np.uint32))


def test_one_hot_lcg_fixture_weights(ctx):
    """The reference's own generator (seed 0xDEADBEEF, 16 superblocks) as one row."""
    q, _ = O.generate_q4km_test_data(16, 0xDEADBEEF)
    batch = 256
    for part in range(16):  # superblock `part` selected by one-hot vectors
        xh = np.zeros((batch, 16 * 256), dtype=np.float16)
        xh[np.arange(batch), part * 256 + np.arange(batch)] = 1.0
        y = _run(ctx, q, xh, 1, 16, batch)
        w16 = O.q4k_dequant(q, 16)[part * 256:(part + 1) * 256].astype(np.float16)
        assert np.array_equal(y[:, 0].astype(np.float16).view(np.uint16), w16.view(np.uint16))


@pytest.mark.parametrize("batch", [8, 32, 128, 256, 512])
def test_c5_down_projection_shapes(ctx, batch):
    """14336 x 4096 weights, B f16 activations ~ N(0, 1)."""
    rows, sb = 14336, 16
    _say(f"matmul C5 batch {batch}")
    q, xh = _inputs(500 + batch, rows, sb, batch)
    y = _run(ctx, q, xh, rows, sb, batch)
    _check(y, q, xh, rows, sb, batch, f"C5 B={batch}", oracle_f32=batch <= 32)


@pytest.mark.parametrize("rows,sb,batch", [(1, 1, 1), (100, 1, 7), (33, 3, 17), (257, 2, 130),
                                           (96, 5, 16), (31, 4, 33)])
def test_edge_shapes(ctx, rows, sb, batch):
    """Partial row and column tiles, single superblock, batch 1."""
    _say(f"matmul edge {rows}x{sb * 256} B={batch}")
    q, xh = _inputs(rows * 7 + sb * 3 + batch, rows, sb, batch)
    y = _run(ctx, q, xh, rows, sb, batch)
    _check(y, q, xh, rows, sb, batch, f"edge {rows}x{sb} B={batch}")


@pytest.mark.parametrize("rows,sb,batch,kernel", [(1024, 16, 250, "sr_w8_s2_n2"),
                                                  (2000, 16, 100, "sr_w8_s2_n2"),
                                                  (1000, 16, 60, "sr_w8_s2"),
                                                  (1024, 56, 128, "lk_c16_x1_w3_r2"),
                                                  (1000, 56, 60, "lk_c16_x1_w3"),
                                                  (500, 33, 127, "lk_c16_x1_w3"),
                                                  (64, 1100, 64, "ks_k8_n1_p1_r1"),
                                                  (20480, 16, 128, "rm_w4_r1_p4"),
                                                  (4000, 56, 30, "lk_c16_x1_w3_r2"),
                                                  (4000, 56, 16, "lk_c16_x1_w3"),
                                                  (4000, 56, 7, "lk_c8_x2_w2"),
                                                  (4000, 43, 3, "lk_c4_x2_w2"),
                                                  (1024, 32, 7, "lk_c4_x2_w2"),
                                                  (8100, 43, 5, "lk_c8_x2_w2_r2"),
                                                  (11000, 43, 5, "kx_r4_n1_k4_p3"),
                                                  (1000, 43, 31, "lk_c8_x2_w2"),
                                                  (4096, 56, 100, "kx_r4_n2_k4_p3")])
def test_grid_fill_defaults(ctx, axc, rows, sb, batch, kernel):
    """The defaults that follow from the grid on few rows: streaming rows past
    32 columns (several column groups, the last one partial), kind 9 at K >
    4096 up to 32 columns and, where one wave of its 16-column tiles fills
    the chip, beyond (partial last column group), the K-split kind for rows
    too long for kind 9, K-split tiles with their columns halved, and 32 x 32
    tiles at 128 columns on enough rows."""
    assert axc.q4k_matmul_kernel_name(rows, sb, batch) == "axh_q4k_matmul_" + kernel
    _say(f"matmul default {kernel} {rows}x{sb * 256} B={batch}")
    q, xh = _inputs(rows + 3 * sb + 5 * batch, rows, sb, batch)
    y = _run(ctx, q, xh, rows, sb, batch)
    _check(y, q, xh, rows, sb, batch, f"default {kernel} {rows}x{sb} B={batch}")


def test_every_variant(ctx, axc):
    rows, sb, batch = 200, 3, 40
    q, xh = _inputs(91, rows, sb, batch)
    for v in axc.compiled_matmul_variants():
        _say(f"matmul variant {v}")
        y = _run(ctx, q, xh, rows, sb, batch, v)
        _check(y, q, xh, rows, sb, batch, f"variant {v}")


@pytest.mark.parametrize("rows,sb,batch", [(1, 1, 1), (37, 7, 129), (130, 2, 15),
                                           (300, 3, 260), (1000, 1, 33)])
def test_tile_kinds_on_odd_shapes(ctx, axc, rows, sb, batch):
    """The K-split tile and 32x32 tile kinds (5, 8) at shapes none of
    their tiles divide: a single row, superblock and column; more superblocks
    than a wave's ring holds, column groups of 129 and 260; rows past one row
    tile; a single superblock (four K steps)."""
    q, xh = _inputs(rows * 11 + sb + batch, rows, sb, batch)
    for v in axc.compiled_matmul_variants():
        if v.kind not in (5, 8):
            continue
        _say(f"matmul odd shape {rows}x{sb} B={batch} variant {v}")
        y = _run(ctx, q, xh, rows, sb, batch, v)
        _check(y, q, xh, rows, sb, batch, f"odd {rows}x{sb} B={batch} {v}")


@pytest.mark.parametrize("rows,sb,batch", [(4096, 56, 8), (1000, 43, 5), (37, 9, 16), (130, 1, 1),
                                           (300, 17, 20), (64, 64, 3), (20, 8, 9), (100, 20, 2)])
def test_long_rows_kind(ctx, axc, rows, sb, batch):
    """Kind 9 (8 waves over one 16-row block, K in chunks of 8 superblocks,
    X through an LDS ring) in every compiled form: whole and partial chunks
    (56, 43, 9, 1, 17 superblocks; 64 and 8 fill the ring rounds exactly),
    more chunks than the ring holds, rows past the last block, 4-, 8- and
    16-column groups with partial ones (2, 3, 5, 9, 16, 20 columns)."""
    q, xh = _inputs(rows * 5 + sb * 7 + batch, rows, sb, batch)
    for v in axc.compiled_matmul_variants():
        if v.kind != 9:
            continue
        _say(f"matmul long rows {rows}x{sb * 256} B={batch} "
             f"{axc.q4k_matmul_kernel_name(rows, sb, batch, v)}")
        y = _run(ctx, q, xh, rows, sb, batch, v)
        _check(y, q, xh, rows, sb, batch, f"long rows {rows}x{sb} B={batch} {v}")


@pytest.mark.parametrize("rows,sb,batch", [(5000, 13, 13), (4097, 16, 16), (17, 7, 1),
                                           (1000, 16, 3), (70000, 2, 9), (4097, 16, 32),
                                           (333, 11, 19), (70000, 3, 25), (14336, 16, 8),
                                           (4099, 5, 7), (7296, 16, 16), (14331, 16, 32),
                                           (34368, 4, 5), (32768, 2, 8), (34368, 2, 30),
                                           (66336, 2, 12), (65536, 2, 16)])
def test_streaming_rows_kind(ctx, axc, rows, sb, batch):
    """Kind 7 (the default up to 32 columns and K <= 4096; 8-column groups up
    to 8 columns, two column groups per workgroup beyond 16 columns): more
    16-row blocks than workgroups (several per workgroup), a partial last
    block, rows not a multiple of 4 (scalar stores), waves whose superblocks
    lie past the row (K < 4096), a single column.  On a 256-CU grid the last
    round's blocks become 8-row half blocks where they fill at most half of it
    (14336 rows: exactly half; 4097, 5000, 70000: fewer; 14331 and 5000: the
    last half block partly past the matrix) and stay whole where they fill
    more (7296 rows: 200 of 256).  The waves' partial tiles are summed when
    their LDS regions fill (16 blocks with one 16-column group, 8 with two or
    with 8-column groups) and at the end: 70000 and 66336 rows sum a full
    group and then the rest; 34368 rows fill a group exactly before the half
    block; 32768 and 65536 rows end on a full group."""
    assert axc.q4k_matmul_kernel_name(rows, sb, batch).startswith("axh_q4k_matmul_sr_w8_s2")
    _say(f"matmul streaming rows {rows}x{sb * 256} B={batch}")
    q, xh = _inputs(rows + sb * 5 + batch, rows, sb, batch)
    y = _run(ctx, q, xh, rows, sb, batch)
    _check(y, q, xh, rows, sb, batch, f"streaming rows {rows}x{sb} B={batch}")


@pytest.mark.parametrize("rows,sb,batch,pf", [(1000, 16, 3, 1), (4097, 16, 8, 1),
                                              (5000, 13, 13, 2), (70000, 3, 25, 2),
                                              (333, 11, 16, 2)])
def test_streaming_rows_group_widths(ctx, axc, rows, sb, batch, pf):
    """Both column-group widths of kind 7 away from their defaults: 16-column
    groups at <= 8 columns, 8-column groups (two or more per matrix) beyond."""
    v = axc.MatmulVariant(7, 8, 1, pf)
    want = "axh_q4k_matmul_sr_w8_s2" + ("_h" if pf == 2 else "")
    assert axc.q4k_matmul_kernel_name(rows, sb, batch, v) == want
    _say(f"matmul streaming rows {rows}x{sb * 256} B={batch} prefetch {pf}")
    q, xh = _inputs(rows + sb * 7 + batch + pf, rows, sb, batch)
    y = _run(ctx, q, xh, rows, sb, batch, v)
    _check(y, q, xh, rows, sb, batch, f"streaming rows {rows}x{sb} B={batch} pf {pf}")


@pytest.mark.parametrize("batch", [8, 40, 200])
def test_output_only_4_byte_aligned(ctx, batch):
    """y 4 bytes past a 16-byte boundary: the tile stores fall back to single
    words (the API asks y for 4-byte alignment only); nothing outside y is
    written."""
    rows, sb = 70, 2
    q, xh = _inputs(900 + batch, rows, sb, batch)
    dq, dx = _dev(ctx, q), _dev(ctx, xh)
    n = batch * rows
    dy = ctx.alloc(n * 4 + 32)
    guard = np.full(n + 8, -7.0, dtype=np.float32)
    ctx.upload(dy, guard)
    _say(f"matmul unaligned y B={batch}")
    ctx.q4k_matmul(dq, dx, dy.ptr + 4, rows, sb, batch)
    ctx.synchronize()
    out = np.frombuffer(ctx.download(dy, (n + 8) * 4), dtype=np.float32)
    for b in (dq, dx, dy):
        b.close()
    assert out[0] == -7.0 and np.all(out[n + 1:] == -7.0)
    y = out[1:n + 1].reshape(batch, rows).copy()
    _check(y, q, xh, rows, sb, batch, f"unaligned y B={batch}")


def test_batch_one_matches_the_matvec_within_f16_weight_rounding(ctx):
    rows, sb = 512, 16
    q, xh = _inputs(93, rows, sb, 1)
    y = _run(ctx, q, xh, rows, sb, 1)[0]
    dq, dx, dy = _dev(ctx, q), _dev(ctx, xh.astype(np.float32)), ctx.alloc(rows * 4)
    ctx.q4k_matvec(dq, dx, dy, rows, sb)
    ctx.synchronize()
    ymv = np.frombuffer(ctx.download(dy, rows * 4), dtype=np.float32)
    for b in (dq, dx, dy):
        b.close()
    absd = np.abs(_w32(q, rows, sb).astype(np.float64)) @ np.abs(xh.astype(np.float64))
    assert np.all(np.abs(y.astype(np.float64) - ymv) <= (2.0 ** -11 + 2e-5) * absd)


@pytest.mark.parametrize("batch", [4, 8, 16, 32])
def test_long_rows_columns_are_independent_at_full_size(ctx, axc, batch):
    """The batched down-projection (4096 x 14336, the north star's weights) at
    its defaults: every column of a batched call equals, bit for bit, the same
    column run alone in the first column slot of the same kernel (the column
    tiles sum the same products in the same order whichever slot a column
    takes), and the whole result meets the f16-weight product check."""
    rows, sb = 4096, 56
    name = axc.q4k_matmul_kernel_name(rows, sb, batch)
    assert name.startswith("axh_q4k_matmul_lk_")
    _say(f"matmul long rows columns {rows}x{sb * 256} B={batch} {name}")
    q, xh = _inputs(700 + batch, rows, sb, batch)
    dq = _dev(ctx, q)
    dx, dy = _dev(ctx, xh), ctx.alloc(batch * rows * 4)
    def named(u):
        try:
            return axc.q4k_matmul_kernel_name(rows, sb, batch, u)
        except axc.DispatchError:  # kinds that do not take this shape
            return None
    v = next(u for u in axc.compiled_matmul_variants() if named(u) == name)
    ctx.q4k_matmul(dq, dx, dy, rows, sb, batch, v)
    ctx.synchronize()
    y = np.frombuffer(ctx.download(dy, batch * rows * 4), dtype=np.float32).reshape(batch, rows)
    x2 = xh.reshape(batch, sb * 256)
    d1, o1 = ctx.alloc(sb * 256 * 2), ctx.alloc(rows * 4)
    for b in range(batch):
        ctx.upload(d1, np.ascontiguousarray(x2[b]))
        ctx.q4k_matmul(dq, d1, o1, rows, sb, 1, v)
        ctx.synchronize()
        y1 = np.frombuffer(ctx.download(o1, rows * 4), dtype=np.float32)
        assert np.array_equal(y1.view(np.uint32), y[b].view(np.uint32)), f"column {b}"
    for buf in (dq, dx, dy, d1, o1):
        buf.close()
    _check(y.copy(), q, xh, rows, sb, batch, f"long rows full size B={batch}", oracle_f32=False)


def test_invalid_arguments_are_typed_errors(ctx, axc):
    b = ctx.alloc(64)
    with pytest.raises(axc.DispatchError):
        ctx.q4k_matmul(b, b, b, 4, 0, 2)  # no superblocks
    with pytest.raises(axc.DispatchError):
        ctx.q4k_matmul(b, b, b, 4, 1, 2, axc.MatmulVariant(1, 3, 3, 1))  # not compiled
    ctx.q4k_matmul(b, b, b, 0, 1, 2)  # empty: nothing to do
    b.close()


def _x32_with_ties(seed, n):
    """N(0, 1) f32 activations plus exact f16 rounding ties (both directions of
    ties-to-even), values in the f16 subnormal range and exact f16 values."""
    x = O.gen_normal_f32(seed, n)
    m = n // 8
    k = np.arange(m, dtype=np.float32)
    x[:m] = (1.0 + (2 * (k % 512) + 1) * 2.0 ** -11).astype(np.float32)  # halfway cases
    x[m:2 * m] = (k % 1000 - 500).astype(np.float32) * np.float32(2.0 ** -25)  # subnormals
    x[2 * m:3 * m] = -x[:m] * np.float32(3.0)
    return x


def _run_f32(ctx, q, x32, rows, sb, batch, variant=None):
    dq, dx, dy = _dev(ctx, q), _dev(ctx, x32), ctx.alloc(batch * rows * 4)
    dx16 = ctx.alloc(max(16, x32.size * 2))
    ctx.q4k_matmul_f32(dq, dx, dx16, dy, rows, sb, batch, variant)
    ctx.synchronize()
    y = np.frombuffer(ctx.download(dy, batch * rows * 4), dtype=np.float32).reshape(batch, rows)
    x16 = np.frombuffer(ctx.download(dx16, x32.size * 2), dtype=np.uint16)
    for b in (dq, dx, dy, dx16):
        b.close()
    return y.copy(), x16.copy()


@pytest.mark.parametrize("rows,sb,batch", [(14336, 16, 8), (14336, 16, 32), (14336, 16, 512),
                                           (257, 2, 130), (31, 4, 1)])
def test_f32_activations_equal_f16_kernel_on_rn_f16_x(ctx, rows, sb, batch):
    """f32 activations: the cast buffer holds numpy's round-to-nearest-even f16
    of x bit for bit, and Y equals the f16 entry point on it bit for bit."""
    _say(f"matmul f32 X {rows}x{sb * 256} B={batch}")
    q = O.gen_q4k_weights(rows + batch, rows * sb)
    x32 = _x32_with_ties(rows + 3 * batch, sb * 256 * batch)
    y32, x16 = _run_f32(ctx, q, x32, rows, sb, batch)
    assert np.array_equal(x16, x32.astype(np.float16).view(np.uint16))
    y16 = _run(ctx, q, x32.astype(np.float16), rows, sb, batch)
    assert np.array_equal(y32.view(np.uint32), y16.view(np.uint32))


def test_f32_activations_every_variant(ctx, axc):
    rows, sb, batch = 200, 3, 40
    q = O.gen_q4k_weights(95, rows * sb)
    x32 = _x32_with_ties(96, sb * 256 * batch)
    xh = x32.astype(np.float16)
    for v in axc.compiled_matmul_variants():
        _say(f"matmul f32 X variant {v}")
        y32, _ = _run_f32(ctx, q, x32, rows, sb, batch, v)
        y16 = _run(ctx, q, xh, rows, sb, batch, v)
        assert np.array_equal(y32.view(np.uint32), y16.view(np.uint32)), str(v)
        _check(y32, q, xh, rows, sb, batch, f"f32 X variant {v}")


def _cast(ctx, x32):
    dx, dh = _dev(ctx, x32), ctx.alloc(max(16, x32.size * 2))
    ctx.f32_to_f16(dx, dh, x32.size)
    ctx.synchronize()
    h = np.frombuffer(ctx.download(dh, x32.size * 2), dtype=np.uint16).copy()
    for b in (dx, dh):
        b.close()
    return h


@pytest.mark.parametrize("n", [1, 7, 8, 9, 15, 17, 4096 * 32 + 5])
def test_f32_to_f16_cast_matches_numpy(ctx, n):
    """Every class of f32 input against numpy's RNE cast, bit for bit (NaN by
    class): ties both ways, f16 subnormals and underflow to zero, overflow to
    infinity, signed zeros, infinities; n covers the 8-value groups and tails."""
    rng = np.random.default_rng(n)
    bits = rng.integers(0, 2 ** 32, size=n, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32).copy()
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65520.0, 65519.99,
                        2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 3 * 2.0 ** -26,
                        1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, -(1 + 2.0 ** -11), 6.1e-5],
                       dtype=np.float32)
    m = min(n, special.size)
    x[:m] = special[:m]
    half = n // 2
    x[m:half] = rng.normal(size=max(0, half - m)).astype(np.float32)
    h = _cast(ctx, x)
    with np.errstate(over="ignore", invalid="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(h[~nan], want[~nan])
    assert np.all(np.isnan(h[nan].view(np.float16)))
