"""GPU parity of the HIP path against the CPU oracle (marked `gpu`).

Bars: dequantised weights and the f16 decode bit-exact; matvec outputs under
the row-wise tolerance criterion of oracle.matvec_tolerance_report (1e-3
relative per well-conditioned row, condition-scaled bound on cancelling
rows, 1e-3 norm-wise) plus the reference's own single-output check
(rel < 1e-3, compile_q4km_dequant_matvec.rs:946-956).
"""
from __future__ import annotations

import struct
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3  # @equiv_fp_tol(1e-3), DESIGN.md:508-513 of the reference


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _to_dev(ctx, arr: np.ndarray):
    b = ctx.alloc(arr.nbytes)
    ctx.upload(b, arr)
    return b


def _run_q4k(ctx, q, x, rows, sb, variant=None):
    dq, dx, dy = _to_dev(ctx, q), _to_dev(ctx, x), ctx.alloc(rows * 4)
    ctx.q4k_matvec(dq, dx, dy, rows, sb, variant)
    ctx.synchronize()
    y = np.frombuffer(ctx.download(dy, rows * 4), dtype=np.float32).copy()
    for b in (dq, dx, dy):
        b.close()
    return y


def _run_q4_0(ctx, q, x, rows, nb, variant=None):
    dq, dx, dy = _to_dev(ctx, q), _to_dev(ctx, x), ctx.alloc(rows * 4)
    ctx.q4_0_matvec(dq, dx, dy, rows, nb, variant)
    ctx.synchronize()
    y = np.frombuffer(ctx.download(dy, rows * 4), dtype=np.float32).copy()
    for b in (dq, dx, dy):
        b.close()
    return y


def _check_q4k(y, q, x, rows, sb, what):
    ref = O.q4k_matvec(q, x, rows, sb)
    yf, absdot = O.q4k_matvec_f64(q, x, rows, sb)
    rep = O.matvec_tolerance_report(y, ref, yf, absdot, sb * 256, REL_TOL)
    _say(f"{what}: {rep}")
    assert rep["ok"], f"{what}: {rep}"


def _check_q4_0(y, q, x, rows, nb, what):
    ref = O.q4_0_matvec(q, x, rows, nb)
    yf, absdot = O.q4_0_matvec_f64(q, x, rows, nb)
    rep = O.matvec_tolerance_report(y, ref, yf, absdot, nb * 32, REL_TOL)
    _say(f"{what}: {rep}")
    assert rep["ok"], f"{what}: {rep}"


# ---- a3: f16 decode --------------------------------------------------------
def test_f16_widen_exhaustive_matches_oracle(ctx):
    _say("f16 widen: all 65536 patterns")
    h = np.arange(65536, dtype=np.uint16)
    dh, df = _to_dev(ctx, h), ctx.alloc(65536 * 4)
    ctx.f16_widen(dh, df, 65536)
    ctx.synchronize()
    gpu = np.frombuffer(ctx.download(df, 65536 * 4), dtype=np.uint32)
    ref = h.view(np.float16).astype(np.float32).view(np.uint32)
    nan = np.isnan(h.view(np.float16))
    assert np.array_equal(gpu[~nan], ref[~nan])
    assert np.isnan(gpu[nan].view(np.float32)).all()
    dh.close()
    df.close()


# ---- a1/a4/a5: bit-exact dequantisation -------------------------------------
@pytest.mark.parametrize("rows,sb", [(1, 128), (4096, 16), (4096, 56)])
def test_q4k_dequant_bit_exact(ctx, rows, sb):
    _say(f"q4k dequant bit-exact {rows}x{sb * 256}")
    n = rows * sb
    q = O.gen_q4k_weights(11 + rows, n)
    dq, dw = _to_dev(ctx, q), ctx.alloc(n * 256 * 4)
    ctx.q4k_dequant(dq, dw, n)
    ctx.synchronize()
    gpu = np.frombuffer(ctx.download(dw, n * 256 * 4), dtype=np.uint32)
    ref = O.q4k_dequant(q, n).view(np.uint32)
    bad = np.flatnonzero(gpu != ref)
    assert bad.size == 0, f"{bad.size} mismatching weights, first at {bad[:5]}"
    dq.close()
    dw.close()


def test_q4k_dequant_bit_exact_lcg_fixture(ctx):
    """Reference generator data (d in [0.1, 2], dmin in [0, 0.5])."""
    q, _ = O.generate_q4km_test_data(512, 0xCAFEBABE)
    dq, dw = _to_dev(ctx, q), ctx.alloc(512 * 256 * 4)
    ctx.q4k_dequant(dq, dw, 512)
    ctx.synchronize()
    gpu = np.frombuffer(ctx.download(dw, 512 * 256 * 4), dtype=np.uint32)
    assert np.array_equal(gpu, O.q4k_dequant(q, 512).view(np.uint32))
    dq.close()
    dw.close()


@pytest.mark.parametrize("rows,nb", [(256, 128), (7, 129)])
def test_q4_0_dequant_bit_exact(ctx, rows, nb):
    _say(f"q4_0 dequant bit-exact {rows}x{nb * 32}")
    n = rows * nb
    q = O.gen_q4_0_weights(5 + rows, n)
    dq, dw = _to_dev(ctx, q), ctx.alloc(n * 32 * 4)
    ctx.q4_0_dequant(dq, dw, n)
    ctx.synchronize()
    gpu = np.frombuffer(ctx.download(dw, n * 32 * 4), dtype=np.uint32)
    assert np.array_equal(gpu, O.q4_0_dequant(q, n).view(np.uint32))
    dq.close()
    dw.close()


# ---- a6: Q4_K matvec at the BASELINE configurations ---------------------------
@pytest.mark.parametrize(
    "rows,sb,sigma",
    [
        (1, 128, 1.0),      # C2: 1 x 32768
        (4096, 16, 1.0),    # C3: 4096 x 4096
        (14336, 16, 1.0),   # C3: 14336 x 4096
        (4096, 56, 0.5),    # C4: 4096 x 14336 (north star)
    ],
)
def test_q4k_matvec_baseline_configs(ctx, rows, sb, sigma):
    _say(f"q4k matvec {rows}x{sb * 256}")
    q = O.gen_q4k_weights(1000 + rows + sb, rows * sb)
    x = O.gen_normal_f32(2000 + sb, sb * 256, sigma)
    y = _run_q4k(ctx, q, x, rows, sb)
    _check_q4k(y, q, x, rows, sb, f"q4k {rows}x{sb * 256}")


def test_q4k_matvec_output_head(ctx):
    """C4 output head 128256 x 4096 (295 MB of weights)."""
    rows, sb = 128256, 16
    _say(f"q4k matvec head {rows}x{sb * 256}")
    q = O.gen_q4k_weights(77, rows * sb)
    x = O.gen_normal_f32(78, sb * 256, 0.5)
    y = _run_q4k(ctx, q, x, rows, sb)
    _check_q4k(y, q, x, rows, sb, "q4k head")


def test_q4k_matvec_every_variant(ctx, axc):
    rows, sb = 1000, 57  # ragged: rows and superblocks not multiples of the tiles
    q = O.gen_q4k_weights(3, rows * sb)
    x = O.gen_normal_f32(4, sb * 256)
    for v in axc.compiled_variants("q4k"):
        _say(f"q4k variant {v}")
        y = _run_q4k(ctx, q, x, rows, sb, v)
        _check_q4k(y, q, x, rows, sb, f"variant {v}")


@pytest.mark.parametrize("rows,sb", [(1, 1), (3, 7), (5, 8), (9, 9), (65, 129), (2, 160), (33, 300),
                                     (31, 128), (17, 56), (4, 33), (30, 100), (32, 56)])
def test_q4k_matvec_edge_shapes(ctx, rows, sb):
    """Single superblock, ragged tails, rows longer than one LDS tile, and the
    few-row shapes that split a row across 1..8 waves (every partial batch)."""
    _say(f"q4k edge {rows}x{sb}")
    q = O.gen_q4k_weights(rows * 31 + sb, rows * sb)
    x = O.gen_normal_f32(rows + 5 * sb, sb * 256)
    y = _run_q4k(ctx, q, x, rows, sb)
    _check_q4k(y, q, x, rows, sb, f"q4k edge {rows}x{sb}")


def test_q4k_matvec_zero_superblocks_gives_positive_zero(ctx):
    """AT-1323: n_superblocks = 0 -> +0.0 (compile_q4km_dequant_matvec.rs:850-856)."""
    dq, dx, dy = ctx.alloc(16), ctx.alloc(16), ctx.alloc(4 * 4)
    ctx.upload(dy, np.full(4, 7.0, dtype=np.float32))
    ctx.q4k_matvec(dq, dx, dy, 4, 0)
    ctx.synchronize()
    y = np.frombuffer(ctx.download(dy, 16), dtype=np.uint32)
    assert (y == 0).all()


def test_q4k_matvec_lcg_fixture_single_row(ctx):
    """AT-1324/1331 data: generate_q4km_test_data(128, 0xDEADBEEF)."""
    q, x = O.generate_q4km_test_data(128, 0xDEADBEEF)
    y = _run_q4k(ctx, q, x, 1, 128)
    cpu = O.q4k_dot(q, x, 128)
    assert O.reference_rel_err(y[0], cpu) < REL_TOL


# ---- a2: Q4_0 matvec ---------------------------------------------------------
def test_q4_0_matvec_c1(ctx):
    rows, nb = 256, 128
    _say("q4_0 matvec C1 256x4096")
    q = O.gen_q4_0_weights(42, rows * nb)
    x = O.gen_normal_f32(43, nb * 32)
    y = _run_q4_0(ctx, q, x, rows, nb)
    _check_q4_0(y, q, x, rows, nb, "q4_0 C1")


def test_q4_0_matvec_every_variant(ctx, axc):
    rows, nb = 300, 130
    q = O.gen_q4_0_weights(9, rows * nb)
    x = O.gen_normal_f32(10, nb * 32)
    for v in axc.compiled_variants("q4_0"):
        _say(f"q4_0 variant {v}")
        y = _run_q4_0(ctx, q, x, rows, nb, v)
        _check_q4_0(y, q, x, rows, nb, f"q4_0 variant {v}")


@pytest.mark.parametrize("rows,nb", [(1, 1), (2, 3), (3, 127), (4, 129), (5, 1025), (17, 2048),
                                     (1, 2), (3, 2), (7, 64), (33, 126), (2049, 128), (100, 10)])
def test_q4_0_matvec_edge_shapes(ctx, rows, nb):
    """Odd block counts and long rows (LDS-tiled kernel); even counts up to
    128 blocks on fewer than 32 rows (column kernel: idle lanes, one block
    pair) and on more rows (tiled, one pass)."""
    _say(f"q4_0 edge {rows}x{nb}")
    q = O.gen_q4_0_weights(rows * 13 + nb, rows * nb)
    x = O.gen_normal_f32(rows + nb, nb * 32)
    y = _run_q4_0(ctx, q, x, rows, nb)
    _check_q4_0(y, q, x, rows, nb, f"q4_0 edge {rows}x{nb}")


@pytest.mark.parametrize("rows,nb", [(1, 2), (3, 2), (7, 64), (31, 128), (100, 10), (33, 126),
                                     (2049, 128)])
def test_q4_0_column_kernel(ctx, axc, rows, nb):
    """The column kernel (on request; rows of an even block count up to 128):
    one block pair per lane, one row and several, within the oracle's
    tolerance."""
    v = axc.Variant(family=axc.FAMILY_COLUMNS)
    assert axc.q4_0_matvec_kernel_name(rows, nb, v) == "axh_q4_0_matvec_cols_r1"
    _say(f"q4_0 columns {rows}x{nb}")
    q = O.gen_q4_0_weights(rows * 11 + nb, rows * nb)
    x = O.gen_normal_f32(rows + 2 * nb, nb * 32)
    y = _run_q4_0(ctx, q, x, rows, nb, v)
    _check_q4_0(y, q, x, rows, nb, f"q4_0 columns {rows}x{nb}")


def _q4_0_octet_variants(axc, rows, nb):
    """Every octet-kernel variant that takes this shape: each compiled
    persistent variant, one pass with x one and two chunks ahead, with x whole,
    and a trip count one past the row's."""
    V = axc.Variant
    need = (nb + 63) // 64
    cands = [V(r, w, pf, 0, axc.FAMILY_PERSISTENT)
             for r, w, pf in ((1, 4, 1), (1, 8, 1), (2, 4, 1), (2, 8, 1), (1, 8, 2), (2, 4, 2),
                              (1, 16, 2))]
    cands += [V(prefetch=1, family=axc.FAMILY_ONE_PASS), V(family=axc.FAMILY_ONE_PASS_X),
              V(prefetch=2, family=axc.FAMILY_ONE_PASS, sb_per_lane=max(need, 3)),
              V(prefetch=1, family=axc.FAMILY_ONE_PASS, sb_per_lane=need + 1)]
    out = []
    for v in cands:
        try:
            out.append((v, axc.q4_0_matvec_kernel_name(rows, nb, v)))
        except axc.DispatchError:
            pass  # row too long for this variant's x staging, or past 16 steps
    return out


@pytest.mark.parametrize("rows,nb", [(1, 2), (2, 66), (3, 130), (33, 130), (5, 8), (100, 446),
                                     (257, 1022), (31, 1024), (1000, 64), (64, 960),
                                     (4097, 128), (47, 512)])
def test_q4_0_octet_kernels_bit_exact(ctx, axc, rows, nb):
    """Q4_0 through the persistent and one-pass kernels (rows read as octets of
    8 blocks): partial last octets (a quarter of 2 blocks live, or 3), odd row
    counts, one row, trip counts 1..16.  Every variant runs the same per-lane
    order and reduction, so all of them agree bit for bit, and with the oracle
    to its tolerance."""
    q = O.gen_q4_0_weights(rows * 17 + nb, rows * nb)
    x = O.gen_normal_f32(rows * 3 + nb, nb * 32)
    got = {}
    for v, kname in _q4_0_octet_variants(axc, rows, nb):
        _say(f"q4_0 octets {rows}x{nb} {kname}")
        y = _run_q4_0(ctx, q, x, rows, nb, v)
        _check_q4_0(y, q, x, rows, nb, f"q4_0 octets {rows}x{nb} {kname}")
        got[kname] = y
    assert len(got) >= 6, sorted(got)
    first = next(iter(got.values()))
    for kname, y in got.items():
        assert np.array_equal(y.view(np.uint32), first.view(np.uint32)), kname


@pytest.mark.parametrize("rows,nb,kernel", [(4096, 448, "one_i7"), (6144, 128, "onex_i2"),
                                            (16385, 258, "flat_r1_w8_p1_x1"),
                                            (4096, 1024, "onep_i16"), (1025, 128, "one_i2"),
                                            (14336, 127, "r4_w4"), (20, 1024, "r1_w4"),
                                            (31, 128, "r1_w4"), (1, 2, "r1_w4"),
                                            (200, 224, "r1_w4"), (257, 224, "one_i4")])
def test_q4_0_defaults_by_shape(ctx, axc, rows, nb, kernel):
    """The default Q4_0 kernel of each shape band (one pass, x whole, x two
    chunks ahead, persistent, LDS-tiled for odd and few rows) against the
    oracle."""
    assert axc.q4_0_matvec_kernel_name(rows, nb) == f"axh_q4_0_matvec_{kernel}"
    _say(f"q4_0 default {rows}x{nb} {kernel}")
    q = O.gen_q4_0_weights(rows + 5 * nb, rows * nb)
    x = O.gen_normal_f32(rows + 11 * nb, nb * 32)
    y = _run_q4_0(ctx, q, x, rows, nb)
    _check_q4_0(y, q, x, rows, nb, f"q4_0 default {rows}x{nb}")


# ---- the reference kernel contract through prepare_kernel / dispatch_handle --
def _plan(axc, pc):
    return axc.BindingPlan(
        buffers=[axc.axh.ACCESS_READ_ONLY, axc.axh.ACCESS_READ_ONLY, axc.axh.ACCESS_READ_WRITE],
        push_constant_total_bytes=pc, workgroup_size=(64, 1, 1))


def test_at_1324_q4km_dispatch_handle_matches_cpu_within_1e_3(ctx, axc):
    """compile_q4km_dequant_matvec.rs:867-957 on the HIP runtime."""
    n = 128
    q, x = O.generate_q4km_test_data(n, 0xDEADBEEF)
    cpu = O.q4k_dot(q, x, n)
    co = axc.builtin_code_object()
    h = ctx.prepare_kernel(co, _plan(axc, 4), 4, "q4km_dequant_matvec")
    out = ctx.dispatch_handle(h, (1, 1, 1), [q.tobytes(), x.tobytes(), bytes(4)],
                              [q.nbytes, x.nbytes, 4], struct.pack("<I", n))
    gpu = struct.unpack("<f", out[2][:4])[0]
    assert out[0] == q.tobytes() and out[1] == x.tobytes()
    assert O.reference_rel_err(gpu, cpu) < REL_TOL, (gpu, float(cpu))
    h.release()


def test_at_918_q4_0_dispatch_matches_cpu_within_1e_3(ctx, axc):
    """compile_q4_0_dequant_matvec.rs:437-537: 128 blocks, one output."""
    nb = 128
    q = O.gen_q4_0_weights(42, nb)
    x = O.gen_normal_f32(42, nb * 32)
    cpu = O.q4_0_dot(q, x, nb)
    req = axc.DispatchRequest(
        code_object=axc.builtin_code_object(), binding_plan=_plan(axc, 4), workgroups=(1, 1, 1),
        inputs=[q.tobytes(), x.tobytes(), bytes(4)], output_sizes=[0, 0, 4],
        push_constants=struct.pack("<I", nb), entry_point="q4_0_dequant_matvec")
    out = ctx.dispatch(req)
    assert out[0] == b"" and out[1] == b""
    gpu = struct.unpack("<f", out[2])[0]
    assert O.reference_rel_err(gpu, cpu) < REL_TOL, (gpu, float(cpu))


@pytest.mark.parametrize("n", [1, 16, 17, 512])
def test_q4km_reference_kernel_many_superblocks(ctx, axc, n):
    """More superblocks than one 16-superblock LDS tile (512 = dispatch_q4km_512)."""
    q, x = O.generate_q4km_test_data(n, 0xCAFEBABE)
    cpu = O.q4k_dot(q, x, n)
    h = ctx.prepare_kernel(axc.builtin_code_object(), _plan(axc, 4), 4, "q4km_dequant_matvec")
    out = ctx.dispatch_handle(h, (1, 1, 1), [q.tobytes(), x.tobytes(), b""], [0, 0, 4],
                              struct.pack("<I", n))
    gpu = struct.unpack("<f", out[2])[0]
    assert O.reference_rel_err(gpu, cpu) < REL_TOL, (n, gpu, float(cpu))


# ---- long rows, up to 4096 of them: one pass, one pair of rows per wave ---------
@pytest.mark.parametrize("rows,sb", [(32, 33), (33, 40), (47, 41), (100, 56), (4095, 57),
                                     (1000, 127), (64, 128), (32, 1), (33, 9), (4096, 16),
                                     (30001, 3), (777, 24)])
def test_q4k_one_pass_shapes(ctx, axc, rows, sb):
    """32..32768 rows of 1..128 superblocks: trip counts 1..16 and their
    boundaries (8k and 8k + 1 superblocks), odd row counts (a half-empty last
    pair) and workgroups past the last pair.  The one-pass family is requested
    (up to 1024 rows of 24+ superblocks the default is the tiled kernel)."""
    v = axc.Variant(family=axc.FAMILY_ONE_PASS)
    assert axc.q4k_matvec_kernel_name(rows, sb, v).startswith("axh_q4k_matvec_one")
    _say(f"q4k one pass {rows}x{sb}")
    q = O.gen_q4k_weights(rows * 23 + sb, rows * sb)
    x = O.gen_normal_f32(rows + 7 * sb, sb * 256)
    y = _run_q4k(ctx, q, x, rows, sb, v)
    _check_q4k(y, q, x, rows, sb, f"q4k one pass {rows}x{sb}")


@pytest.mark.parametrize("rows,sb", [(32, 24), (33, 40), (100, 56), (777, 24), (1000, 127),
                                     (1024, 128), (64, 113), (512, 14), (32, 13), (999, 17),
                                     (257, 20)])
def test_q4k_tiled_default_on_few_long_rows(ctx, axc, rows, sb):
    """32..1024 rows of 24..128 superblocks (17+ from 513 rows, 13+ up to 512)
    default to the tiled kernel with one row per wave: odd row counts, partial
    last workgroups and tiles."""
    assert axc.q4k_matvec_kernel_name(rows, sb) == "axh_q4k_matvec_tiled_r1_w4_p2"
    _say(f"q4k tiled default {rows}x{sb}")
    q = O.gen_q4k_weights(rows * 41 + sb, rows * sb)
    x = O.gen_normal_f32(rows + 19 * sb, sb * 256)
    y = _run_q4k(ctx, q, x, rows, sb)
    _check_q4k(y, q, x, rows, sb, f"q4k tiled default {rows}x{sb}")


@pytest.mark.parametrize("rows,sb", [(24576, 25), (28673, 32)])
def test_q4k_tall_persistent_default(ctx, axc, rows, sb):
    """24576-32768 rows of 25-32 superblocks default to the persistent kernel
    with 4 waves and early refill (an odd row count: a half-empty last pair)."""
    assert axc.q4k_matvec_kernel_name(rows, sb) == "axh_q4k_matvec_flat_r1_w4_p1_n0"
    _say(f"q4k tall persistent default {rows}x{sb}")
    q = O.gen_q4k_weights(rows + 29 * sb, rows * sb)
    x = O.gen_normal_f32(rows + 31 * sb, sb * 256)
    y = _run_q4k(ctx, q, x, rows, sb)
    _check_q4k(y, q, x, rows, sb, f"q4k tall persistent {rows}x{sb}")


@pytest.mark.parametrize("rows,sb,xd", [(32, 17, 2), (33, 24, 2), (4096, 25, 2), (4095, 56, 2),
                                        (4096, 56, 1), (2047, 128, 2), (100, 113, 2),
                                        (5000, 40, 2), (4096, 40, 1), (64, 121, 2)])
def test_q4k_one_pass_x_ahead(ctx, axc, rows, sb, xd):
    """Both x prefetch distances of the chunked one-pass kernel (the prefetch
    hole: one_i* one chunk ahead, onep_i* two), at trip counts 3..16 with a
    partial last chunk, odd row counts and partial last workgroups."""
    v = axc.Variant(prefetch=xd, family=axc.FAMILY_ONE_PASS)
    want = f"axh_q4k_matvec_one{'p' if xd == 2 else ''}_i{(sb + 7) // 8}"
    assert axc.q4k_matvec_kernel_name(rows, sb, v) == want
    _say(f"q4k one pass x {xd} ahead {rows}x{sb}")
    q = O.gen_q4k_weights(rows * 31 + sb + xd, rows * sb)
    x = O.gen_normal_f32(rows + 13 * sb, sb * 256)
    y = _run_q4k(ctx, q, x, rows, sb, v)
    _check_q4k(y, q, x, rows, sb, f"q4k one pass x {xd} ahead {rows}x{sb}")


@pytest.mark.parametrize("rows,sb", [(6144, 1), (6145, 8), (6151, 9), (8192, 17), (11008, 16),
                                     (14336, 16), (9999, 24), (6200, 25), (7001, 32),
                                     (32768, 2), (40001, 16), (65535, 3), (65536, 5)])
def test_q4k_one_pass_whole_x_shapes(ctx, axc, rows, sb):
    """The one-pass kernel that stages x whole (6144-32768 rows of at most 32
    superblocks, up to 65536 rows of at most 16): trip counts 1..4 and their
    boundaries, odd row counts and partial last workgroups."""
    assert axc.q4k_matvec_kernel_name(rows, sb) == f"axh_q4k_matvec_onex_i{(sb + 7) // 8}"
    _say(f"q4k one pass whole x {rows}x{sb}")
    q = O.gen_q4k_weights(rows * 29 + sb, rows * sb)
    x = O.gen_normal_f32(rows + 11 * sb, sb * 256)
    y = _run_q4k(ctx, q, x, rows, sb)
    _check_q4k(y, q, x, rows, sb, f"q4k one pass whole x {rows}x{sb}")


@pytest.mark.parametrize("rows,sb,kernel", [(4097, 1, "onex_i1"), (4160, 16, "onex_i2"),
                                            (5121, 24, "onex_i3"), (6143, 9, "onex_i2"),
                                            (4097, 25, "flat_r1_w4_p1_n0"),
                                            (4608, 32, "flat_r1_w4_p1_n0"),
                                            (6143, 31, "flat_r1_w4_p1_n0"),
                                            (4097, 74, "flat_r1_w16_p2_n0"),
                                            (8191, 128, "flat_r1_w16_p2_n0")])
def test_q4k_defaults_between_4097_and_6143_rows(ctx, axc, rows, sb, kernel):
    """The default between 4097 and 6143 rows: x staged whole for rows of up
    to 24 superblocks, the persistent kernel with one row per lane group for
    25-32, at both ends of the band and with odd row counts; and the
    persistent kernel for 4097-8191 rows of 74 or more superblocks."""
    assert axc.q4k_matvec_kernel_name(rows, sb) == f"axh_q4k_matvec_{kernel}"
    _say(f"q4k default {rows}x{sb} ({kernel})")
    q = O.gen_q4k_weights(rows * 37 + sb, rows * sb)
    x = O.gen_normal_f32(rows + 17 * sb, sb * 256)
    y = _run_q4k(ctx, q, x, rows, sb)
    _check_q4k(y, q, x, rows, sb, f"q4k default {rows}x{sb}")


@pytest.mark.parametrize("sb", [9, 40])
def test_q4k_early_refill_several_pairs_per_wave(ctx, axc, sb):
    """Prefetch-1 variants on more rows than the persistent grid holds, so
    each wave walks several bundle pairs after its chunk-staged first pass."""
    rows = 20011
    q = O.gen_q4k_weights(sb + 5, rows * sb)
    x = O.gen_normal_f32(sb + 6, sb * 256)
    vs = [v for v in axc.compiled_variants("q4k") if v.prefetch == 1]
    assert vs
    for v in vs:
        _say(f"q4k early refill {rows}x{sb} {v}")
        y = _run_q4k(ctx, q, x, rows, sb, v)
        _check_q4k(y, q, x, rows, sb, f"early refill {rows}x{sb} {v}")


# ---- few long rows: one workgroup (1-4 rows of up to 128 superblocks) ----------
@pytest.mark.parametrize("rows,sb", [(1, 33), (1, 64), (1, 65), (1, 127), (1, 128), (2, 33),
                                     (2, 100), (3, 64), (3, 71), (4, 128)])
def test_q4k_one_workgroup_shapes(ctx, axc, rows, sb):
    """1-4 rows of 33..128 superblocks take the one-workgroup kernel: idle
    lanes past the row, odd superblock counts, every row-batch size."""
    assert axc.q4k_matvec_kernel_name(rows, sb).startswith("axh_q4k_matvec_wg_")
    _say(f"q4k one-workgroup {rows}x{sb}")
    q = O.gen_q4k_weights(rows * 19 + sb, rows * sb)
    x = O.gen_normal_f32(rows + 5 * sb, sb * 256)
    y = _run_q4k(ctx, q, x, rows, sb)
    _check_q4k(y, q, x, rows, sb, f"q4k one-workgroup {rows}x{sb}")


# ---- few long rows: split-K across workgroups with a last-workgroup reduction --
@pytest.mark.parametrize("rows,sb", [(5, 64), (5, 65), (8, 128), (31, 128), (2, 255),
                                     (1, 256), (31, 200), (4, 129)])
def test_q4k_split_k_shapes(ctx, axc, rows, sb):
    """The split-K kernel (the default for fewer than 32 rows of 129-256
    superblocks the one-workgroup kernel does not take; requested here):
    ragged last slices, the 16-workgroup limit, and row counts up to 31."""
    v = axc.Variant(family=axc.FAMILY_SPLIT_K)
    assert axc.q4k_matvec_kernel_name(rows, sb, v).startswith("axh_q4k_matvec_sk_")
    if sb > 128:
        assert axc.q4k_matvec_kernel_name(rows, sb).startswith("axh_q4k_matvec_sk_")
    _say(f"q4k split-K {rows}x{sb}")
    q = O.gen_q4k_weights(rows * 17 + sb, rows * sb)
    x = O.gen_normal_f32(rows + 3 * sb, sb * 256)
    y = _run_q4k(ctx, q, x, rows, sb, v)
    _check_q4k(y, q, x, rows, sb, f"q4k split-K {rows}x{sb}")


def test_q4k_split_k_back_to_back_calls_reset_the_counter(ctx, axc):
    """Consecutive split-K calls with different grids on one stream, without
    synchronising in between: each must see a zero counter (the last
    workgroup of the previous call resets it)."""
    shapes = [(1, 128), (5, 250), (1, 64), (31, 128), (1, 128)]
    cases = []
    for i, (rows, sb) in enumerate(shapes):
        q = O.gen_q4k_weights(900 + i, rows * sb)
        x = O.gen_normal_f32(950 + i, sb * 256)
        dq, dx, dy = _to_dev(ctx, q), _to_dev(ctx, x), ctx.alloc(rows * 4)
        cases.append((rows, sb, q, x, dq, dx, dy))
    _say("split-K back-to-back")
    sk = axc.Variant(family=axc.FAMILY_SPLIT_K)
    for _ in range(3):
        for rows, sb, q, x, dq, dx, dy in cases:
            ctx.q4k_matvec(dq, dx, dy, rows, sb, sk)
    ctx.synchronize()
    for rows, sb, q, x, dq, dx, dy in cases:
        y = np.frombuffer(ctx.download(dy, rows * 4), dtype=np.float32).copy()
        _check_q4k(y, q, x, rows, sb, f"back-to-back {rows}x{sb}")
        for b in (dq, dx, dy):
            b.close()
