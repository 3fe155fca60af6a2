"""Fused SwiGLU gate/up projection on the GPU (marked `gpu`):
h[r] = silu(Wg[r] . x) * (Wu[r] . x) for two Q4_K_M matrices.

The reference has no such kernel (its dispatches stop at one matvec,
ROADMAP.md:54-72); the checks hold the fused result to the matvec's own
criterion:
  * against the f64 oracle (oracle.gate_up_tolerance_report: each dot product
    within the matvec tolerance, propagated through silu(g) * u, plus 1e-3
    norm-wise);
  * against two axh_q4k_matvec calls with the same holes, whose per-row
    arithmetic the fused kernel shares: silu(g) * u of those outputs agrees
    to f32 rounding of the final combination (pins the gate/up row pairing
    and the row order).
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _dev(ctx, arr):
    b = ctx.alloc(max(arr.nbytes, 16))
    ctx.upload(b, arr)
    return b


def _inputs(seed, rows, sb, sigma=0.5):
    qg = O.gen_q4k_weights(seed, rows * sb)
    qu = O.gen_q4k_weights(seed + 1, rows * sb)
    x = O.gen_normal_f32(seed + 2, sb * 256, sigma)
    return qg, qu, x


def _gate_up(ctx, qg, qu, x, rows, sb, variant=None):
    dg, du, dx, dh = _dev(ctx, qg), _dev(ctx, qu), _dev(ctx, x), ctx.alloc(rows * 4)
    ctx.q4k_gate_up(dg, du, dx, dh, rows, sb, variant)
    ctx.synchronize()
    h = np.frombuffer(ctx.download(dh, rows * 4), dtype=np.float32).copy()
    for b in (dg, du, dx, dh):
        b.close()
    return h


def _matvec(ctx, q, x, rows, sb, variant=None):
    dq, dx, dy = _dev(ctx, q), _dev(ctx, x), ctx.alloc(rows * 4)
    ctx.q4k_matvec(dq, dx, dy, rows, sb, variant)
    ctx.synchronize()
    y = np.frombuffer(ctx.download(dy, rows * 4), dtype=np.float32).copy()
    for b in (dq, dx, dy):
        b.close()
    return y


def _check(h, qg, qu, x, rows, sb, what):
    _, g, ag, u, au = O.q4k_gate_up_f64(qg, qu, x, rows, sb)
    rep = O.gate_up_tolerance_report(h, g, ag, u, au, sb * 256, REL_TOL)
    _say(f"{what}: {rep}")
    assert rep["ok"], f"{what}: {rep}"


def test_llama3_8b_ffn_shape(ctx):
    """Gate and up projections of Llama-3-8B: 14336 rows x 4096 columns each."""
    rows, sb = 14336, 16
    _say("gate_up 14336x4096")
    qg, qu, x = _inputs(700, rows, sb)
    h = _gate_up(ctx, qg, qu, x, rows, sb)
    _check(h, qg, qu, x, rows, sb, "gate_up 14336x4096")


@pytest.mark.parametrize("rows,sb", [(1, 1), (2, 1), (3, 5), (31, 128), (257, 16), (1000, 64),
                                     (100, 100), (4097, 8), (64, 33)])
def test_edge_shapes(ctx, rows, sb):
    """Odd row counts (partial bundles and pairs), one superblock, the longest
    staged row (128 superblocks), rows needing two staged x sub-blocks."""
    _say(f"gate_up edge {rows}x{sb}")
    qg, qu, x = _inputs(rows * 3 + sb, rows, sb, sigma=1.0)
    h = _gate_up(ctx, qg, qu, x, rows, sb)
    _check(h, qg, qu, x, rows, sb, f"edge {rows}x{sb}")


def test_every_variant_matches_two_matvecs(ctx, axc):
    rows, sb = 1531, 24
    qg, qu, x = _inputs(710, rows, sb)
    for v in axc.compiled_variants("gate_up"):
        _say(f"gate_up variant {v}")
        h = _gate_up(ctx, qg, qu, x, rows, sb, v)
        _check(h, qg, qu, x, rows, sb, f"variant {v}")
        mv = axc.Variant(v.rows_per_wave, v.waves_per_workgroup, v.prefetch, 2)
        try:
            g = _matvec(ctx, qg, x, rows, sb, mv)
            u = _matvec(ctx, qu, x, rows, sb, mv)
        except axc.DispatchError:
            continue  # no matvec compiled with these holes
        want = O.silu(g.astype(np.float64)) * u.astype(np.float64)
        assert np.all(np.abs(h - want) <= 4 * 2.0 ** -24 * np.abs(want) + 1e-30), str(v)


def test_early_refill_several_pairs_per_wave(ctx, axc):
    """Prefetch-1 variants with more rows than the persistent grid holds."""
    rows, sb = 20011, 9
    qg, qu, x = _inputs(711, rows, sb)
    vs = [v for v in axc.compiled_variants("gate_up") if v.prefetch == 1]
    assert vs
    for v in vs:
        _say(f"gate_up early refill {v}")
        h = _gate_up(ctx, qg, qu, x, rows, sb, v)
        _check(h, qg, qu, x, rows, sb, f"early refill {v}")


def test_large_gate_saturates_and_negative_gate_vanishes(ctx):
    """Rows scaled so |g| reaches hundreds: silu(g) -> g for g >> 0 and -> 0
    (no NaN from exp overflow) for g << 0."""
    rows, sb = 256, 4
    qg, qu, x = _inputs(720, rows, sb)
    x = (x * np.float32(40.0)).astype(np.float32)
    h = _gate_up(ctx, qg, qu, x, rows, sb)
    assert np.all(np.isfinite(h))
    _check(h, qg, qu, x, rows, sb, "saturating gates")


def test_invalid_arguments_are_typed_errors(ctx, axc):
    b = ctx.alloc(1 << 20)
    with pytest.raises(axc.DispatchError):
        ctx.q4k_gate_up(b, b, b, b, 4, 0)  # no superblocks
    with pytest.raises(axc.DispatchError):
        ctx.q4k_gate_up(b, b, b, b, 4, 129)  # row longer than the staged x
    with pytest.raises(axc.DispatchError):
        ctx.q4k_gate_up(b, b, b, b, 4, 1, axc.Variant(0, 0, 0, 1))  # no non-temporal kernel
    with pytest.raises(axc.DispatchError):
        ctx.q4k_gate_up(b, b, b, b, 4, 1, axc.Variant(3, 4, 2, 0))  # not compiled
    ctx.q4k_gate_up(b, b, b, b, 0, 1)  # empty: nothing to do
    b.close()


# ---- the same fusion over two Q4_0 matrices ---------------------------------------
def _inputs0(seed, rows, nb, sigma=0.5):
    qg = O.gen_q4_0_weights(seed, rows * nb)
    qu = O.gen_q4_0_weights(seed + 1, rows * nb)
    x = O.gen_normal_f32(seed + 2, nb * 32, sigma)
    return qg, qu, x


def _gate_up0(ctx, qg, qu, x, rows, nb, variant=None):
    dg, du, dx, dh = _dev(ctx, qg), _dev(ctx, qu), _dev(ctx, x), ctx.alloc(rows * 4)
    ctx.q4_0_gate_up(dg, du, dx, dh, rows, nb, variant)
    ctx.synchronize()
    h = np.frombuffer(ctx.download(dh, rows * 4), dtype=np.float32).copy()
    for b in (dg, du, dx, dh):
        b.close()
    return h


def _matvec0(ctx, q, x, rows, nb, variant=None):
    dq, dx, dy = _dev(ctx, q), _dev(ctx, x), ctx.alloc(rows * 4)
    ctx.q4_0_matvec(dq, dx, dy, rows, nb, variant)
    ctx.synchronize()
    y = np.frombuffer(ctx.download(dy, rows * 4), dtype=np.float32).copy()
    for b in (dq, dx, dy):
        b.close()
    return y


def _check0(h, qg, qu, x, rows, nb, what):
    _, g, ag, u, au = O.q4_0_gate_up_f64(qg, qu, x, rows, nb)
    rep = O.gate_up_tolerance_report(h, g, ag, u, au, nb * 32, REL_TOL)
    _say(f"{what}: {rep}")
    assert rep["ok"], f"{what}: {rep}"


def test_q4_0_llama3_8b_ffn_shape(ctx):
    """Gate and up projections of a Q4_0 Llama-3-8B: 14336 rows x 4096 columns."""
    rows, nb = 14336, 128
    _say("q4_0 gate_up 14336x4096")
    qg, qu, x = _inputs0(730, rows, nb)
    h = _gate_up0(ctx, qg, qu, x, rows, nb)
    _check0(h, qg, qu, x, rows, nb, "q4_0 gate_up 14336x4096")


@pytest.mark.parametrize("rows,nb", [(1, 2), (3, 66), (31, 1024), (257, 130), (1000, 64),
                                     (4097, 8), (64, 446), (20011, 18)])
def test_q4_0_edge_shapes(ctx, rows, nb):
    """Odd row counts, one block pair, partial last octets (a quarter of 2
    blocks live, or 3), the longest row (1024 blocks), more rows than the
    persistent grid holds."""
    _say(f"q4_0 gate_up edge {rows}x{nb}")
    qg, qu, x = _inputs0(rows * 3 + nb, rows, nb, sigma=1.0)
    h = _gate_up0(ctx, qg, qu, x, rows, nb)
    _check0(h, qg, qu, x, rows, nb, f"q4_0 edge {rows}x{nb}")


@pytest.mark.parametrize("holes", [(1, 4, 1), (1, 8, 1), (2, 4, 1), (1, 4, 2), (1, 8, 2)])
def test_q4_0_every_variant_matches_two_matvecs(ctx, axc, holes):
    """Each compiled Q4_0 gate/up variant against the oracle, and against two
    persistent Q4_0 matvecs with the same holes where one is compiled:
    silu(g) * u of their outputs agrees to f32 rounding of the combination."""
    rows, nb = 1531, 194
    qg, qu, x = _inputs0(740, rows, nb)
    v = axc.Variant(*holes, 0)
    _say(f"q4_0 gate_up variant {holes}: {axc.q4_0_gate_up_kernel_name(rows, nb, v)}")
    h = _gate_up0(ctx, qg, qu, x, rows, nb, v)
    _check0(h, qg, qu, x, rows, nb, f"q4_0 variant {holes}")
    mv = axc.Variant(*holes, 2, axc.FAMILY_PERSISTENT)
    try:
        g = _matvec0(ctx, qg, x, rows, nb, mv)
        u = _matvec0(ctx, qu, x, rows, nb, mv)
    except axc.DispatchError:
        return  # no matvec compiled with these holes
    want = O.silu(g.astype(np.float64)) * u.astype(np.float64)
    assert np.all(np.abs(h - want) <= 4 * 2.0 ** -24 * np.abs(want) + 1e-30), str(holes)


def test_q4_0_invalid_arguments_are_typed_errors(ctx, axc):
    b = ctx.alloc(1 << 20)
    for bad in ((4, 0, None), (4, 127, None), (4, 1026, None), (4, 2, axc.Variant(0, 0, 0, 1)),
                (4, 2, axc.Variant(4, 4, 1, 0)), (4, 2, axc.Variant(family=1))):
        with pytest.raises(axc.DispatchError):
            ctx.q4_0_gate_up(b, b, b, b, *bad)
    ctx.q4_0_gate_up(b, b, b, b, 0, 2)  # empty: nothing to do
    b.close()


# ---- wave-paired one-pass gate/up kernels (both formats) ------------------------
_PAIRED_SHAPES = [(1, 1, False), (7, 3, False), (14336, 16, False), (1531, 24, False),
                  (33, 64, False), (9, 2, True), (1531, 194, True), (14336, 128, True),
                  (100, 512, True), (17, 66, True)]


def _paired_cases():
    """Every shape with family 2 and 3, at the row's trip count and one past
    it where that is still at most 8 steps."""
    out = []
    for rows, units, q40 in _PAIRED_SHAPES:
        need = (units + (64 if q40 else 8) - 1) // (64 if q40 else 8)
        for extra in (0, 1):
            if need + extra <= 8:
                out += [(rows, units, q40, fam, extra) for fam in (2, 3)]
    return out


@pytest.mark.parametrize("rows,units,q40,fam,nit_extra", _paired_cases())
def test_paired_one_pass_kernels(ctx, axc, rows, units, q40, fam, nit_extra):
    """One workgroup per 8 output rows, gate rows on the even wave of a pair
    and up rows on the odd one, x chunk by chunk (family 2) or whole (3), the
    row's trip count and one past it: odd row counts (a pair with one row),
    partial last workgroups and octets, the longest rows (8 steps), against
    the f64 oracle and, for the Q4_K kernels, within 4 ulp of two one-pass
    matvecs with the same trip count."""
    per = 64 if q40 else 8
    nit = (units + per - 1) // per + nit_extra
    v = axc.Variant(family=fam, sb_per_lane=nit)
    name = (axc.q4_0_gate_up_kernel_name if q40 else axc.q4k_gate_up_kernel_name)(rows, units, v)
    assert name == f"axh_{'q4_0' if q40 else 'q4k'}_gate_up_one{'x' if fam == 3 else ''}_i{nit}"
    _say(f"paired gate_up {rows}x{units} {name}")
    if q40:
        qg, qu, x = _inputs0(rows * 11 + units, rows, units)
        h = _gate_up0(ctx, qg, qu, x, rows, units, v)
        _check0(h, qg, qu, x, rows, units, f"paired {name} {rows}x{units}")
        mv = axc.Variant(prefetch=1 if fam == 2 else 0, family=fam, sb_per_lane=nit)
        g = _matvec0(ctx, qg, x, rows, units, mv)
        u = _matvec0(ctx, qu, x, rows, units, mv)
    else:
        qg, qu, x = _inputs(rows * 11 + units, rows, units)
        h = _gate_up(ctx, qg, qu, x, rows, units, v)
        _check(h, qg, qu, x, rows, units, f"paired {name} {rows}x{units}")
        mv = axc.Variant(prefetch=1 if fam == 2 else 0, family=fam, sb_per_lane=nit)
        g = _matvec(ctx, qg, x, rows, units, mv)
        u = _matvec(ctx, qu, x, rows, units, mv)
    want = O.silu(g.astype(np.float64)) * u.astype(np.float64)
    assert np.all(np.abs(h - want) <= 4 * 2.0 ** -24 * np.abs(want) + 1e-30), name


# ---- the fusion over two Q5_K matrices (one-pass kernels only) -------------------
Q5 = O.GGML_Q5_K


def _gate_up5(ctx, qg, qu, x, rows, sb, variant=None):
    dg, du, dx, dh = _dev(ctx, qg), _dev(ctx, qu), _dev(ctx, x), ctx.alloc(rows * 4)
    ctx.q5k_gate_up(dg, du, dx, dh, rows, sb, variant)
    ctx.synchronize()
    h = np.frombuffer(ctx.download(dh, rows * 4), dtype=np.float32).copy()
    for b in (dg, du, dx, dh):
        b.close()
    return h


def _matvec5(ctx, q, x, rows, sb, variant=None):
    dq, dx, dy = _dev(ctx, q), _dev(ctx, x), ctx.alloc(rows * 4)
    ctx.q5k_matvec(dq, dx, dy, rows, sb, variant)
    ctx.synchronize()
    y = np.frombuffer(ctx.download(dy, rows * 4), dtype=np.float32).copy()
    for b in (dq, dx, dy):
        b.close()
    return y


@pytest.mark.parametrize("rows,sb,fam,nit", [(12288, 16, 0, 2), (1, 1, 0, 1), (7, 3, 2, 1),
                                             (1531, 24, 3, 3), (33, 64, 2, 8), (2049, 17, 3, 4),
                                             (100, 40, 2, 5), (4097, 8, 3, 1)])
def test_q5k_gate_up(ctx, axc, rows, sb, fam, nit):
    """Q5_K gate/up through the one-pass kernels (family 0 = the default)
    against the f64 oracle, and within 4 ulp of silu(g) * u of two Q5_K
    one-pass matvecs with the same trip count (the same per-row
    arithmetic)."""
    qg = O.gen_kq_weights(Q5, rows * 5 + sb, rows * sb)
    qu = O.gen_kq_weights(Q5, rows * 5 + sb + 1, rows * sb)
    x = O.gen_normal_f32(rows + 3 * sb, sb * 256, 0.5)
    v = axc.Variant(family=fam, sb_per_lane=nit) if fam else None
    name = axc.q5k_gate_up_kernel_name(rows, sb, v)
    _say(f"q5k gate_up {rows}x{sb} {name}")
    h = _gate_up5(ctx, qg, qu, x, rows, sb, v)
    _, g, ag, u, au = O.kq_gate_up_f64(Q5, qg, qu, x, rows, sb)
    rep = O.gate_up_tolerance_report(h, g, ag, u, au, sb * 256, REL_TOL)
    _say(f"q5k gate_up {rows}x{sb}: {rep}")
    assert rep["ok"], rep
    ffam = fam or (axc.FAMILY_ONE_PASS_X if "onex" in name else axc.FAMILY_ONE_PASS)
    mv = axc.Variant(prefetch=1 if ffam == 2 else 0, family=axc.FAMILY_ONE_PASS,
                     sb_per_lane=int(name.rsplit("_i", 1)[1]))
    gm = _matvec5(ctx, qg, x, rows, sb, mv)
    um = _matvec5(ctx, qu, x, rows, sb, mv)
    want = O.silu(gm.astype(np.float64)) * um.astype(np.float64)
    assert np.all(np.abs(h - want) <= 4 * 2.0 ** -24 * np.abs(want) + 1e-30), name


@pytest.mark.parametrize("rows,sb,holes", [(12289, 16, None), (1531, 24, (1, 4, 1)),
                                           (1531, 24, (1, 8, 1)), (1531, 24, (1, 4, 2)),
                                           (333, 64, (1, 4, 2)), (257, 100, None),
                                           (20011, 9, (1, 4, 1))])
def test_q5k_gate_up_persistent(ctx, axc, rows, sb, holes):
    """The persistent Q5_K gate/up (the default past 12288 rows or 64
    superblocks; every compiled variant): x whole in one and two staged
    sub-blocks per thread, early refill, more rows than the grid holds,
    against the f64 oracle."""
    v = axc.Variant(*holes, 0) if holes else None
    name = axc.q5k_gate_up_kernel_name(rows, sb, v)
    assert name.startswith("axh_q5k_gate_up_r"), name
    _say(f"q5k gate_up persistent {rows}x{sb} {name}")
    qg = O.gen_kq_weights(Q5, rows * 7 + sb, rows * sb)
    qu = O.gen_kq_weights(Q5, rows * 7 + sb + 1, rows * sb)
    x = O.gen_normal_f32(rows + 5 * sb, sb * 256, 0.5)
    h = _gate_up5(ctx, qg, qu, x, rows, sb, v)
    _, g, ag, u, au = O.kq_gate_up_f64(Q5, qg, qu, x, rows, sb)
    rep = O.gate_up_tolerance_report(h, g, ag, u, au, sb * 256, REL_TOL)
    _say(f"q5k gate_up persistent {rows}x{sb}: {rep}")
    assert rep["ok"], rep
