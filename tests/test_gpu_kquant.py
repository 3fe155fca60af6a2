"""Q5_K / Q6_K on the GPU (marked `gpu`) and GGUF tensors end to end.

The reference has no Q5_K / Q6_K code; the oracle is the CPU restatement of
ggml's dequantisation (oracle/kq_oracle.c, pinned in test_oracle_pins.py).
Bars: decode bit-exact; matvec under the row-wise tolerance criterion of
oracle.matvec_tolerance_report (1e-3 relative per well-conditioned row,
condition-scaled bound on cancelling rows, 1e-3 norm-wise).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3
GOLDEN = Path(__file__).resolve().parent / "golden"
Q5, Q6 = O.GGML_Q5_K, O.GGML_Q6_K


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _dev(ctx, arr):
    b = ctx.alloc(max(arr.nbytes, 16))
    ctx.upload(b, arr)
    return b


def _matvec(ctx, kind, q, x, rows, sb, variant=None):
    dq, dx, dy = _dev(ctx, q), _dev(ctx, x), ctx.alloc(rows * 4)
    fn = ctx.q5k_matvec if kind == Q5 else ctx.q6k_matvec
    fn(dq, dx, dy, rows, sb, variant)
    ctx.synchronize()
    y = np.frombuffer(ctx.download(dy, rows * 4), dtype=np.float32).copy()
    for b in (dq, dx, dy):
        b.close()
    return y


def _check(y, kind, q, x, rows, sb, what):
    ref = O.kq_matvec(kind, q, x, rows, sb)
    yf, ad = O.kq_matvec_f64(kind, q, x, rows, sb)
    rep = O.matvec_tolerance_report(y, ref, yf, ad, sb * 256, REL_TOL)
    _say(f"{what}: {rep}")
    assert rep["ok"], f"{what}: {rep}"


@pytest.mark.parametrize("kind", [Q5, Q6])
def test_dequant_bit_exact(ctx, kind):
    n = 4099
    q = O.gen_kq_weights(kind, 900 + kind, n)
    nb = O.KQ_SB_BYTES[kind]
    blocks = q.reshape(-1, nb)
    d_off = 208 if kind == Q6 else 0
    blocks[0, d_off:d_off + 2] = np.array([0x0001], np.uint16).view(np.uint8)  # subnormal d
    blocks[1, d_off:d_off + 2] = np.array([0x7BFF], np.uint16).view(np.uint8)  # 65504
    _say(f"dequant kind {kind}")
    dq, dw = _dev(ctx, q), ctx.alloc(n * 256 * 4)
    (ctx.q5k_dequant if kind == Q5 else ctx.q6k_dequant)(dq, dw, n)
    ctx.synchronize()
    w = np.frombuffer(ctx.download(dw, n * 256 * 4), dtype=np.float32)
    dq.close()
    dw.close()
    ref = O.kq_dequant(kind, q, n)
    assert np.array_equal(w.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("kind,rows,sb,sigma", [
    (Q6, 128256, 16, 1.0),   # Llama-3-8B output head (Q6_K in Q4_K_M files)
    (Q6, 4096, 56, 0.5),     # ffn_down (Q6_K in half the layers of Q4_K_M files)
    (Q5, 14336, 16, 1.0),    # ffn_gate / ffn_up of Q5_K_M files
    (Q5, 4096, 56, 0.5),
])
def test_model_shapes(ctx, kind, rows, sb, sigma):
    _say(f"kquant {kind} {rows}x{sb * 256}")
    q = O.gen_kq_weights(kind, rows + sb + kind, rows * sb)
    x = O.gen_normal_f32(rows + 1, sb * 256, sigma)
    y = _matvec(ctx, kind, q, x, rows, sb)
    _check(y, kind, q, x, rows, sb, f"kind {kind} {rows}x{sb * 256}")


@pytest.mark.parametrize("kind", [Q5, Q6])
@pytest.mark.parametrize("rows,sb", [(1, 1), (2, 1), (3, 5), (31, 128), (257, 16), (1000, 64),
                                     (100, 100), (4097, 8), (64, 33), (7, 3)])
def test_edge_shapes(ctx, kind, rows, sb):
    """Odd rows and odd superblock counts (Q6_K superblocks then start at
    both 4-byte residues), one superblock, the longest staged row."""
    _say(f"kquant edge {kind} {rows}x{sb}")
    q = O.gen_kq_weights(kind, rows * 3 + sb, rows * sb)
    x = O.gen_normal_f32(rows + sb, sb * 256)
    y = _matvec(ctx, kind, q, x, rows, sb)
    _check(y, kind, q, x, rows, sb, f"edge {kind} {rows}x{sb}")


@pytest.mark.parametrize("kind", [Q5, Q6])
def test_every_variant(ctx, axc, kind):
    rows, sb = 1531, 24
    q = O.gen_kq_weights(kind, 77, rows * sb)
    x = O.gen_normal_f32(78, sb * 256)
    for v in axc.compiled_variants("q5k" if kind == Q5 else "q6k"):
        _say(f"kquant {kind} variant {v}")
        y = _matvec(ctx, kind, q, x, rows, sb, v)
        _check(y, kind, q, x, rows, sb, f"variant {v}")


@pytest.mark.parametrize("kind", [Q5, Q6])
def test_early_refill_several_pairs_per_wave(ctx, axc, kind):
    """Prefetch-1 variants with more rows than the persistent grid holds."""
    rows, sb = 20011, 9
    q = O.gen_kq_weights(kind, 79, rows * sb)
    x = O.gen_normal_f32(80, sb * 256)
    vs = [v for v in axc.compiled_variants("q5k" if kind == Q5 else "q6k") if v.prefetch == 1]
    assert vs
    for v in vs:
        _say(f"kquant {kind} early refill {v}")
        y = _matvec(ctx, kind, q, x, rows, sb, v)
        _check(y, kind, q, x, rows, sb, f"early refill {v}")


def _flat_for(axc, sb):
    """A persistent variant that stages a row of `sb` superblocks."""
    return axc.Variant(1, 4, 1, 0) if sb <= 32 else axc.Variant(1, 8, 1, 0)


@pytest.mark.parametrize("rows,sb,nit,xd", [(1, 1, 1, 1), (7, 3, 1, 1), (33, 8, 2, 1),
                                            (17, 9, 2, 1), (4097, 16, 2, 1), (2048, 8, 1, 1),
                                            (100, 16, 2, 1), (4096, 56, 7, 1), (2049, 17, 3, 1),
                                            (33, 64, 8, 1), (50, 40, 5, 2), (4095, 56, 7, 2),
                                            (9, 24, 4, 2)])
def test_q5k_one_pass_family(ctx, axc, rows, sb, nit, xd):
    """The Q5_K one-pass kernel (the default for 768-32768 rows of up to 16
    superblocks and 2049-4096 rows of up to 64) at ragged row counts, trip
    counts 1-8 (one past the row's too), x one or two chunks ahead, requested
    explicitly: within the oracle's tolerance, and bit for bit the persistent
    kernel's output (the same per-lane loads, decode and reduction order)."""
    q = O.gen_kq_weights(Q5, rows * 5 + sb, rows * sb)
    x = O.gen_normal_f32(rows + 2 * sb, sb * 256)
    v = axc.Variant(0, 0, xd, 0, axc.FAMILY_ONE_PASS, nit)
    _say(f"kquant Q5_K one-pass {rows}x{sb} i{nit} x{xd}")
    y = _matvec(ctx, Q5, q, x, rows, sb, v)
    _check(y, Q5, q, x, rows, sb, f"one-pass {rows}x{sb} i{nit} x{xd}")
    flat = _matvec(ctx, Q5, q, x, rows, sb, _flat_for(axc, sb))
    assert np.array_equal(y.view(np.uint32), flat.view(np.uint32))


@pytest.mark.parametrize("rows,sb,nit,xd", [(1, 1, 1, 1), (7, 3, 1, 1), (33, 8, 2, 1),
                                            (17, 9, 2, 1), (4097, 16, 2, 1), (1024, 16, 2, 1),
                                            (100, 16, 2, 1), (256, 8, 1, 1), (4096, 40, 5, 1),
                                            (8192, 24, 3, 1), (2049, 17, 3, 1), (33, 64, 8, 1),
                                            (50, 56, 7, 2), (4095, 24, 3, 2), (9, 33, 6, 2)])
def test_q6k_one_pass_family(ctx, axc, rows, sb, nit, xd):
    """The Q6_K one-pass kernel (the default for 256-4096 rows of up to 16
    superblocks and 2049-8192 rows of up to 40) at ragged row counts, trip
    counts 1-8, x one or two chunks ahead, requested explicitly: within the
    oracle's tolerance, and bit for bit the persistent kernel's output (the
    same per-lane loads, decode and reduction order)."""
    q = O.gen_kq_weights(Q6, rows * 7 + sb, rows * sb)
    x = O.gen_normal_f32(rows + 3 * sb, sb * 256)
    v = axc.Variant(0, 0, xd, 0, axc.FAMILY_ONE_PASS, nit)
    _say(f"kquant Q6_K one-pass {rows}x{sb} i{nit} x{xd}")
    y = _matvec(ctx, Q6, q, x, rows, sb, v)
    _check(y, Q6, q, x, rows, sb, f"one-pass {rows}x{sb} i{nit} x{xd}")
    flat = _matvec(ctx, Q6, q, x, rows, sb, _flat_for(axc, sb))
    assert np.array_equal(y.view(np.uint32), flat.view(np.uint32))


@pytest.mark.parametrize("kind,rows,sb,kernel", [
    (Q5, 1024, 56, "flat_r1_w4_p2_x2"), (Q5, 14336, 40, "flat_r1_w4_p2_x2"),
    (Q5, 4096, 40, "one_i5"), (Q6, 2048, 24, "flat_r1_w4_p2_x1"),
    (Q6, 14336, 56, "flat_r1_w4_p2_x2"), (Q6, 8192, 40, "one_i5")])
def test_kquant_defaults_by_shape(ctx, axc, kind, rows, sb, kernel):
    """The Q5_K / Q6_K default of each band that takes 4 waves with x whole
    or the one-pass kernel on longer rows, against the oracle."""
    fam = "q5k" if kind == Q5 else "q6k"
    name = getattr(axc, f"{fam}_matvec_kernel_name")
    assert name(rows, sb) == f"axh_{fam}_matvec_{kernel}"
    q = O.gen_kq_weights(kind, rows + 3 * sb, rows * sb)
    x = O.gen_normal_f32(rows + 5 * sb, sb * 256)
    _say(f"kquant {fam} default {rows}x{sb} {kernel}")
    y = _matvec(ctx, kind, q, x, rows, sb)
    _check(y, kind, q, x, rows, sb, f"{fam} default {rows}x{sb}")


def test_one_hot_x_reads_single_weights(ctx):
    """x = e_k picks column k: y = W[:, k] exactly (exact products, one term;
    compared as values: a zero Q6_K weight with a negative scale is -0.0 in
    the oracle and +0.0 after the kernel's accumulation)."""
    rows, sb = 64, 2
    for kind in (Q5, Q6):
        q = O.gen_kq_weights(kind, 79, rows * sb)
        w = O.kq_dequant(kind, q, rows * sb).reshape(rows, sb * 256)
        for k in (0, 17, 100, 255, 256, 300, 511):
            x = np.zeros(sb * 256, np.float32)
            x[k] = 1.0
            y = _matvec(ctx, kind, q, x, rows, sb)
            assert np.array_equal(y, w[:, k]), (kind, k)


def test_gguf_fixture_tensors_through_matvec_ggml(ctx, axc):
    """The fixture's Q4_K, Q5_K and Q6_K tensors, uploaded by the native
    reader, through the type-dispatching matvec, against the oracles."""
    from importlib import import_module

    gg = import_module(axc.__name__ + ".gguf")
    with gg.GgufFile(GOLDEN / "tiny_v3.gguf") as f:
        for name, t in f.tensors.items():
            if t.type not in (gg.GGML_Q4_K, gg.GGML_Q5_K, gg.GGML_Q6_K):
                continue
            _say(f"gguf tensor {name}")
            buf = f.upload(ctx, name)
            x = O.gen_normal_f32(len(name), t.n_cols)
            dx, dy = _dev(ctx, x), ctx.alloc(t.n_rows * 4)
            ctx.matvec_ggml(t.type, buf, dx, dy, t.n_rows, t.n_cols)
            ctx.synchronize()
            y = np.frombuffer(ctx.download(dy, t.n_rows * 4), dtype=np.float32)
            q = np.frombuffer(f.tensor_bytes(name), dtype=np.uint8)
            sb = t.n_cols // 256
            if t.type == gg.GGML_Q4_K:
                ref = O.q4k_matvec(q, x, t.n_rows, sb)
                yf, ad = O.q4k_matvec_f64(q, x, t.n_rows, sb)
            else:
                ref = O.kq_matvec(t.type, q, x, t.n_rows, sb)
                yf, ad = O.kq_matvec_f64(t.type, q, x, t.n_rows, sb)
            rep = O.matvec_tolerance_report(y, ref, yf, ad, t.n_cols, REL_TOL)
            assert rep["ok"], (name, rep)
            for b in (buf, dx, dy):
                b.close()


def test_invalid_arguments_are_typed_errors(ctx, axc):
    b = ctx.alloc(1 << 20)
    for fn in (ctx.q5k_matvec, ctx.q6k_matvec):
        with pytest.raises(axc.DispatchError):
            fn(b, b, b, 4, 0)
        with pytest.raises(axc.DispatchError):
            fn(b, b, b, 4, 129)
        fn(b, b, b, 0, 1)  # empty
    with pytest.raises(axc.DispatchError):
        ctx.matvec_ggml(O.GGML_Q6_K, b, b, b, 4, 300)  # not a whole number of superblocks
    with pytest.raises(axc.DispatchError):
        ctx.matvec_ggml(3, b, b, b, 4, 256)  # Q4_1: no matvec kernel
    b.close()
