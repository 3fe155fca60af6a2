"""Performance regression gates on ratios measured on the same box in the same
run (marked `gpu`), so that they do not depend on which MI355X runs them: the
north-star Q4_K_M matvec against a pure read of the same bytes, and the
batched matmul's 32x32 tile kind against the K-split tile kind, the next
fastest at that shape.

Each side is timed by the library's own launch loop (axh_bench_loop) over
weight copies rotated through more than the 256 MiB Infinity Cache, in
interleaved rounds, and the gate (tests/perf_gate.py) compares medians.  The
thresholds sit below the measured ratios (matvec / read 0.80-0.86; K-split
tile / 32x32 1.41) by the run-to-run spread of these boxes.  Each gate also
runs on a positive control, a kernel known to be slower, which it must
reject: the GPU counterpart of the reference's planted slowdown
(crates/axc-driver/tests/bench_regression.rs:185-195).
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import perf_gate as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ROUNDS, CALLS = 5, 100
NORTH_STAR_MIN = 0.76   # read / matvec
WIDE_MATMUL_MIN = 0.97  # K-split tiles / default


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _rotated(ctx, q: np.ndarray, min_total: int = 600 << 20):
    """Device copies of q, 256-byte aligned, more than min_total bytes in all."""
    stride = (q.nbytes + 255) // 256 * 256
    n = max(2, -(-min_total // stride))
    buf = ctx.alloc(stride * n)
    for c in range(n):
        ctx.upload(buf.ptr + c * stride, q)
    return buf, stride, n


@pytest.fixture(scope="module")
def north_star(ctx, axc):
    rows, sb = 4096, 56
    q = O.gen_q4k_weights(31, rows * sb)
    x = O.gen_normal_f32(32, sb * 256)
    wbuf, stride, n = _rotated(ctx, q)
    dx, dy = ctx.alloc(x.nbytes), ctx.alloc(rows * 4)
    ctx.upload(dx, x)
    words = 8 * ctx.cu_count()
    dout = ctx.alloc(words * 4)
    mv = dict(op="q4k", q=wbuf, q_stride=stride, n_copies=n, x=dx, y=dy, n_rows=rows, units=sb)
    ops = {
        "matvec": mv,
        "read": dict(op="read_floor", q=wbuf, q_stride=stride, n_copies=n, x=None, y=dout,
                     units=q.nbytes // 16, batch=words),
        # positive control: the persistent kernel with 7 iterations in flight
        # and non-temporal weight loads (0.50 of the read in one run)
        "slow": dict(mv, variant=axc.Variant(1, 8, 7, 1, axc.FAMILY_PERSISTENT)),
    }
    yield rows, sb, ops
    for b in (wbuf, dx, dy, dout):
        b.close()


def test_north_star_matvec_against_the_read_floor(ctx, axc, north_star):
    """4096 x 14336 Q4_K_M: the matvec's time per call within 1 / 0.76 of a
    read of the same bytes by a kernel of its launch shape."""
    rows, sb, ops = north_star
    _say(f"perf gate: q4k matvec {rows}x{sb * 256} vs read floor")
    r = G.gate_from_rounds(G.bench_loop_measure(ctx, ops, CALLS), "read", "matvec",
                           NORTH_STAR_MIN, ROUNDS)
    _say(f"  matvec {r.candidate_us:.3f} us, read {r.floor_us:.3f} us, ratio {r.ratio:.4f} "
         f"({axc.q4k_matvec_kernel_name(rows, sb)})")
    assert r.ok, r


def test_north_star_gate_rejects_a_slower_kernel(ctx, axc, north_star):
    """The same gate on the positive control fails."""
    rows, sb, ops = north_star
    name = axc.q4k_matvec_kernel_name(rows, sb, ops["slow"]["variant"])
    _say(f"perf gate positive control: {name} vs read floor")
    r = G.gate_from_rounds(G.bench_loop_measure(ctx, ops, CALLS), "read", "slow",
                           NORTH_STAR_MIN, ROUNDS)
    _say(f"  {name} {r.candidate_us:.3f} us, read {r.floor_us:.3f} us, ratio {r.ratio:.4f}")
    assert not r.ok, r


@pytest.fixture(scope="module")
def wide_matmul(ctx, axc):
    rows, sb, batch = 14336, 16, 512
    q = O.gen_q4k_weights(33, rows * sb)
    xh = np.random.default_rng(34).standard_normal(batch * sb * 256).astype(np.float16)
    wbuf, stride, n = _rotated(ctx, q)
    dx, dy = ctx.alloc(xh.nbytes), ctx.alloc(rows * batch * 4)
    ctx.upload(dx, xh)
    base = dict(op="matmul_f16", q=wbuf, q_stride=stride, n_copies=n, x=dx, y=dy, n_rows=rows,
                units=sb, batch=batch)
    ops = {"default": base, "k_split": dict(base, variant=axc.MatmulVariant(5, 4, 8, 2, 4)),
           # positive control: the K-split kind (3) at 512 columns
           "slow": dict(base, variant=axc.MatmulVariant(3, 8, 1, 1, 2))}
    yield rows, sb, batch, ops
    for b in (wbuf, dx, dy):
        b.close()


def test_wide_matmul_tiles_against_the_k_split_tile_kind(ctx, axc, wide_matmul):
    """14336 x 4096 x 512: the default (32x32 tiles) at least as fast as the
    K-split tile kind with 128 columns per workgroup, within the run-to-run
    spread."""
    rows, sb, batch, ops = wide_matmul
    _say(f"perf gate: q4k matmul {rows}x{sb * 256} B={batch}, default vs K-split tiles")
    r = G.gate_from_rounds(G.bench_loop_measure(ctx, ops, CALLS), "k_split", "default",
                           WIDE_MATMUL_MIN, ROUNDS)
    _say(f"  default {r.candidate_us:.2f} us ({axc.q4k_matmul_kernel_name(rows, sb, batch)}), "
         f"K-split tiles {r.floor_us:.2f} us, ratio {r.ratio:.3f}")
    assert r.ok, r


def test_wide_matmul_gate_rejects_a_slower_kernel(ctx, axc, wide_matmul):
    """The same gate with a slower kind in the default's place fails."""
    rows, sb, batch, ops = wide_matmul
    name = axc.q4k_matmul_kernel_name(rows, sb, batch, ops["slow"]["variant"])
    _say(f"perf gate positive control: {name} vs K-split tiles")
    r = G.gate_from_rounds(G.bench_loop_measure(ctx, ops, CALLS), "k_split", "slow",
                           WIDE_MATMUL_MIN, ROUNDS)
    _say(f"  {name} {r.candidate_us:.2f} us, K-split tiles {r.floor_us:.2f} us, "
         f"ratio {r.ratio:.3f}")
    assert not r.ok, r
