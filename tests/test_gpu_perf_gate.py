"""Performance regression gates on ratios measured on the same box in the same
run (marked `gpu`), so that they do not depend on which MI355X runs them: the
north-star Q4_K_M matvec against a pure read of the same bytes, and the
batched matmul's 32x32 tile kind against the K-split tile kind, the next
fastest at that shape.

Each side is timed by the library's own launch loop (axh_bench_loop) over
weight copies rotated through more than the 256 MiB Infinity Cache, in
interleaved rounds, and the gate compares medians.  The thresholds sit below
the measured ratios (matvec / read 0.80-0.86; K-split tile / 32x32 1.41) by
the run-to-run spread of these boxes.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

ROUNDS, CALLS = 5, 100


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


def _median_us(ctx, ops: dict) -> dict:
    rounds = {k: [] for k in ops}
    for _ in range(ROUNDS):
        for k, op in ops.items():
            ms = ctx.bench_loop(**op, warmup=20, groups=1, calls_per_group=CALLS)
            rounds[k].append(sum(ms) * 1e3 / CALLS)
    return {k: sorted(v)[len(v) // 2] for k, v in rounds.items()}


def test_north_star_matvec_against_the_read_floor(ctx, axc):
    """4096 x 14336 Q4_K_M: the matvec's time per call within 1 / 0.76 of a
    read of the same bytes by a kernel of its launch shape."""
    rows, sb = 4096, 56
    _say(f"perf gate: q4k matvec {rows}x{sb * 256} vs read floor")
    q = O.gen_q4k_weights(31, rows * sb)
    x = O.gen_normal_f32(32, sb * 256)
    wbuf, stride, n = _rotated(ctx, q)
    dx, dy = ctx.alloc(x.nbytes), ctx.alloc(rows * 4)
    ctx.upload(dx, x)
    words = 8 * ctx.cu_count()
    dout = ctx.alloc(words * 4)
    ops = {
        "matvec": dict(op="q4k", q=wbuf, q_stride=stride, n_copies=n, x=dx, y=dy, n_rows=rows,
                       units=sb),
        "read": dict(op="read_floor", q=wbuf, q_stride=stride, n_copies=n, x=None, y=dout,
                     units=q.nbytes // 16, batch=words),
    }
    med = _median_us(ctx, ops)
    ratio = med["read"] / med["matvec"]
    _say(f"  matvec {med['matvec']:.3f} us, read {med['read']:.3f} us, ratio {ratio:.4f} "
         f"({axc.q4k_matvec_kernel_name(rows, sb)})")
    for b in (wbuf, dx, dy, dout):
        b.close()
    assert ratio >= 0.76, med


def test_wide_matmul_tiles_against_the_k_split_tile_kind(ctx, axc):
    """14336 x 4096 x 512: the default (32x32 tiles) at least as fast as the
    K-split tile kind with 128 columns per workgroup, within the run-to-run
    spread."""
    rows, sb, batch = 14336, 16, 512
    _say(f"perf gate: q4k matmul {rows}x{sb * 256} B={batch}, default vs K-split tiles")
    q = O.gen_q4k_weights(33, rows * sb)
    xh = np.random.default_rng(34).standard_normal(batch * sb * 256).astype(np.float16)
    wbuf, stride, n = _rotated(ctx, q)
    dx, dy = ctx.alloc(xh.nbytes), ctx.alloc(rows * batch * 4)
    ctx.upload(dx, xh)
    base = dict(op="matmul_f16", q=wbuf, q_stride=stride, n_copies=n, x=dx, y=dy, n_rows=rows,
                units=sb, batch=batch)
    ops = {"default": base, "k_split": dict(base, variant=axc.MatmulVariant(5, 4, 8, 2, 4))}
    med = _median_us(ctx, ops)
    ratio = med["k_split"] / med["default"]
    _say(f"  default {med['default']:.2f} us "
         f"({axc.q4k_matmul_kernel_name(rows, sb, batch)}), K-split tiles {med['k_split']:.2f} us, "
         f"ratio {ratio:.3f}")
    for b in (wbuf, dx, dy):
        b.close()
    assert ratio >= 0.97, med
