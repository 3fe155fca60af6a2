"""The allocation-free matvec entry point (axh_q4k_matvec_noalloc) against
axh_q4k_matvec, through the C ABI (marked `gpu`).

Both run the split-K kernel on these shapes (fewer than 32 rows of 64-256
superblocks), so their outputs must agree bit for bit; both are also held to
the oracle's matvec tolerance.  Two calls in a row, the second smaller, share
the device's scratch array: the second must not see the first's partial sums
or counter.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _dev(ctx, arr):
    b = ctx.alloc(arr.nbytes)
    ctx.upload(b, arr)
    return b


def _both(ctx, axc, rows, sb, seed):
    q = O.gen_q4k_weights(seed, rows * sb)
    x = O.gen_normal_f32(seed + 1, sb * 256)
    dq, dx = _dev(ctx, q), _dev(ctx, x)
    y0, y1 = ctx.alloc(rows * 4), ctx.alloc(rows * 4)
    ctx.upload(y1, np.full(rows, np.nan, dtype=np.float32))
    ctx.q4k_matvec(dq, dx, y0, rows, sb)
    ctx.q4k_matvec_noalloc(dq, dx, y1, rows, sb)
    ctx.synchronize()
    a = np.frombuffer(ctx.download(y0, rows * 4), dtype=np.float32).copy()
    b = np.frombuffer(ctx.download(y1, rows * 4), dtype=np.float32).copy()
    for buf in (dq, dx, y0, y1):
        buf.close()
    return q, x, a, b


def test_noalloc_matches_the_allocating_entry_point_twice(ctx, axc):
    for rows, sb, seed in ((31, 200, 501), (5, 150, 502)):  # second call smaller
        assert axc.q4k_matvec_kernel_name(rows, sb).startswith("axh_q4k_matvec_sk_")
        _say(f"noalloc vs q4k_matvec {rows}x{sb}")
        q, x, a, b = _both(ctx, axc, rows, sb, seed)
        assert a.tobytes() == b.tobytes(), f"{rows}x{sb}: outputs differ"
        ref = O.q4k_matvec(q, x, rows, sb)
        yf, ad = O.q4k_matvec_f64(q, x, rows, sb)
        rep = O.matvec_tolerance_report(b, ref, yf, ad, sb * 256)
        assert rep["ok"], rep


def test_noalloc_shapes_outside_the_split_k_default(ctx, axc):
    """Shapes where axh_q4k_matvec picks another kernel: the same function,
    held to the oracle's tolerance (the summation order differs)."""
    for rows, sb, seed in ((32, 256, 511), (1, 1, 512), (3, 17, 513), (2, 64, 514)):
        _say(f"noalloc {rows}x{sb} vs oracle")
        q, x, a, b = _both(ctx, axc, rows, sb, seed)
        ref = O.q4k_matvec(q, x, rows, sb)
        yf, ad = O.q4k_matvec_f64(q, x, rows, sb)
        for y in (a, b):
            rep = O.matvec_tolerance_report(y, ref, yf, ad, sb * 256)
            assert rep["ok"], rep


def test_noalloc_rejects_sizes_beyond_its_scratch(ctx, axc):
    buf = ctx.alloc(1 << 16)
    for rows, sb in ((33, 16), (4, 257), (4, 0)):
        with pytest.raises(axc.DispatchError) as e:
            ctx.q4k_matvec_noalloc(buf, buf, buf, rows, sb)
        assert e.value.variant == "InvalidArgument"
    ctx.q4k_matvec_noalloc(buf, buf, buf, 0, 16)  # no rows: nothing to do
    buf.close()
