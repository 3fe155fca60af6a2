"""Tuning tools on the device (marked `gpu`): bench_variant returns timings
with a real correctness verdict for every Q4 kernel, grid_search ranks the
compiled hole space and appends one history line (reference:
crates/axc-driver/src/mcp/tools/bench_variant.rs:209-282,
grid_search.rs:256-410)."""
from __future__ import annotations

import importlib
import io
import json
import sys

import pytest

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def mcp(axc):
    return importlib.import_module("axiom_compute_amd.mcp")


@pytest.mark.parametrize("kernel,shape", [
    ("q4km_dequant_matvec", {"n_rows": 512, "units_per_row": 16}),
    ("q4_0_dequant_matvec", {"n_rows": 256, "units_per_row": 128}),
    ("q4k_matmul_f16", {"n_rows": 256, "units_per_row": 4, "batch": 24}),
])
def test_bench_variant_checks_every_kernel(mcp, tmp_path, kernel, shape):
    _say(f"bench_variant {kernel} {shape}")
    ctx = mcp.McpContext(history_dir=tmp_path)
    r = mcp.bench_variant({"kernel": kernel, "shape": shape, "sample_count": 3,
                           "launches_per_sample": 4}, ctx)
    assert r["correctness"] == {"status": "ok"}, r["correctness"]
    assert len(r["samples"]) == 3 and r["median_ns"] > 0
    assert r["machine"]["device_name"]
    assert r["kernel_entry"].startswith("axh_q4")


def test_bench_variant_uncompiled_assignment_is_an_error(mcp, tmp_path):
    ctx = mcp.McpContext(history_dir=tmp_path)
    with pytest.raises(mcp.McpToolError) as e:
        mcp.bench_variant({"kernel": "q4km_dequant_matvec",
                           "shape": {"n_rows": 64, "units_per_row": 4}, "sample_count": 1,
                           "assignments": {"rows_per_wave": 3}}, ctx)
    assert e.value.code == mcp.DEVICE_UNAVAILABLE and e.value.category == "dispatch_failed"


def test_q4_0_grid_search_over_every_family(mcp, tmp_path, axc):
    """grid_search over the Q4_0 families that take 2048 x 128 blocks: every
    assignment that names a compiled kernel runs and passes the host checker,
    the rest fail to plan and rank last."""
    _say("grid_search q4_0 2048x128 every family")
    ctx = mcp.McpContext(history_dir=tmp_path)
    shape = {"n_rows": 2048, "units_per_row": 128}
    res = mcp.grid_search({"kernel": "q4_0_dequant_matvec", "shape": shape,
                           "sample_count": 2}, ctx)
    ranked = res["ranked"]
    ok = [r for r in ranked if r["outcome"] == "ok"]
    assert ok and all(r["median_ns"] for r in ok)
    fams = {int(r["assignments"].get("family", 0)) for r in ok}
    assert fams == {0, axc.FAMILY_PERSISTENT, axc.FAMILY_ONE_PASS, axc.FAMILY_ONE_PASS_X,
                    axc.FAMILY_COLUMNS}, fams
    assert not [r for r in ranked if r["outcome"].startswith("correctness_rejected")]
    assert all(r["median_ns"] is None for r in ranked[len(ok):])


def test_grid_search_over_the_stdio_server(mcp, tmp_path):
    """Two JSON-RPC calls through serve(): a grid search (some assignments are
    not compiled and rank last as failures) and the history it appended."""
    ctx = mcp.McpContext(history_dir=tmp_path)
    shape = {"n_rows": 1024, "units_per_row": 16}
    reqs = [
        {"jsonrpc": "2.0", "id": 1, "method": "grid_search",
         "params": {"kernel": "q4km_dequant_matvec", "shape": shape, "sample_count": 2,
                    "holes_override": {"rows_per_wave": [1, 2, 3], "waves_per_workgroup": [4, 8],
                                       "prefetch": [2], "nontemporal": [2]}}},
        {"jsonrpc": "2.0", "id": 2, "method": "optimization_history",
         "params": {"kernel": "q4km_dequant_matvec", "shape": shape}},
    ]
    out = io.StringIO()
    mcp.serve(io.StringIO("\n".join(json.dumps(r) for r in reqs) + "\n"), out, ctx)
    r1, r2 = [json.loads(ln) for ln in out.getvalue().splitlines()]
    res = r1["result"]
    assert len(res["ranked"]) == 6 and not res["fallback_used"]
    ok = [r for r in res["ranked"] if r["median_ns"] is not None]
    assert [r["median_ns"] for r in ok] == sorted(r["median_ns"] for r in ok)
    assert all(r["outcome"] == "ok" for r in ok)
    failed = [r for r in res["ranked"] if r["median_ns"] is None]
    assert failed and all(r["assignments"]["rows_per_wave"] == 3 for r in failed)
    assert res["ranked"][-1]["median_ns"] is None  # failures rank last
    assert res["winner"]["variant_id"] == ok[0]["variant_id"]
    entries = r2["result"]["entries"]
    assert len(entries) == 1
    assert entries[0]["grid_search"]["winner_variant_id"] == res["winner"]["variant_id"]
    assert entries[0]["source_xxh3"] == r2["result"]["history_path"].split("/")[-1][:16]


def test_grid_search_over_the_default_space_at_c4(mcp, axc, tmp_path):
    """4096 x 14336 over the tool's default hole space
    (every family the autotuner searches): the default kernel is among the
    accepted variants, and the winner, timed again against the default on
    rotated copies in interleaved rounds, is no slower than it beyond the
    run-to-run spread (grid_search.rs:265-276 searches the kernel's own
    holes)."""
    rows, sb = 4096, 56
    shape = {"n_rows": rows, "units_per_row": sb}
    _say(f"grid_search q4km_dequant_matvec {shape} over the default space")
    ctx = mcp.McpContext(history_dir=tmp_path)
    res = mcp.grid_search({"kernel": "q4km_dequant_matvec", "shape": shape, "sample_count": 5,
                           "launches_per_sample": 20}, ctx)
    assert not res["fallback_used"] and res["weight_copies"] >= 9
    dflt = axc.q4k_matvec_kernel_name(rows, sb)
    ok = [r for r in res["ranked"] if r["median_ns"] is not None]
    assert all(r["correctness"]["status"] == "ok" for r in ok)
    assert dflt in {r["kernel_entry"] for r in ok}
    win = res["winner"]
    _say(f"  winner {win['kernel_entry']} {res['winner_median_ns']} ns "
         f"({len(ok)} of {len(res['ranked'])} variants timed); default {dflt}")
    if win["kernel_entry"] == dflt:
        return  # the search returned the default kernel itself: nothing to re-time
    # another kernel won: re-time it against the default
    import numpy as np
    from oracle import oracle as O
    hip = ctx.hip()
    q = O.gen_q4k_weights(20241, rows * sb)
    x = O.gen_normal_f32(20242, sb * 256, 0.5)
    stride = (q.nbytes + 255) // 256 * 256
    n = -(-(600 << 20) // stride)
    wbuf = hip.alloc(stride * n)
    for c in range(n):
        hip.upload(wbuf.ptr + c * stride, q)
    dx, dy = hip.alloc(x.nbytes), hip.alloc(rows * 4)
    hip.upload(dx, x)
    base = dict(op="q4k", q=wbuf, q_stride=stride, n_copies=n, x=dx, y=dy, n_rows=rows, units=sb)
    wv = mcp._variant_obj("q4km_dequant_matvec", win["assignments"])
    t = {"winner": [], "default": []}
    order = (("winner", wv), ("default", None))
    for i in range(10):  # alternating order (ABBA), so neither side always runs first
        for k, v in (order if i % 2 == 0 else order[::-1]):
            t[k].append(sum(hip.bench_loop(**base, variant=v, warmup=5, groups=1,
                                           calls_per_group=50)) * 1e3 / 50)
    med = {k: sorted(v)[len(v) // 2] for k, v in t.items()}
    _say(f"  re-timed: winner {med['winner']:.3f} us, default {med['default']:.3f} us")
    for b in (wbuf, dx, dy):
        b.close()
    # the same kernel under two labels measured 4.2 % apart in one run of these
    # rounds: the margin sits above that spread
    assert med["winner"] <= 1.06 * med["default"], med
