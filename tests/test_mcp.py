"""Tuning-tool surface (CPU): JSON-RPC envelope handling, history files,
variant ids, seeded inputs and the host correctness checker, following the
reference's MCP tests (crates/axc-driver/src/mcp/tools/grid_search.rs:
470-560 AT-1118/1119/1119b, protocol.rs:200-240, dispatch.rs)."""
from __future__ import annotations

import importlib
import json
import multiprocessing as mp
from datetime import datetime, timezone

import numpy as np
import pytest

from oracle import oracle as O


@pytest.fixture(scope="module")
def mcp(axc):
    return importlib.import_module("axiom_compute_amd.mcp")


@pytest.fixture(scope="module")
def tune(axc):
    return importlib.import_module("axiom_compute_amd.tune")


def test_rfc3339_millisecond_format(mcp):
    assert mcp.format_rfc3339_utc(datetime(1970, 1, 1, tzinfo=timezone.utc)) == \
        "1970-01-01T00:00:00.000Z"
    t = datetime(2024, 2, 29, 23, 59, 58, 987654, tzinfo=timezone.utc)
    assert mcp.format_rfc3339_utc(t) == "2024-02-29T23:59:58.987Z"
    assert len(mcp.format_rfc3339_utc()) == 24


def test_at_1118_history_path_is_xxh3_hex16(mcp, tmp_path):
    k1 = mcp.source_key("q4km_dequant_matvec", {"n_rows": 4, "units_per_row": 2})
    p1, p2 = mcp.history_path(tmp_path, k1), mcp.history_path(tmp_path, k1)
    assert p1 == p2 and p1.suffix == ".jsonl"
    assert len(p1.stem) == 16 and all(c in "0123456789abcdef" for c in p1.stem)
    assert mcp.history_path(tmp_path, mcp.source_key("q4km_dequant_matvec",
                                                     {"n_rows": 5, "units_per_row": 2})) != p1


def test_at_1119_history_append_is_line_preserving(mcp, tmp_path):
    p = tmp_path / "h.jsonl"
    mcp.append_history_entry(p, {"a": 1, "s": "x\ny"})
    mcp.append_history_entry(p, {"a": 2})
    raw = p.read_bytes()
    assert raw.count(b"\n") == 2 and b"\r" not in raw
    assert [json.loads(ln)["a"] for ln in raw.decode().splitlines()] == [1, 2]


def _writer(args):
    import importlib as il
    import sys
    sys.path.insert(0, args[2])
    import __graft_entry__ as g
    g.load_package()
    m = il.import_module("axiom_compute_amd.mcp")
    for i in range(40):
        m.append_history_entry(__import__("pathlib").Path(args[0]),
                               {"writer": args[1], "i": i, "pad": "z" * 3000})
    return 0


def test_at_1119b_concurrent_writers_do_not_interleave(mcp, tmp_path):
    import os
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    p = str(tmp_path / "c.jsonl")
    with mp.get_context("spawn").Pool(4) as pool:
        pool.map(_writer, [(p, w, root) for w in range(4)])
    lines = open(p).read().splitlines()
    assert len(lines) == 160
    recs = [json.loads(ln) for ln in lines]
    for w in range(4):
        assert [r["i"] for r in recs if r["writer"] == w] == list(range(40))


def test_variant_id_matches_the_enumerator(mcp, tune):
    spaces = mcp.default_holes("q4km_dequant_matvec", {"n_rows": 4096, "units_per_row": 56})
    assert len(spaces) >= 3
    for holes in spaces:
        assert "family" in holes and len(holes["family"]) == 1
        for v in tune.enumerate_strategy(holes):
            assert mcp.variant_id(v.assignments) == v.variant_id
    assert mcp.variant_id({}) == 0


def test_matvec_hole_space_is_the_autotuners_and_reaches_the_default(mcp, tune, axc):
    """The tool searches the autotuner's per-family space (every family that
    takes the shape, in family order), so the shipped default kernel of each
    shape is one of its variants (a space of the persistent family's holes
    alone cannot reach it)."""
    for rows, sb in ((4096, 56), (4096, 16), (14336, 16), (1, 128), (3, 100), (128256, 16)):
        shape = {"n_rows": rows, "units_per_row": sb}
        spaces = mcp.default_holes("q4km_dequant_matvec", shape)
        assert spaces == tune.q4k_matvec_hole_spaces(rows, sb)
        fams = [h["family"][0] for h in spaces]
        assert fams == sorted(fams) and axc.FAMILY_PERSISTENT in fams
        vs = mcp._enumerate_spaces(spaces)
        assert [v.ordinal for v in vs] == list(range(len(vs)))
        d = axc.q4k_matvec_default_variant(rows, sb)
        names = {axc.q4k_matvec_kernel_name(rows, sb, mcp._variant_obj("q4km_dequant_matvec",
                                                                         v.assignments))
                 for v in vs
                 if _plans(axc, rows, sb, mcp._variant_obj("q4km_dequant_matvec", v.assignments))}
        assert axc.q4k_matvec_kernel_name(rows, sb, d) in names, (rows, sb)
        assert axc.q4k_matvec_kernel_name(rows, sb) in names


def _plans(axc, rows, sb, v):
    try:
        axc.q4k_matvec_kernel_name(rows, sb, v)
        return True
    except axc.DispatchError:
        return False


def test_variant_objects_carry_every_hole(mcp, axc):
    v = mcp._variant_obj("q4km_dequant_matvec", {"family": 2, "prefetch": 2, "sb_per_lane": 7})
    assert v == axc.Variant(0, 0, 2, 0, 2, 7)
    assert axc.q4k_matvec_kernel_name(4096, 56, v) == "axh_q4k_matvec_onep_i7"


def test_default_hole_spaces_come_from_compiled_variants(mcp, axc):
    (h,) = mcp.default_holes("q4k_matmul_f16")
    assert set(h["kind"]) == {3, 5, 7, 8, 9}
    assert 0 in h["row_tiles"] and 4 in h["row_tiles"]
    assert mcp.default_holes("q4_0_dequant_matvec")[0]["waves_per_workgroup"] == [1, 4]


def test_q4_0_hole_spaces_follow_the_shape(mcp, axc):
    """With a shape, the Q4_0 space is the LDS-tiled kernel's map and one map
    per other family that takes the shape; each family's plain assignment
    plans to that family's kernel."""
    sp = mcp.default_holes("q4_0_dequant_matvec", {"n_rows": 256, "units_per_row": 128})
    assert sp[0] == mcp.default_holes("q4_0_dequant_matvec")[0]
    fams = [m["family"][0] for m in sp[1:]]
    assert fams == [axc.FAMILY_PERSISTENT, axc.FAMILY_ONE_PASS, axc.FAMILY_ONE_PASS_X,
                    axc.FAMILY_COLUMNS]
    one = sp[2]
    assert one["sb_per_lane"] == [2, 3] and one["prefetch"] == [1, 2]
    # odd block counts take only the tiled kernel; 130 blocks no column kernel
    assert len(mcp.default_holes("q4_0_dequant_matvec", {"n_rows": 64, "units_per_row": 127})) == 1
    sp = mcp.default_holes("q4_0_dequant_matvec", {"n_rows": 64, "units_per_row": 130})
    assert [m["family"][0] for m in sp[1:]] == [axc.FAMILY_PERSISTENT, axc.FAMILY_ONE_PASS,
                                                 axc.FAMILY_ONE_PASS_X]
    sp = mcp.default_holes("q4_0_dequant_matvec", {"n_rows": 64, "units_per_row": 1024})
    assert sp[2]["sb_per_lane"] == [16]
    for m in sp[1:]:
        a = {k: v[0] for k, v in m.items()}
        name = axc.q4_0_matvec_kernel_name(64, 1024, mcp._variant_obj("q4_0_dequant_matvec", a))
        assert name.startswith("axh_q4_0_matvec_" + {1: "flat", 2: "one", 3: "onex"}[a["family"]])


def test_seeded_inputs_are_deterministic_and_well_formed(mcp):
    shape = {"n_rows": 3, "units_per_row": 2}
    q1, x1 = mcp.seeded_inputs("q4km_dequant_matvec", shape, 77)
    q2, x2 = mcp.seeded_inputs("q4km_dequant_matvec", shape, 77)
    q3, _ = mcp.seeded_inputs("q4km_dequant_matvec", shape, 78)
    assert np.array_equal(q1, q2) and np.array_equal(x1, x2) and not np.array_equal(q1, q3)
    assert q1.size == 3 * 2 * 144 and x1.size == 2 * 256
    d = q1.reshape(-1, 144)[:, :2].copy().view(np.float16).astype(np.float32)
    assert np.all((d >= 0.0009) & (d <= 0.0501))
    q0, x0 = mcp.seeded_inputs("q4_0_dequant_matvec", shape, 5)
    assert q0.size == 3 * 2 * 18 and x0.size == 64
    qm, xm = mcp.seeded_inputs("q4k_matmul_f16", {**shape, "batch": 3}, 5)
    assert xm.dtype == np.float16 and xm.size == 3 * 512


def test_host_checker_agrees_with_the_oracle(mcp):
    rows, sb = 64, 8
    q = O.gen_q4k_weights(11, rows * sb)
    x = O.gen_normal_f32(12, sb * 256)
    y = O.q4k_matvec(q, x, rows, sb)
    shape = {"n_rows": rows, "units_per_row": sb}
    rep = mcp.check_result("q4km_dequant_matvec", shape, q, x, y)
    assert rep["ok"] and rep["rows_checked"] == rows and rep["norm_rel_err"] < 1e-5
    bad = y.copy()
    bad[5] *= np.float32(1.01)
    rep = mcp.check_result("q4km_dequant_matvec", shape, q, x, bad)
    assert not rep["ok"] and rep["rows_failed"] >= 1 and rep["worst_row"] == 5


def test_host_checker_q4_0_and_matmul(mcp):
    rows, nb = 32, 8
    q = O.gen_q4_0_weights(13, rows * nb)
    x = O.gen_normal_f32(14, nb * 32)
    y = O.q4_0_matvec(q, x, rows, nb)
    shape = {"n_rows": rows, "units_per_row": nb}
    assert mcp.check_result("q4_0_dequant_matvec", shape, q, x, y)["ok"]
    y2 = y.copy()
    y2[0] = -y2[0] + 1.0
    assert not mcp.check_result("q4_0_dequant_matvec", shape, q, x, y2)["ok"]
    rows, sb, batch = 16, 2, 3
    qk = O.gen_q4k_weights(15, rows * sb)
    xh = O.gen_normal_f32(16, sb * 256 * batch).astype(np.float16)
    w16 = O.q4k_dequant(qk, rows * sb).reshape(rows, -1).astype(np.float16).astype(np.float64)
    ym = (xh.astype(np.float64).reshape(batch, -1) @ w16.T).astype(np.float32)
    shape = {"n_rows": rows, "units_per_row": sb, "batch": batch}
    assert mcp.check_result("q4k_matmul_f16", shape, qk, xh, ym)["ok"]
    ym[1, 3] += 1.0
    assert not mcp.check_result("q4k_matmul_f16", shape, qk, xh, ym)["ok"]


def test_host_f16_rounding_matches_numpy_on_every_pattern(mcp):
    """The checker's RN_f16 weights: one-superblock matmul against one-hot
    activations reproduces numpy's float16 rounding of the f32 weights."""
    q = O.gen_q4k_weights(17, 1)
    w32 = O.q4k_dequant(q, 1)
    xh = np.eye(256, dtype=np.float16)
    y = w32.astype(np.float16).astype(np.float32)[None, :].repeat(1, 0).T.copy()  # 256 x 1
    shape = {"n_rows": 1, "units_per_row": 1, "batch": 256}
    assert mcp.check_result("q4k_matmul_f16", shape, q, xh, y.reshape(256, 1))["ok"]
    y2 = w32[:, None].copy()  # f32 weights, not rounded: must differ somewhere
    rep = mcp.check_result("q4k_matmul_f16", shape, q, xh, y2, rel_tol=1e-7)
    assert not rep["ok"]


def test_jsonrpc_envelopes(mcp, tmp_path):
    ctx = mcp.McpContext(history_dir=tmp_path)
    r = mcp.handle_line("{not json", ctx)
    assert r["error"]["code"] == mcp.PARSE_ERROR and r["id"] is None
    r = mcp.handle_line(json.dumps({"jsonrpc": "2.0", "id": 3, "method": "nope"}), ctx)
    assert r["error"]["code"] == mcp.METHOD_NOT_FOUND and r["id"] == 3
    assert "bench_variant" in r["error"]["data"]["available"]
    assert mcp.handle_line(json.dumps({"jsonrpc": "2.0", "method": "initialize"}), ctx) is None
    r = mcp.handle_line(json.dumps({"jsonrpc": "2.0", "id": None, "method": "initialize"}), ctx)
    assert r["id"] is None and "q4km_dequant_matvec" in r["result"]["kernels"]
    r = mcp.handle_line(json.dumps({"jsonrpc": "2.0", "id": 4, "method": "bench_variant",
                                    "params": {"kernel": "saxpy"}}), ctx)
    assert r["error"]["code"] == mcp.INVALID_PARAMS
    r = mcp.handle_line(json.dumps({"jsonrpc": "2.0", "id": 5, "method": "enumerate_variants",
                                    "params": {"kernel": "q4_0_dequant_matvec"}}), ctx)
    (h,) = mcp.default_holes("q4_0_dequant_matvec")
    assert r["result"]["count"] == len(h["rows_per_wave"]) * len(h["waves_per_workgroup"])
    r = mcp.handle_line(json.dumps({"jsonrpc": "2.0", "id": 6, "method": "enumerate_variants",
                                    "params": {"kernel": "q4_0_dequant_matvec",
                                               "holes_override": {}}}), ctx)
    assert r["error"]["code"] == mcp.ENUMERATE_ERROR


def test_bench_without_a_device_reports_device_unavailable(mcp, tmp_path, axc):
    try:
        axc.HipContext.new().close()
        pytest.skip("a GPU is present")
    except axc.DispatchError:
        pass
    ctx = mcp.McpContext(history_dir=tmp_path)
    req = {"jsonrpc": "2.0", "id": 1, "method": "bench_variant",
           "params": {"kernel": "q4km_dequant_matvec", "shape": {"n_rows": 4, "units_per_row": 1},
                      "sample_count": 1}}
    r1 = mcp.handle_line(json.dumps(req), ctx)
    r2 = mcp.handle_line(json.dumps(req), ctx)  # the failure is cached
    assert r1["error"]["code"] == r2["error"]["code"] == mcp.DEVICE_UNAVAILABLE
