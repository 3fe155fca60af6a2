"""Kernel-family holes and the tuned-winner table (CPU).

Every default kernel of the Q4_K matvec is a hole assignment (the autotuner
can reach it), the family holes are validated, and the winner table - the
counterpart of the reference's strategy sidecar and pipeline cache
(crates/axc-driver/src/optimize.rs:103-128, crates/axc-runtime/src/
pipeline_cache.rs:45-170) - round-trips through its JSON file and reports a
malformed file as PipelineCacheLoadFailed.
"""
from __future__ import annotations

import json

import pytest

SHAPES = [(1, 1), (1, 16), (1, 33), (1, 128), (2, 40), (3, 64), (4, 128), (5, 128), (31, 256),
          (31, 16), (32, 16), (256, 16), (4096, 56), (4096, 16), (14336, 16), (6144, 32),
          (6144, 33), (32768, 16), (32769, 17), (40000, 16), (65536, 16), (65537, 16),
          (128256, 16), (4096, 129), (100, 300), (3000, 200), (4160, 16), (5120, 24),
          (5120, 32), (6143, 25), (6144, 112), (8191, 74), (777, 24), (32, 56)]


@pytest.fixture(scope="module")
def tune(axc):
    import importlib
    return importlib.import_module("axiom_compute_amd.tune")


@pytest.mark.parametrize("rows,sb", SHAPES)
def test_every_default_is_a_hole_assignment(axc, rows, sb):
    d = axc.q4k_matvec_default_variant(rows, sb)
    assert d.family != axc.FAMILY_DEFAULT
    assert axc.q4k_matvec_kernel_name(rows, sb, d) == axc.q4k_matvec_kernel_name(rows, sb)
    if d.family in (axc.FAMILY_ONE_PASS, axc.FAMILY_ONE_PASS_X):
        assert d.sb_per_lane == (sb + 7) // 8
        assert d.prefetch == (0 if d.family == axc.FAMILY_ONE_PASS_X else
                              2 if (sb + 7) // 8 >= 4 and rows <= 4096 else 1)
    if d.family == axc.FAMILY_PERSISTENT:
        assert 0 not in (d.rows_per_wave, d.waves_per_workgroup, d.prefetch, d.nontemporal)


def test_family_defaults_by_shape(axc):
    F = axc
    fam = lambda r, s: axc.q4k_matvec_default_variant(r, s).family
    assert fam(1, 128) == F.FAMILY_WORKGROUP
    assert fam(5, 129) == F.FAMILY_SPLIT_K
    assert fam(5, 128) == fam(5, 16) == F.FAMILY_TILED
    assert fam(4096, 56) == F.FAMILY_ONE_PASS
    assert fam(14336, 16) == F.FAMILY_ONE_PASS_X
    assert fam(128256, 16) == F.FAMILY_PERSISTENT
    assert fam(5120, 16) == F.FAMILY_ONE_PASS_X  # 4097-6143 rows, up to 24 superblocks
    assert fam(5120, 32) == F.FAMILY_PERSISTENT  # 4097-6143 rows, 25-32 superblocks
    assert fam(6144, 112) == F.FAMILY_PERSISTENT  # 4097-8191 rows, 74+ superblocks
    assert fam(1024, 32) == F.FAMILY_TILED  # up to 1024 rows of 24+ superblocks
    assert fam(4096, 129) == F.FAMILY_TILED


def test_each_family_names_its_kernel(axc):
    V, F = axc.Variant, axc
    n = axc.q4k_matvec_kernel_name
    assert n(4096, 56, V(family=F.FAMILY_ONE_PASS)) == "axh_q4k_matvec_onep_i7"
    assert n(4096, 56, V(family=F.FAMILY_ONE_PASS, sb_per_lane=9)) == "axh_q4k_matvec_onep_i9"
    assert n(4096, 56, V(prefetch=1, family=F.FAMILY_ONE_PASS)) == "axh_q4k_matvec_one_i7"
    assert n(8192, 56, V(family=F.FAMILY_ONE_PASS)) == "axh_q4k_matvec_one_i7"
    assert n(8192, 56, V(prefetch=2, family=F.FAMILY_ONE_PASS)) == "axh_q4k_matvec_onep_i7"
    assert n(4096, 24, V(prefetch=2, family=F.FAMILY_ONE_PASS)) == "axh_q4k_matvec_onep_i3"
    assert n(4096, 56, V(family=F.FAMILY_ONE_PASS_X)) == "axh_q4k_matvec_onex_i7"
    assert n(4096, 56, V(family=F.FAMILY_PERSISTENT)) == "axh_q4k_matvec_flat_r1_w8_p2_n0"
    assert n(4096, 56, V(2, 8, 1, 2, F.FAMILY_PERSISTENT)) == "axh_q4k_matvec_flat_r2_w8_p1_n0"
    assert n(4096, 56, V(family=F.FAMILY_TILED)) == "axh_q4k_matvec_tiled_r2_w8_p2"
    assert n(100, 56, V(family=F.FAMILY_TILED)) == "axh_q4k_matvec_tiled_r1_w4_p2"
    assert n(4096, 56, V(1, 4, 2, 0, F.FAMILY_TILED)) == "axh_q4k_matvec_tiled_r1_w4_p2"
    assert n(3, 100, V(family=F.FAMILY_WORKGROUP)) == "axh_q4k_matvec_wg_w8_x2_r4"
    assert n(1, 100, V(2, family=F.FAMILY_WORKGROUP)) == "axh_q4k_matvec_wg_w8_x2_r2"
    assert n(20, 100, V(family=F.FAMILY_SPLIT_K)) == "axh_q4k_matvec_sk_s16"
    assert n(4096, 56, V(family=F.FAMILY_COLUMNS)) == "axh_q4k_matvec_cols_r4_w4_n0_x1"
    # the persistent holes alone still select the persistent family
    assert n(4096, 56, V(2, 4, 1, 2)) == "axh_q4k_matvec_flat_r2_w4_p1_n0"


@pytest.mark.parametrize("rows,sb,v,what", [
    (4096, 56, dict(family=2, sb_per_lane=6), "sb_per_lane too short for the row"),
    (4096, 56, dict(family=2, sb_per_lane=17), "no one-pass kernel beyond 16 steps"),
    (4096, 56, dict(family=1, sb_per_lane=7), "sb_per_lane outside the one-pass families"),
    (4096, 56, dict(family=2, rows_per_wave=2), "one pass has no rows_per_wave hole"),
    (4096, 56, dict(family=2, prefetch=3), "x at most two chunks ahead"),
    (4096, 16, dict(family=2, prefetch=2), "two ahead needs three steps"),
    (14336, 16, dict(family=3, prefetch=1), "whole x has no prefetch hole"),
    (5, 56, dict(family=4), "one workgroup takes at most 4 rows"),
    (3, 56, dict(family=4, rows_per_wave=2), "rows_per_wave below n_rows"),
    (33, 56, dict(family=5), "split-K takes at most 32 rows"),
    (4, 257, dict(family=5), "split-K takes at most 256 superblocks"),
    (4, 129, dict(family=6), "columns take at most 128 superblocks"),
    (4096, 129, dict(family=2), "one pass takes at most 128 superblocks"),
    (4096, 129, dict(family=1), "persistent family cannot stage this row"),
    (4096, 56, dict(family=7, rows_per_wave=4), "no such tiled kernel"),
    (4096, 56, dict(family=8), "unknown family"),
])
def test_invalid_family_assignments_are_typed_errors(axc, rows, sb, v, what):
    with pytest.raises(axc.DispatchError) as e:
        axc.q4k_matvec_kernel_name(rows, sb, axc.Variant(**v))
    assert e.value.variant == "InvalidArgument", what


def test_family_holes_belong_to_the_matvec_families(axc):
    """The family hole belongs to the Q4_K and Q4_0 matvecs (Q5_K / Q6_K take
    only their one-pass family); sb_per_lane only with a one-pass family."""
    for fn in (axc.q4k_gate_up_kernel_name, axc.q5k_matvec_kernel_name,
               axc.q6k_matvec_kernel_name):
        for v in (axc.Variant(family=1), axc.Variant(sb_per_lane=2)):
            with pytest.raises(axc.DispatchError):
                fn(4096, 16, v)
    q40 = axc.q4_0_matvec_kernel_name
    assert q40(4096, 16, axc.Variant(family=1)) == "axh_q4_0_matvec_flat_r1_w8_p1_x1"
    for v in (axc.Variant(sb_per_lane=2), axc.Variant(family=axc.FAMILY_WORKGROUP),
              axc.Variant(family=axc.FAMILY_SPLIT_K)):
        with pytest.raises(axc.DispatchError):
            q40(4096, 16, v)


# ---- the winner table -----------------------------------------------------------
def test_winner_table_round_trip(tune, axc, tmp_path):
    t = tune.WinnerTable()
    assert len(t) == 0 and t.get("q4k_matvec", 4096, 56) is None
    v1 = axc.Variant(2, 4, 1, 2, axc.FAMILY_PERSISTENT)
    v2 = axc.Variant(family=axc.FAMILY_ONE_PASS, sb_per_lane=7)
    t.put("q4k_matvec", 4096, 56, v1, 9100)
    t.put("q4k_matvec", 14336, 16, v2, 8200)
    t.put('op "quoted" \\ name', 1, 2, v2, 1)
    t.put("q4k_matvec", 4096, 56, v2, 8000)  # replaces
    assert len(t) == 3
    p = tmp_path / "axh_winners.json"
    t.save(p)
    doc = json.loads(p.read_text())  # the file is plain JSON
    assert doc["schema"] == "axh-winners-1" and len(doc["entries"]) == 3
    u = tune.WinnerTable.load(p)
    assert len(u) == 3
    assert u.get("q4k_matvec", 4096, 56) == (v2, 8000)
    assert u.get("q4k_matvec", 14336, 16) == (v2, 8200)
    assert u.get('op "quoted" \\ name', 1, 2) == (v2, 1)
    assert u.get("q4k_matvec", 4096, 57) is None
    assert not list(tmp_path.glob("*.tmp.*"))  # the atomic write left nothing behind
    t.close()
    u.close()


def test_missing_winner_table_loads_empty(tune, tmp_path):
    t = tune.WinnerTable.load(tmp_path / "absent.json")
    assert len(t) == 0


GOOD = ('{"schema": "axh-winners-1", "entries": [{"op": "q4k_matvec", "n_rows": 8, "units": 2, '
        '"family": 1, "rows_per_wave": 2, "waves_per_workgroup": 4, "prefetch": 1, '
        '"nontemporal": 2, "sb_per_lane": 0, "median_ns": 5}]}')


@pytest.mark.parametrize("text", [
    "", "{", "[]", "null", GOOD[:-1], GOOD + "x", GOOD.replace("axh-winners-1", "axh-winners-2"),
    GOOD.replace('"n_rows": 8, ', ""), GOOD.replace('"median_ns": 5', '"median_ns": -5'),
    GOOD.replace('"units": 2', '"units": 4294967296'), GOOD.replace('"units": 2', '"units": 2.5'),
    GOOD.replace('"units": 2', '"units": 2, "units": 3'), GOOD.replace('"op"', '"opp"'),
    GOOD.replace('"entries"', '"extra": 1, "entries"'), GOOD.replace('[{', '[{}, {'),
    GOOD.replace('"q4k_matvec"', '"q4k\\nmatvec"'), '{"schema": "axh-winners-1"}',
])
def test_malformed_winner_table_is_pipeline_cache_load_failed(tune, tmp_path, text):
    p = tmp_path / "w.json"
    p.write_text(text)
    with pytest.raises(tune.TuneError) as e:
        tune.WinnerTable.load(p)
    assert e.value.variant == "PipelineCacheLoadFailed", text


def test_good_fixture_parses(tune, axc, tmp_path):
    p = tmp_path / "w.json"
    p.write_text(GOOD)
    t = tune.WinnerTable.load(p)
    assert t.get("q4k_matvec", 8, 2) == (axc.Variant(2, 4, 1, 2, 1, 0), 5)
