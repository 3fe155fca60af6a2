"""Autotuner surface (CPU): the reference's AT-1014..AT-1042 semantics over
the C ABI, with mock bench/correctness callbacks like the reference's own
grid-search tests (crates/axc-optimize/src/grid_search.rs:325-526)."""
from __future__ import annotations

import struct

import pytest
import xxhash


@pytest.fixture(scope="module")
def tune(axc):
    import importlib
    return importlib.import_module("axiom_compute_amd.tune")


def test_xxh3_matches_published_implementation_all_lengths(tune):
    """Every length path of XXH3-64 (0..3, 4..8, 9..16, 17..128, 129..240, long)."""
    import random
    rnd = random.Random(5)
    for n in list(range(0, 300)) + [511, 512, 1023, 1024, 1025, 2047, 4096, 9999, 70000]:
        data = bytes(rnd.getrandbits(8) for _ in range(n))
        assert tune.xxh3_64(data) == xxhash.xxh3_64_intdigest(data), n


def test_at_1014_empty_strategy_is_an_error(tune):
    with pytest.raises(tune.TuneError) as e:
        tune.enumerate_strategy({})
    assert e.value.variant == "EmptyStrategy"


def test_at_1015_single_hole_three_candidates_in_order(tune):
    vs = tune.enumerate_strategy({"workgroup_x": [32, 64, 128]})
    assert [v.ordinal for v in vs] == [0, 1, 2]
    assert [v.assignments["workgroup_x"] for v in vs] == [32, 64, 128]


def test_at_1016_two_holes_last_key_varies_fastest(tune):
    vs = tune.enumerate_strategy({"b": [10, 20], "a": [1, 2]})
    assert [(v.assignments["a"], v.assignments["b"]) for v in vs] == [(1, 10), (1, 20), (2, 10), (2, 20)]


def test_at_1037_variant_id_is_xxh3_of_canonical_encoding(tune):
    name = b"workgroup_x"
    enc = struct.pack("<I", len(name)) + name + struct.pack("<q", 64)
    vs = tune.enumerate_strategy({"workgroup_x": [32, 64, 128]})
    assert vs[1].variant_id == xxhash.xxh3_64_intdigest(enc)


def test_variant_id_multi_key_encoding_and_negative_values(tune):
    vs = tune.enumerate_strategy({"rows_per_wave": [1, 2], "prefetch": [-3, 7]})
    for v in vs:
        enc = b""
        for k in sorted(v.assignments):
            enc += struct.pack("<I", len(k)) + k.encode() + struct.pack("<q", v.assignments[k])
        assert v.variant_id == xxhash.xxh3_64_intdigest(enc)
    assert len({v.variant_id for v in vs}) == 4


def test_at_1039_three_holes_cartesian_count_and_order(tune):
    vs = tune.enumerate_strategy({"c": [100, 200], "a": [1, 2], "b": [10, 20, 30]})
    assert len(vs) == 12
    assert vs[0].assignments == {"a": 1, "b": 10, "c": 100}
    assert vs[11].assignments == {"a": 2, "b": 30, "c": 200}


def test_duplicate_or_empty_candidate_lists_are_rejected(tune):
    with pytest.raises(tune.TuneError):
        tune.enumerate_strategy({"a": []})


def tune_stats(median):
    import importlib
    t = importlib.import_module("axiom_compute_amd.tune")
    return t.SampleStats(median, median - 5, median + 5, 5)


def test_at_1022_no_strategy_is_an_error(tune):
    with pytest.raises(tune.TuneError) as e:
        tune.grid_search({}, tune.CorrectnessPolicy(), None, lambda a: tune_stats(100))
    assert e.value.variant == "NoStrategy"


def test_at_1023_picks_fastest_variant(tune):
    calls = []

    def bench(a):
        calls.append(a["workgroup_x"])
        return tune_stats(50 if len(calls) == 1 else 100)

    r = tune.grid_search({"workgroup_x": [32, 64]}, tune.CorrectnessPolicy(), None, bench)
    assert r.winner_ordinal == 0 and not r.fallback_used and len(r.results) == 2
    assert calls == [32, 64]


def test_ties_keep_the_lowest_ordinal(tune):
    r = tune.grid_search({"w": [1, 2, 3]}, tune.CorrectnessPolicy(), None,
                         lambda a: tune_stats(70 if a["w"] > 1 else 90))
    assert r.winner_ordinal == 1


def test_at_1024_fallback_when_all_bench_fail(tune):
    def bench(a):
        raise RuntimeError("simulated bench failure")

    r = tune.grid_search({"workgroup_x": [32, 64, 128]}, tune.CorrectnessPolicy(), None, bench)
    assert r.fallback_used and r.winner_ordinal == 0
    assert all(x.outcome == "Failed" and "simulated" in x.message for x in r.results)


def test_at_1025_correctness_failure_excludes_variant(tune):
    def correct(a):
        if a["workgroup_x"] == 32:
            raise ValueError("bit mismatch")

    r = tune.grid_search({"workgroup_x": [32, 64]},
                         tune.CorrectnessPolicy(tune.CorrectnessPolicy.BIT_EXACT), correct,
                         lambda a: tune_stats(10 if a["workgroup_x"] == 32 else 99))
    assert r.results[0].outcome == "CorrectnessRejected"
    assert r.winner_ordinal == 1


def test_policy_none_skips_correctness_callback(tune):
    def correct(a):
        raise AssertionError("must not be called")

    r = tune.grid_search({"w": [1, 2]}, tune.CorrectnessPolicy(), correct, lambda a: tune_stats(5))
    assert all(x.outcome == "Ok" for x in r.results)


def test_at_1026_warn_threshold_is_100(tune):
    assert tune.CARTESIAN_WARN_THRESHOLD == 100
    r = tune.grid_search({"a": list(range(11)), "b": list(range(10))}, tune.CorrectnessPolicy(),
                         None, lambda a: tune_stats(1 + a["a"] + a["b"]))
    assert len(r.results) == 110 and r.warnings


def test_at_1040_winner_variant_id_matches_enumerator(tune):
    holes = {"x": [1, 2, 3], "y": [5, 6]}
    r = tune.grid_search(holes, tune.CorrectnessPolicy(), None,
                         lambda a: tune_stats(100 - a["x"] * 10 - a["y"]))
    vs = tune.enumerate_strategy(holes)
    assert r.winner_variant_id == vs[r.winner_ordinal].variant_id
    assert r.winner_assignments == {"x": 3, "y": 6}


def test_at_1042_results_contain_all_variants_in_ordinal_order(tune):
    r = tune.grid_search({"x": [1, 2, 3], "y": [5, 6]}, tune.CorrectnessPolicy(), None,
                         lambda a: tune_stats(7))
    assert [x.ordinal for x in r.results] == list(range(6))
