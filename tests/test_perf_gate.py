"""The performance gate trips (CPU): its decision on planted numbers, and on
the oracle timed against a copy of itself with a planted slowdown, the CPU
counterpart of the reference's fixture (benches/common.rs:113-124 adds a busy
loop to a CPU reference under feature bench_regression_fixture_slowdown, and
crates/axc-driver/tests/bench_regression.rs:185-195 asserts the gate fails).
"""
from __future__ import annotations

import pytest

import perf_gate as G
from oracle import oracle as O


def test_gate_decision():
    assert G.ratio_gate(6.6, 7.8, 0.76).ok
    r = G.ratio_gate(6.6, 10.0, 0.76)
    assert not r.ok and abs(r.ratio - 0.66) < 1e-12
    assert G.ratio_gate(6.6, 6.6 / 0.76, 0.76).ok  # exactly at the threshold passes
    assert not G.ratio_gate(6.6, 6.6 / 0.76 * 1.0001, 0.76).ok
    for bad in ((0.0, 1.0, 0.5), (1.0, -1.0, 0.5), (1.0, 1.0, 0.0)):
        with pytest.raises(ValueError):
            G.ratio_gate(*bad)


def test_interleaved_medians_take_one_sample_of_each_per_round():
    order = []
    seq = {"a": iter([5, 1, 3]), "b": iter([9, 7, 8])}

    def measure(k):
        order.append(k)
        return next(seq[k])

    med = G.interleaved_medians(measure, ("a", "b"), 3)
    assert order == ["a", "b", "b", "a", "a", "b"]  # ABBA
    assert med == {"a": 3, "b": 8}


def _oracle_case():
    rows, sb = 64, 16
    q = O.gen_q4k_weights(5, rows * sb)
    x = O.gen_normal_f32(6, sb * 256)
    return lambda: O.q4k_matvec(q, x, rows, sb, threads=1)


def test_planted_slowdown_in_the_oracle_fails_the_gate():
    """The oracle against itself passes; the same oracle made 3x slower by a
    planted repeat of its work (the result unchanged) fails."""
    run = _oracle_case()
    ref = run()

    def planted():
        y = run()
        run()
        run()  # the planted slowdown: the work done three times
        return y

    assert (planted() == ref).all()  # same output, only slower
    ops = {"floor": run, "same": run, "slow": planted}
    # about 10 ms of oracle calls per sample, each sample the fastest of three
    # timings (host noise only adds time), 9 rounds: a scheduler hiccup on this
    # shared host moves one timing, not the sample or the median
    measure = lambda k: min(G.wall_us(ops[k], 7) for _ in range(3))
    same = G.gate_from_rounds(measure, "floor", "same", 0.76, rounds=9)
    slow = G.gate_from_rounds(measure, "floor", "slow", 0.76, rounds=9)
    assert same.ok, same
    assert not slow.ok, slow
    assert slow.ratio < 0.5, slow
