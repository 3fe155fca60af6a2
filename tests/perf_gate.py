"""The decision of the performance regression gates, shared by the GPU gate
tests and the CPU tests that prove a gate trips.

A gate compares two timings taken on the same box in the same run, in
interleaved rounds (so that clock drift falls on both alike): a floor (a pure
read of the same bytes, or a reference kernel) and the candidate.  It passes
when floor / candidate reaches the gate's minimum ratio.  The reference's
regression gate (crates/axc-driver/tests/bench_regression.rs:185-195) fails a
bench above its baseline by more than 15 %; its fixture plants a slowdown
(benches/common.rs:113-124, feature bench_regression_fixture_slowdown) to
show that the gate trips.  Here the planted slowdown runs in the oracle, on
the CPU, and on the GPU a kernel known to be slower stands in for it.
"""
from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Callable, Mapping


@dataclass(frozen=True)
class GateResult:
    ok: bool
    ratio: float          # floor / candidate (1.0 = as fast as the floor)
    floor_us: float
    candidate_us: float
    min_ratio: float


def ratio_gate(floor_us: float, candidate_us: float, min_ratio: float) -> GateResult:
    """Pass when the candidate is within 1 / min_ratio of the floor's time."""
    if not (floor_us > 0 and candidate_us > 0 and 0 < min_ratio):
        raise ValueError(f"gate needs positive times and ratio: {floor_us}, {candidate_us}, "
                         f"{min_ratio}")
    ratio = floor_us / candidate_us
    return GateResult(ratio >= min_ratio, ratio, floor_us, candidate_us, min_ratio)


def interleaved_medians(measure: Callable[[str], float], names, rounds: int) -> dict:
    """Median of `rounds` measurements of each name, one of each per round, the
    order reversed every other round (ABBA), so that no name always runs first."""
    names = list(names)
    t = {k: [] for k in names}
    for i in range(rounds):
        for k in (names if i % 2 == 0 else names[::-1]):
            t[k].append(measure(k))
    return {k: sorted(v)[len(v) // 2] for k, v in t.items()}


def gate_from_rounds(measure: Callable[[str], float], floor: str, candidate: str,
                     min_ratio: float, rounds: int = 5) -> GateResult:
    """Times `floor` and `candidate` in interleaved rounds and applies the gate."""
    med = interleaved_medians(measure, (floor, candidate), rounds)
    return ratio_gate(med[floor], med[candidate], min_ratio)


def wall_us(fn: Callable[[], object], calls: int) -> float:
    """Host wall time per call of fn (CPU measurements)."""
    t0 = time.perf_counter()
    for _ in range(calls):
        fn()
    return (time.perf_counter() - t0) * 1e6 / calls


def bench_loop_measure(ctx, ops: Mapping[str, dict], calls: int) -> Callable[[str], float]:
    """measure(name): us per call of `calls` back-to-back calls of ops[name]
    launched by the library's loop (axh_bench_loop)."""
    def measure(k: str) -> float:
        return sum(ctx.bench_loop(**ops[k], warmup=20, groups=1, calls_per_group=calls)) \
            * 1e3 / calls
    return measure
