"""Python mirror of the autotuner surface (crates/axc-optimize) over axh_tune.h.

  enumerate_strategy(holes) -> list[StrategyVariant]        (enumerator.rs:68-129)
  grid_search(holes, policy, correctness_fn, bench_fn)       (grid_search.rs:158-283)
  q4k_matvec_autotune(ctx, q, x, y, n_rows, sb_per_row)      (every Q4_K family, checked)
  WinnerTable / load_winners(path)                           (per-shape winners, JSON)

`holes` is a mapping name -> candidate list (source order; index 0 is the
baseline), like StrategyHoles.map.  bench_fn(assignments) returns SampleStats
or raises; correctness_fn(assignments) returns None or raises.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Callable, Mapping, Optional, Sequence

from . import axh as _axh

CARTESIAN_WARN_THRESHOLD = 100


class _Hole(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("candidates", ctypes.POINTER(ctypes.c_int64)),
                ("n_candidates", ctypes.c_uint32)]


class _Policy(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_uint32), ("ulp", ctypes.c_uint32)]


class _Stats(ctypes.Structure):
    _fields_ = [("median_ns", ctypes.c_uint64), ("min_ns", ctypes.c_uint64),
                ("max_ns", ctypes.c_uint64), ("n_samples", ctypes.c_uint32)]


class _Result(ctypes.Structure):
    _fields_ = [("ordinal", ctypes.c_uint64), ("variant_id", ctypes.c_uint64),
                ("outcome", ctypes.c_uint32), ("stats", _Stats), ("message", ctypes.c_char * 120)]


class _Summary(ctypes.Structure):
    _fields_ = [("winner_ordinal", ctypes.c_uint64), ("winner_variant_id", ctypes.c_uint64),
                ("fallback_used", ctypes.c_uint32), ("warned_large_product", ctypes.c_uint32),
                ("n_results", ctypes.c_uint64)]


class _Report(ctypes.Structure):
    _fields_ = [("best", _axh._Variant), ("best_median_ns", ctypes.c_uint64),
                ("dflt", _axh._Variant), ("default_median_ns", ctypes.c_uint64),
                ("variants", ctypes.c_uint32), ("accepted", ctypes.c_uint32),
                ("rejected", ctypes.c_uint32), ("failed", ctypes.c_uint32),
                ("best_kernel", ctypes.c_char * 64), ("confirm_best_ns", ctypes.c_uint64),
                ("confirm_default_ns", ctypes.c_uint64), ("kept_default", ctypes.c_uint32),
                ("weight_copies", ctypes.c_uint32)]


_BENCH = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64,
                          ctypes.POINTER(ctypes.c_int64), ctypes.c_uint32,
                          ctypes.POINTER(_Stats), ctypes.c_void_p, ctypes.c_size_t)
_CORRECT = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64,
                            ctypes.POINTER(ctypes.c_int64), ctypes.c_uint32,
                            ctypes.c_void_p, ctypes.c_size_t)

_configured = False


def _lib():
    global _configured
    lib = _axh.load_library()
    if not _configured:
        c = ctypes
        lib.axh_xxh3_64.restype = c.c_uint64
        lib.axh_xxh3_64.argtypes = [c.c_void_p, c.c_size_t]
        lib.axh_enumerate_strategy.restype = c.c_int
        lib.axh_enumerate_strategy.argtypes = [c.POINTER(_Hole), c.c_uint32,
                                               c.POINTER(c.c_uint64), c.POINTER(c.c_uint32),
                                               c.POINTER(c.c_int64), c.POINTER(c.c_uint64),
                                               c.c_uint64]
        lib.axh_grid_search.restype = c.c_int
        lib.axh_grid_search.argtypes = [c.POINTER(_Hole), c.c_uint32, c.POINTER(_Policy),
                                        _CORRECT, _BENCH, c.c_void_p, c.POINTER(_Result),
                                        c.c_uint64, c.POINTER(_Summary)]
        lib.axh_q4k_matvec_family_holes.restype = c.c_int
        lib.axh_q4k_matvec_family_holes.argtypes = [c.c_uint32, c.c_uint32, c.c_uint32,
                                                    c.POINTER(c.c_char_p),
                                                    c.POINTER(c.c_uint32),
                                                    c.POINTER(c.c_int64), c.c_uint32,
                                                    c.c_uint32, c.POINTER(c.c_uint32)]
        lib.axh_q4k_matvec_autotune.restype = c.c_int
        lib.axh_q4k_matvec_autotune.argtypes = [c.c_void_p, c.c_void_p, c.c_void_p, c.c_void_p,
                                                c.c_uint32, c.c_uint32, c.c_uint32, c.c_double,
                                                c.POINTER(_Report)]
        vp, u32, u64 = c.c_void_p, c.c_uint32, c.c_uint64
        V = c.POINTER(_axh._Variant)
        for name, res, args in (
                ("axh_winners_new", vp, []), ("axh_winners_free", None, [vp]),
                ("axh_winners_count", u64, [vp]),
                ("axh_winners_load", c.c_int, [c.c_char_p, c.POINTER(vp)]),
                ("axh_winners_save", c.c_int, [vp, c.c_char_p]),
                ("axh_winners_put", c.c_int, [vp, c.c_char_p, u32, u32, V, u64]),
                ("axh_winners_get", c.c_int, [vp, c.c_char_p, u32, u32, c.POINTER(u32), V,
                                              c.POINTER(u64)]),
                ("axh_context_winner_put", c.c_int, [vp, c.c_char_p, u32, u32, V, u64]),
                ("axh_context_winner_get", c.c_int, [vp, c.c_char_p, u32, u32, c.POINTER(u32),
                                                     V, c.POINTER(u64)]),
                ("axh_context_winners_save", c.c_int, [vp]),
                ("axh_context_winners_path", c.c_char_p, [vp]),
                ("axh_context_q4k_matvec_kernel_name", c.c_int, [vp, u32, u32, V, c.c_char_p,
                                                                 c.c_size_t])):
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _configured = True
    return lib


class TuneError(_axh.DispatchError):
    NAMES = {40: "EmptyStrategy", 41: "UnknownHole", 42: "NoStrategy", 43: "EnumerateFailed",
             44: "NoSuccessfulVariants"}

    def __init__(self, status: int, message: str):
        super().__init__(status, message)
        self.variant = self.NAMES.get(self.status, self.variant)


def _check(status: int) -> None:
    if status != 0:
        raise TuneError(status, _lib().axh_last_error().decode(errors="replace"))


def xxh3_64(data: bytes) -> int:
    b = bytes(data)
    return int(_lib().axh_xxh3_64(ctypes.c_char_p(b) if b else None, len(b)))


@dataclass(frozen=True)
class StrategyVariant:
    ordinal: int
    variant_id: int
    assignments: dict


@dataclass
class SampleStats:
    median_ns: int
    min_ns: int
    max_ns: int
    n_samples: int


@dataclass
class CorrectnessPolicy:
    """NONE, BIT_EXACT or EQUIV_FP_TOL(ulp) (grid_search.rs:55-66)."""

    kind: int = 0
    ulp: int = 0
    NONE = 0
    BIT_EXACT = 1
    EQUIV_FP_TOL = 2


@dataclass
class VariantResult:
    ordinal: int
    variant_id: int
    assignments: dict
    outcome: str  # "Ok" | "Failed" | "CorrectnessRejected"
    stats: Optional[SampleStats]
    message: str


@dataclass
class GridSearchResult:
    winner_ordinal: int
    winner_variant_id: int
    winner_assignments: dict
    results: list
    fallback_used: bool
    warnings: list = field(default_factory=list)


def _holes(holes: Mapping[str, Sequence[int]]):
    names = list(holes)
    keep = []
    arr = (_Hole * max(1, len(names)))()
    for i, n in enumerate(names):
        cand = (ctypes.c_int64 * max(1, len(holes[n])))(*holes[n])
        nb = n.encode()
        keep += [cand, nb]
        arr[i] = _Hole(nb, ctypes.cast(cand, ctypes.POINTER(ctypes.c_int64)), len(holes[n]))
    return arr, names, keep


def enumerate_strategy(holes: Mapping[str, Sequence[int]]) -> list:
    arr, names, keep = _holes(holes)
    lib = _lib()
    n = ctypes.c_uint64()
    order = (ctypes.c_uint32 * max(1, len(names)))()
    _check(lib.axh_enumerate_strategy(arr, len(names), ctypes.byref(n), order, None, None, 0))
    total = n.value
    vals = (ctypes.c_int64 * max(1, total * len(names)))()
    ids = (ctypes.c_uint64 * max(1, total))()
    _check(lib.axh_enumerate_strategy(arr, len(names), ctypes.byref(n), order, vals, ids, total))
    keys = [names[order[k]] for k in range(len(names))]
    out = []
    for v in range(total):
        a = {keys[k]: int(vals[v * len(keys) + k]) for k in range(len(keys))}
        out.append(StrategyVariant(v, int(ids[v]), a))
    return out


_OUTCOMES = {0: "Ok", 1: "Failed", 2: "CorrectnessRejected"}


def grid_search(holes: Mapping[str, Sequence[int]], policy: CorrectnessPolicy,
                correctness_fn: Optional[Callable[[dict], None]],
                bench_fn: Callable[[dict], SampleStats]) -> GridSearchResult:
    arr, names, keep = _holes(holes)
    lib = _lib()
    n_keys = len(names)
    variants = enumerate_strategy(holes) if n_keys else []
    keys = list(variants[0].assignments) if variants else []

    def _assign(vals, nh):
        return {keys[k]: int(vals[k]) for k in range(nh)}

    def _write(buf, cap, msg):
        raw = str(msg).encode(errors="replace")[: max(0, cap - 1)]
        ctypes.memmove(buf, raw + b"\0", len(raw) + 1)

    @_BENCH
    def cb_bench(user, ordinal, vals, nh, out, err, cap):
        try:
            s = bench_fn(_assign(vals, nh))
            out[0].median_ns, out[0].min_ns = s.median_ns, s.min_ns
            out[0].max_ns, out[0].n_samples = s.max_ns, s.n_samples
            return 0
        except Exception as e:  # reported as BenchOutcome::Failed
            _write(err, cap, e)
            return 1

    @_CORRECT
    def cb_correct(user, ordinal, vals, nh, err, cap):
        try:
            correctness_fn(_assign(vals, nh))
            return 0
        except Exception as e:  # reported as CorrectnessRejected
            _write(err, cap, e)
            return 1

    total = len(variants)
    res = (_Result * max(1, total))()
    summ = _Summary()
    pol = _Policy(policy.kind, policy.ulp)
    _check(lib.axh_grid_search(arr, n_keys, ctypes.byref(pol),
                               cb_correct if correctness_fn else _CORRECT(),
                               cb_bench, None, res, total, ctypes.byref(summ)))
    results = []
    for v in range(total):
        r = res[v]
        st = SampleStats(r.stats.median_ns, r.stats.min_ns, r.stats.max_ns, r.stats.n_samples)
        results.append(VariantResult(int(r.ordinal), int(r.variant_id), variants[v].assignments,
                                     _OUTCOMES[r.outcome], st if r.outcome == 0 else None,
                                     r.message.decode(errors="replace")))
    warnings = []
    if summ.warned_large_product:
        warnings.append(f"Cartesian product size {total} exceeds CARTESIAN_WARN_THRESHOLD "
                        f"({CARTESIAN_WARN_THRESHOLD}); grid search may take a long time")
    w = int(summ.winner_ordinal)
    return GridSearchResult(w, int(summ.winner_variant_id), variants[w].assignments, results,
                            bool(summ.fallback_used), warnings)


@dataclass
class AutotuneReport:
    best: "_axh.Variant"
    best_median_ns: int
    default: "_axh.Variant"
    default_median_ns: int
    variants: int
    accepted: int
    rejected: int
    failed: int
    best_kernel: str
    confirm_best_ns: int = 0
    confirm_default_ns: int = 0
    kept_default: bool = False
    weight_copies: int = 1


def q4k_matvec_family_holes(family: int, n_rows: int, sb_per_row: int) -> Optional[dict]:
    """The hole space the autotuner searches for `family` at this shape
    ({hole: [candidates]}, the family hole included), or None when the family
    has no kernel for the shape."""
    lib = _lib()
    n = ctypes.c_uint32()
    if lib.axh_q4k_matvec_family_holes(family, n_rows, sb_per_row, None, None, None, 0, 0,
                                       ctypes.byref(n)) != 0:
        return None
    names = (ctypes.c_char_p * n.value)()
    counts = (ctypes.c_uint32 * n.value)()
    cands = (ctypes.c_int64 * 256)()
    _check(lib.axh_q4k_matvec_family_holes(family, n_rows, sb_per_row, names, counts, cands,
                                           n.value, 256, ctypes.byref(n)))
    out, k = {}, 0
    for h in range(n.value):
        out[names[h].decode()] = [int(cands[k + i]) for i in range(counts[h])]
        k += counts[h]
    return out


def q4k_matvec_hole_spaces(n_rows: int, sb_per_row: int) -> list:
    """One hole map per Q4_K matvec family that takes the shape, in family
    order: the space axh_q4k_matvec_autotune searches."""
    return [h for f in range(1, 8) if (h := q4k_matvec_family_holes(f, n_rows, sb_per_row))]


def q4_0_matvec_hole_spaces(n_rows: int, blocks_per_row: int) -> list:
    """One hole map per Q4_0 matvec family that takes the shape: the LDS-tiled
    kernel's holes first (family 0 with rows_per_wave / waves_per_workgroup),
    then the persistent, one-pass, one-pass-with-x-whole and column families
    (the family hole first, with the family as its one candidate).  A family
    takes the shape when its plain assignment plans to a kernel; assignments
    of a map that name no compiled kernel fail to plan and rank as failures."""
    V = _axh.Variant

    def takes(v):
        try:
            _axh.q4_0_matvec_kernel_name(n_rows, blocks_per_row, v)
            return True
        except _axh.DispatchError:
            return False

    vs = _axh.compiled_variants("q4_0")
    out = [{"rows_per_wave": sorted({v.rows_per_wave for v in vs}),
            "waves_per_workgroup": sorted({v.waves_per_workgroup for v in vs})}]
    need = (blocks_per_row + 63) // 64
    steps = [need] + ([need + 1] if need < 16 else [])
    if takes(V(family=_axh.FAMILY_PERSISTENT)):
        out.append({"family": [_axh.FAMILY_PERSISTENT], "prefetch": [1, 2],
                    "rows_per_wave": [1, 2], "waves_per_workgroup": [4, 8, 16]})
    if takes(V(prefetch=1, family=_axh.FAMILY_ONE_PASS)):
        out.append({"family": [_axh.FAMILY_ONE_PASS], "prefetch": [1, 2], "sb_per_lane": steps})
        out.append({"family": [_axh.FAMILY_ONE_PASS_X], "sb_per_lane": steps})
    if takes(V(family=_axh.FAMILY_COLUMNS)):
        out.append({"family": [_axh.FAMILY_COLUMNS]})
    return out


def q4k_matvec_autotune(ctx, q, x, y, n_rows: int, sb_per_row: int, samples: int = 5,
                        tol: float = 1e-3) -> AutotuneReport:
    """Grid search over every Q4_K matvec kernel family on resident buffers; each
    variant is judged by the f64 host checker (relative `tol`) and timed.  The
    winner is stored in the context's table (and its file, if it has one)."""
    r = _Report()
    _check(_lib().axh_q4k_matvec_autotune(ctx.raw, _axh._ptr(q), _axh._ptr(x), _axh._ptr(y),
                                          n_rows, sb_per_row, samples, tol, ctypes.byref(r)))
    return AutotuneReport(_axh._variant_from_c(r.best), int(r.best_median_ns),
                          _axh._variant_from_c(r.dflt), int(r.default_median_ns),
                          r.variants, r.accepted, r.rejected, r.failed, r.best_kernel.decode(),
                          int(r.confirm_best_ns), int(r.confirm_default_ns),
                          bool(r.kept_default), int(r.weight_copies))


class WinnerTable:
    """Per-shape tuned winners (axh_winners_*): op, n_rows, units -> (Variant, median_ns)."""

    def __init__(self, raw: Optional[int] = None):
        self._raw = raw if raw is not None else _lib().axh_winners_new()

    @classmethod
    def load(cls, path) -> "WinnerTable":
        raw = ctypes.c_void_p()
        _check(_lib().axh_winners_load(str(path).encode(), ctypes.byref(raw)))
        return cls(raw.value)

    def save(self, path) -> None:
        _check(_lib().axh_winners_save(self._raw, str(path).encode()))

    def __len__(self) -> int:
        return int(_lib().axh_winners_count(self._raw))

    def put(self, op: str, n_rows: int, units: int, v: "_axh.Variant", median_ns: int) -> None:
        c = v._c()
        _check(_lib().axh_winners_put(self._raw, op.encode(), n_rows, units, ctypes.byref(c),
                                      median_ns))

    def get(self, op: str, n_rows: int, units: int):
        found, c, ns = ctypes.c_uint32(), _axh._Variant(), ctypes.c_uint64()
        _check(_lib().axh_winners_get(self._raw, op.encode(), n_rows, units, ctypes.byref(found),
                                      ctypes.byref(c), ctypes.byref(ns)))
        return (_axh._variant_from_c(c), int(ns.value)) if found.value else None

    def close(self) -> None:
        if self._raw:
            _lib().axh_winners_free(self._raw)
            self._raw = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def context_winner_put(ctx, op: str, n_rows: int, units: int, v: "_axh.Variant",
                       median_ns: int = 0) -> None:
    c = v._c()
    _check(_lib().axh_context_winner_put(ctx.raw, op.encode(), n_rows, units, ctypes.byref(c),
                                         median_ns))


def context_winner_get(ctx, op: str, n_rows: int, units: int):
    found, c, ns = ctypes.c_uint32(), _axh._Variant(), ctypes.c_uint64()
    _check(_lib().axh_context_winner_get(ctx.raw, op.encode(), n_rows, units,
                                         ctypes.byref(found), ctypes.byref(c), ctypes.byref(ns)))
    return (_axh._variant_from_c(c), int(ns.value)) if found.value else None


def context_winners_save(ctx) -> None:
    _check(_lib().axh_context_winners_save(ctx.raw))


def context_winners_path(ctx) -> str:
    return _lib().axh_context_winners_path(ctx.raw).decode()


def context_q4k_matvec_kernel_name(ctx, n_rows: int, sb_per_row: int, variant=None) -> str:
    """Kernel axh_q4k_matvec launches on this context (consults its winner table)."""
    v = variant._c() if variant else None
    buf = ctypes.create_string_buffer(64)
    _check(_lib().axh_context_q4k_matvec_kernel_name(ctx.raw, n_rows, sb_per_row,
                                                     ctypes.byref(v) if v else None, buf, 64))
    return buf.value.decode()
