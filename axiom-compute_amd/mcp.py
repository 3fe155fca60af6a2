"""Tuning tools for LLM-driven search over the HIP kernels' strategy holes.

Mirrors the reference's MCP tool surface (crates/axc-driver/src/mcp/):
JSON-RPC 2.0 over stdio (dispatch.rs), `enumerate_variants`, `bench_variant`
(tools/bench_variant.rs) and `grid_search` (tools/grid_search.rs) with the
JSONL optimisation history, and `optimization_history`.  Where the reference
compiles `.axc` source with `@strategy` holes, the kernels here are the
library's compiled Q4 operations, named like the reference kernels:

  q4km_dequant_matvec  one hole map per kernel family that takes the shape
                       (family, then that family's holes among rows_per_wave,
                       waves_per_workgroup, prefetch, nontemporal, sb_per_lane):
                       the space of the library's autotuner, default kernels
                       included
  q4_0_dequant_matvec  holes rows_per_wave, waves_per_workgroup (the LDS-tiled
                       kernel), and with a shape one map per other kernel
                       family that takes it (persistent, one pass, one pass
                       with x whole, columns)
  q4k_matmul_f16       holes kind, waves_per_workgroup, col_tiles, prefetch, row_tiles

and a request names a shape ({"n_rows", "units_per_row", "batch"}) instead of
input byte sizes.  A search over several hole maps enumerates each map as the
reference enumerates one (keys sorted, last key fastest) and numbers the
variants on across the maps.  Correctness is a real verdict for every kernel (the
reference reports its Q4 kernel "not_checked", bench_variant.rs:395-400):
the device result is compared with an f64 accumulation of the reference's
dequantised weights by the library's host checker (include/axh_check.h).

Timing samples are HIP-event times on resident buffers (each sample the mean
of `launches_per_sample` back-to-back launches), not host round trips.  The
weights are copied on the device until the copies pass 512 MiB and the
launches rotate through them, so each launch reads HBM rather than the
256 MiB Infinity Cache.  grid_search runs one set of inputs for the whole
search and times the variants in interleaved rounds (one sample of every
variant per round), so drift of the clocks over a search falls on all
variants alike.
"""
from __future__ import annotations

import ctypes
import fcntl
import json
import os
import sys
from dataclasses import dataclass, field
from datetime import datetime, timezone
from pathlib import Path
from typing import Any, Optional

import numpy as np

from . import axh as _axh

# JSON-RPC error codes (protocol.rs:102-125; the reference's wire values).
PARSE_ERROR = -32700
INVALID_REQUEST = -32600
METHOD_NOT_FOUND = -32601
INVALID_PARAMS = -32602
INTERNAL_ERROR = -32603
ENUMERATE_ERROR = -32002
GRID_SEARCH_ERROR = -32003
DEVICE_UNAVAILABLE = -32004
IO_ERROR = -32005

METHODS = ("initialize", "enumerate_variants", "bench_variant", "grid_search",
           "optimization_history")
KERNELS = ("q4km_dequant_matvec", "q4_0_dequant_matvec", "q4k_matmul_f16")
CARTESIAN_WARN_THRESHOLD = 100
DEFAULT_REL_TOL = 1e-3


class McpToolError(Exception):
    def __init__(self, code: int, category: str, message: str):
        super().__init__(message)
        self.code, self.category, self.message = code, category, message

    def rpc(self) -> dict:
        return {"code": self.code, "message": self.message,
                "data": {"category": self.category, "detail": self.message}}


def invalid(msg: str) -> McpToolError:
    return McpToolError(INVALID_PARAMS, "invalid_params", msg)


# ---- small utilities ----------------------------------------------------------
def format_rfc3339_utc(t: Optional[datetime] = None) -> str:
    """`YYYY-MM-DDTHH:MM:SS.mmmZ` (grid_search.rs:34-75)."""
    t = (t or datetime.now(timezone.utc)).astimezone(timezone.utc)
    return t.strftime("%Y-%m-%dT%H:%M:%S.") + f"{t.microsecond // 1000:03d}Z"


def hex16(h: int) -> str:
    return f"{h:016x}"


def source_key(kernel: str, shape: dict) -> str:
    """What stands for the reference's source text: the kernel and its shape."""
    return json.dumps({"kernel": kernel, "shape": shape}, sort_keys=True)


def history_path(history_dir: Path, key: str) -> Path:
    """`<history_dir>/<xxh3_hex16(key)>.jsonl` (grid_search.rs:86-91)."""
    from . import tune
    return Path(history_dir) / f"{hex16(tune.xxh3_64(key.encode()))}.jsonl"


def append_history_entry(path: Path, entry: dict) -> None:
    """One JSON line per call under an exclusive flock (grid_search.rs:161-186)."""
    line = json.dumps(entry, separators=(",", ":"))
    assert "\n" not in line
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "a", encoding="utf-8") as f:
        fcntl.flock(f.fileno(), fcntl.LOCK_EX)
        try:
            f.write(line + "\n")
            f.flush()
        finally:
            fcntl.flock(f.fileno(), fcntl.LOCK_UN)


def read_git_sha(start: Path) -> Optional[str]:
    """Best-effort 7-character HEAD sha, or None."""
    for d in [start, *start.parents]:
        head = d / ".git" / "HEAD"
        if head.is_file():
            try:
                ref = head.read_text().strip()
                if ref.startswith("ref: "):
                    p = d / ".git" / ref[5:]
                    if p.is_file():
                        return p.read_text().strip()[:7]
                    packed = d / ".git" / "packed-refs"
                    if packed.is_file():
                        for ln in packed.read_text().splitlines():
                            if ln.endswith(ref[5:]):
                                return ln.split()[0][:7]
                    return None
                return ref[:7]
            except OSError:
                return None
    return None


def variant_id(assignments: dict) -> int:
    """xxh3_64 of the canonical encoding; 0 for no holes (bench_variant.rs:284-297)."""
    if not assignments:
        return 0
    from . import tune
    enc = b""
    for k in sorted(assignments):
        kb = k.encode()
        enc += len(kb).to_bytes(4, "little") + kb + int(assignments[k]).to_bytes(8, "little",
                                                                                  signed=True)
    return tune.xxh3_64(enc)


# ---- seeded inputs ------------------------------------------------------------
def seeded_inputs(kernel: str, shape: dict, vid: int):
    """Deterministic inputs per (variant_id, binding): binding i draws from
    PCG64(variant_id ^ i) (the reference seeds StdRng the same way,
    bench_variant.rs:84-99, but its byte stream is not reproduced).  Weights
    follow the benchmark distributions: d ~ U(0.001, 0.05), dmin ~ U(0, 0.02)
    as f16, uniform scale and quant bytes; x ~ N(0, 1)."""
    rows, units = int(shape["n_rows"]), int(shape["units_per_row"])
    rq = np.random.Generator(np.random.PCG64(vid ^ 0))
    rx = np.random.Generator(np.random.PCG64(vid ^ 1))
    if kernel == "q4_0_dequant_matvec":
        blk = rq.integers(0, 256, size=(rows * units, 18), dtype=np.uint8)
        d = rq.uniform(0.001, 0.05, rows * units).astype(np.float16)
        blk[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
        x = rx.standard_normal(units * 32).astype(np.float32)
        return blk.reshape(-1), x
    sb = rq.integers(0, 256, size=(rows * units, 144), dtype=np.uint8)
    d = rq.uniform(0.001, 0.05, rows * units).astype(np.float16)
    dmin = rq.uniform(0.0, 0.02, rows * units).astype(np.float16)
    sb[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    sb[:, 2:4] = dmin.view(np.uint8).reshape(-1, 2)
    if kernel == "q4k_matmul_f16":
        batch = int(shape.get("batch", 1))
        x = rx.standard_normal(units * 256 * batch).astype(np.float16)
    else:
        x = rx.standard_normal(units * 256).astype(np.float32)
    return sb.reshape(-1), x


# ---- host checker bindings -------------------------------------------------------
class _Report(ctypes.Structure):
    _fields_ = [("ok", ctypes.c_uint32), ("rows_checked", ctypes.c_uint64),
                ("rows_failed", ctypes.c_uint64), ("worst_row", ctypes.c_uint64),
                ("worst_over_allowed", ctypes.c_double), ("norm_rel_err", ctypes.c_double)]


_check_configured = False


def _check_lib():
    global _check_configured
    lib = _axh.load_library()
    if not _check_configured:
        c = ctypes
        vp, u32, dbl, rp = c.c_void_p, c.c_uint32, c.c_double, c.POINTER(_Report)
        lib.axh_check_last_error.restype = c.c_char_p
        lib.axh_check_q4k_matvec.argtypes = [vp, vp, vp, u32, u32, dbl, rp]
        lib.axh_check_q4_0_matvec.argtypes = [vp, vp, vp, u32, u32, dbl, rp]
        lib.axh_check_q4k_matmul_f16.argtypes = [vp, vp, vp, u32, u32, u32, dbl, rp]
        for f in ("axh_check_q4k_matvec", "axh_check_q4_0_matvec", "axh_check_q4k_matmul_f16"):
            getattr(lib, f).restype = c.c_int
        _check_configured = True
    return lib


def check_result(kernel: str, shape: dict, q, x, y, rel_tol: float = DEFAULT_REL_TOL) -> dict:
    """Host verdict for a device result (see include/axh_check.h)."""
    lib = _check_lib()
    rows, units = int(shape["n_rows"]), int(shape["units_per_row"])
    q = np.ascontiguousarray(q)
    x = np.ascontiguousarray(x)
    y = np.ascontiguousarray(y, dtype=np.float32)
    rep = _Report()
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    if kernel == "q4km_dequant_matvec":
        st = lib.axh_check_q4k_matvec(p(q), p(x), p(y), rows, units, rel_tol, ctypes.byref(rep))
    elif kernel == "q4_0_dequant_matvec":
        st = lib.axh_check_q4_0_matvec(p(q), p(x), p(y), rows, units, rel_tol, ctypes.byref(rep))
    else:
        st = lib.axh_check_q4k_matmul_f16(p(q), p(x), p(y), rows, units,
                                          int(shape.get("batch", 1)), rel_tol, ctypes.byref(rep))
    if st != 0:
        raise invalid(lib.axh_check_last_error().decode(errors="replace"))
    return {"ok": bool(rep.ok), "rows_checked": rep.rows_checked, "rows_failed": rep.rows_failed,
            "worst_row": rep.worst_row, "worst_over_allowed": rep.worst_over_allowed,
            "norm_rel_err": rep.norm_rel_err}


# ---- hole spaces ----------------------------------------------------------------
def default_holes(kernel: str, shape: Optional[dict] = None) -> list:
    """The kernel's hole space as a list of hole maps.  q4km_dequant_matvec:
    one map per kernel family that takes the shape (the autotuner's space,
    tune.q4k_matvec_hole_spaces); q4_0_dequant_matvec with a shape: the
    LDS-tiled kernel's map, then one map per other family that takes the shape
    (tune.q4_0_matvec_hole_spaces); otherwise one map of the candidate values
    of every hole among the compiled variants (sorted)."""
    if kernel == "q4km_dequant_matvec":
        from . import tune
        shape = shape or {"n_rows": 1, "units_per_row": 1}
        return tune.q4k_matvec_hole_spaces(int(shape["n_rows"]), int(shape["units_per_row"]))
    if kernel == "q4_0_dequant_matvec" and shape:
        from . import tune
        return tune.q4_0_matvec_hole_spaces(int(shape["n_rows"]), int(shape["units_per_row"]))
    if kernel == "q4k_matmul_f16":
        vs = [(v.kind, v.waves_per_workgroup, v.col_tiles, v.prefetch, v.row_tiles)
              for v in _axh.compiled_matmul_variants()]
        names = ("kind", "waves_per_workgroup", "col_tiles", "prefetch", "row_tiles")
    else:
        vs = [(v.rows_per_wave, v.waves_per_workgroup) for v in _axh.compiled_variants("q4_0")]
        names = ("rows_per_wave", "waves_per_workgroup")
    return [{n: sorted({v[i] for v in vs}) for i, n in enumerate(names)}]


def _variant_obj(kernel: str, a: dict):
    g = lambda k: int(a.get(k, 0))
    if kernel == "q4k_matmul_f16":
        return _axh.MatmulVariant(g("kind"), g("waves_per_workgroup"), g("col_tiles"),
                                  g("prefetch"), g("row_tiles"))
    return _axh.Variant(g("rows_per_wave"), g("waves_per_workgroup"), g("prefetch"),
                        g("nontemporal"), g("family"), g("sb_per_lane"))


def _enumerate_spaces(spaces: list) -> list:
    """Variants of every map in turn; ordinals continue across the maps."""
    from . import tune
    out = []
    for holes in spaces:
        for v in tune.enumerate_strategy(holes):
            out.append(tune.StrategyVariant(len(out), v.variant_id, v.assignments))
    return out


# ---- context ---------------------------------------------------------------------
@dataclass
class McpContext:
    history_dir: Path = field(default_factory=lambda: Path(".pipeline") / "history")
    git_sha: Optional[str] = None
    _hip: Any = None
    _unavailable: Optional[str] = None

    def __post_init__(self):
        if self.git_sha is None:
            self.git_sha = read_git_sha(Path.cwd())

    def hip(self):
        """Lazily created HIP context; a failure is cached (dispatch.rs:85-127)."""
        if self._hip is not None:
            return self._hip
        if self._unavailable is not None:
            raise McpToolError(DEVICE_UNAVAILABLE, "device_unavailable", self._unavailable)
        try:
            self._hip = _axh.HipContext.new()
        except Exception as e:  # no GPU, no library, ...
            self._unavailable = f"HIP device unavailable: {e}"
            raise McpToolError(DEVICE_UNAVAILABLE, "device_unavailable", self._unavailable)
        return self._hip

    def machine(self) -> dict:
        return {"device_name": self._hip.device_name if self._hip else "", "driver_version": 0,
                "api_version": 0, "physical_device_index": 0, "icd_path": None,
                "git_sha": self.git_sha}


# ---- tools -----------------------------------------------------------------------
def _kernel_and_shape(params: dict):
    kernel = params.get("kernel")
    if kernel not in KERNELS:
        raise invalid(f"kernel must be one of {list(KERNELS)}, got {kernel!r}")
    shape = params.get("shape") or {}
    try:
        rows, units = int(shape["n_rows"]), int(shape["units_per_row"])
    except (KeyError, TypeError, ValueError):
        raise invalid("shape needs integer n_rows and units_per_row")
    if rows < 1 or units < 1:
        raise invalid("n_rows and units_per_row must be >= 1")
    out = {"n_rows": rows, "units_per_row": units}
    if kernel == "q4k_matmul_f16":
        out["batch"] = int(shape.get("batch", 1))
        if out["batch"] < 1:
            raise invalid("batch must be >= 1")
    return kernel, out


def _holes(params: dict, kernel: str, shape: Optional[dict] = None) -> list:
    """`holes_override` REPLACES the kernel's hole space when present, even if
    empty (grid_search.rs:268-272): one map, or a list of maps; otherwise the
    kernel's default space."""
    h = params.get("holes_override")
    if h is None:
        return default_holes(kernel, shape)
    maps = h if isinstance(h, list) else [h]
    for m in maps:
        if not isinstance(m, dict) or not all(isinstance(v, list) for v in m.values()):
            raise invalid("holes_override must map hole names to lists of integers "
                          "(or be a list of such maps)")
    return [{k: [int(x) for x in v] for k, v in m.items()} for m in maps]


def enumerate_variants(params: dict, ctx: McpContext) -> dict:
    from . import tune
    kernel, shape = _kernel_and_shape({**params, "shape": params.get("shape") or
                                       {"n_rows": 1, "units_per_row": 1}})
    spaces = _holes(params, kernel, shape)
    try:
        vs = _enumerate_spaces(spaces)
    except tune.TuneError as e:
        raise McpToolError(ENUMERATE_ERROR, "enumerate_error", str(e))
    return {"variants": [{"ordinal": v.ordinal, "variant_id": v.variant_id,
                          "assignments": v.assignments} for v in vs],
            "count": len(vs)}


ROTATE_BYTES = 512 << 20


class _Workload:
    """One set of inputs on the device, the weights copied until the copies
    pass ROTATE_BYTES; launch(variant, i) runs call i on copy i mod n."""

    def __init__(self, hip, kernel: str, shape: dict, q, x):
        self.hip, self.kernel, self.shape, self.q, self.x = hip, kernel, shape, q, x
        self.rows, self.units = shape["n_rows"], shape["units_per_row"]
        self.batch = shape.get("batch", 1)
        self.stride = -(-max(q.nbytes, 16) // 256) * 256
        self.n = max(1, min(64, -(-ROTATE_BYTES // self.stride)))
        self.y_bytes = self.rows * self.batch * 4
        self.bufs = []
        try:
            self.w = hip.alloc(self.stride * self.n)
            self.bufs.append(self.w)
            for c in range(self.n):
                hip.upload(self.w.ptr + c * self.stride, q)
            self.dx = hip.alloc(max(x.nbytes, 16))
            self.bufs.append(self.dx)
            hip.upload(self.dx, x)
            self.dy = hip.alloc(self.y_bytes)
            self.bufs.append(self.dy)
        except Exception:
            self.close()
            raise

    def launch(self, variant, i: int = 0) -> None:
        w = self.w.ptr + (i % self.n) * self.stride
        if self.kernel == "q4km_dequant_matvec":
            self.hip.q4k_matvec(w, self.dx, self.dy, self.rows, self.units, variant)
        elif self.kernel == "q4_0_dequant_matvec":
            self.hip.q4_0_matvec(w, self.dx, self.dy, self.rows, self.units, variant)
        else:
            self.hip.q4k_matmul(w, self.dx, self.dy, self.rows, self.units, self.batch, variant)

    def run_once(self, variant) -> np.ndarray:
        """One call on copy 0 and its output (DispatchError if it cannot run)."""
        self.launch(variant, 0)
        self.hip.synchronize()
        return np.frombuffer(self.hip.download(self.dy, self.y_bytes), dtype=np.float32).copy()

    def sample_ns(self, variant, per: int, e0, e1) -> int:
        """Mean ns per call of `per` back-to-back calls over the copies."""
        for i in range(3):
            self.launch(variant, i)
        e0.record()
        for i in range(per):
            self.launch(variant, i)
        e1.record()
        e1.synchronize()
        return int(round(e0.elapsed_ms(e1) * 1e6 / per))

    def verdict(self, y, params: dict) -> dict:
        if params.get("correctness", "check") == "none":
            return {"status": "not_checked", "reason": "correctness policy `none`"}
        rep = check_result(self.kernel, self.shape, self.q, self.x, y,
                           float(params.get("rel_tol", DEFAULT_REL_TOL)))
        return {"status": "ok"} if rep["ok"] else {
            "status": "failed",
            "reason": f"{rep['rows_failed']} of {rep['rows_checked']} outputs outside tolerance; "
                      f"worst output {rep['worst_row']} at {rep['worst_over_allowed']:.3g} x "
                      f"allowed; norm error {rep['norm_rel_err']:.3g}"}

    def kernel_entry(self, variant) -> str:
        if self.kernel == "q4k_matmul_f16":
            return _axh.q4k_matmul_kernel_name(self.rows, self.units, self.batch, variant)
        if self.kernel == "q4km_dequant_matvec":
            return _axh.q4k_matvec_kernel_name(self.rows, self.units, variant)
        return _axh.q4_0_matvec_kernel_name(self.rows, self.units, variant)

    def close(self) -> None:
        for b in self.bufs:
            b.close()
        self.bufs = []


def bench_variant(params: dict, ctx: McpContext) -> dict:
    kernel, shape = _kernel_and_shape(params)
    samples_n = int(params.get("sample_count", 0))
    if samples_n < 1:
        raise invalid("sample_count must be >= 1")
    per = max(1, int(params.get("launches_per_sample", 10)))
    assignments = {k: int(v) for k, v in (params.get("assignments") or {}).items()}
    vid = variant_id(assignments)
    hip = ctx.hip()
    q, x = seeded_inputs(kernel, shape, vid)
    variant = _variant_obj(kernel, assignments)
    wl = _Workload(hip, kernel, shape, q, x)
    try:
        try:
            y = wl.run_once(variant)
        except _axh.DispatchError as e:
            raise McpToolError(DEVICE_UNAVAILABLE, "dispatch_failed", f"{e.variant}: {e}")
        e0, e1 = hip.event(), hip.event()
        samples = [wl.sample_ns(variant, per, e0, e1) for _ in range(samples_n)]
        verdict = wl.verdict(y, params)
        name = wl.kernel_entry(variant)
        copies = wl.n
    finally:
        wl.close()
    srt = sorted(samples)
    return {"median_ns": srt[len(srt) // 2], "samples": samples, "correctness": verdict,
            "machine": ctx.machine(), "kernel_entry": name, "variant_id": vid,
            "weight_copies": copies}


def grid_search(params: dict, ctx: McpContext) -> dict:
    """The reference's grid search (grid_search.rs:158-283) over the kernel's
    hole space: every variant runs once and is judged, then the accepted ones
    are timed in `sample_count` interleaved rounds of `launches_per_sample`
    calls each; the winner has the lowest median (ties: lowest ordinal)."""
    from . import tune
    kernel, shape = _kernel_and_shape(params)
    sample_count = int(params.get("sample_count", 5))
    if sample_count < 1:
        raise invalid("sample_count must be >= 1")
    per = max(1, int(params.get("launches_per_sample", 10)))
    spaces = _holes(params, kernel, shape)
    try:
        variants = _enumerate_spaces(spaces)
    except tune.TuneError as e:
        raise McpToolError(ENUMERATE_ERROR, "enumerate_error", str(e))
    if not variants:
        raise McpToolError(ENUMERATE_ERROR, "enumerate_error", "the hole space is empty")
    warnings = []
    if len(variants) > CARTESIAN_WARN_THRESHOLD:
        warnings.append(f"Cartesian product ({len(variants)}) exceeds CARTESIAN_WARN_THRESHOLD "
                        f"({CARTESIAN_WARN_THRESHOLD}); search may take a long time")
    hip = ctx.hip()
    key = source_key(kernel, shape)
    # one input set for the whole search, seeded by the source key
    q, x = seeded_inputs(kernel, shape, tune.xxh3_64(key.encode()))
    wl = _Workload(hip, kernel, shape, q, x)
    ranked, timed = [], []
    try:
        for v in variants:
            variant = _variant_obj(kernel, v.assignments)
            row = {"ordinal": v.ordinal, "variant_id": v.variant_id,
                   "assignments": v.assignments, "median_ns": None}
            try:
                y = wl.run_once(variant)
            except _axh.DispatchError as e:
                row.update(correctness={"status": "not_checked", "reason": str(e)},
                           outcome=f"failed: {e.variant}: {e}")
                ranked.append(row)
                continue
            verdict = wl.verdict(y, params)
            row["correctness"] = verdict
            row["kernel_entry"] = wl.kernel_entry(variant)
            if verdict["status"] == "failed":
                row["outcome"] = f"correctness_rejected: {verdict['reason']}"
            else:
                row["outcome"] = "ok" if verdict["status"] == "ok" else "not_checked"
                row["samples"] = []
                timed.append((row, variant))
            ranked.append(row)
        e0, e1 = hip.event(), hip.event()
        for _ in range(sample_count):  # interleaved rounds
            for row, variant in timed:
                row["samples"].append(wl.sample_ns(variant, per, e0, e1))
        for row, _ in timed:
            srt = sorted(row["samples"])
            row["median_ns"] = srt[len(srt) // 2]
        copies = wl.n
    finally:
        wl.close()
    ranked.sort(key=lambda r: (r["median_ns"] is None, r["median_ns"] or 0, r["ordinal"]))
    win = next((r for r in ranked if r["median_ns"] is not None), ranked[0])
    fallback = win["median_ns"] is None
    from . import tune as _t
    path = history_path(ctx.history_dir, key)
    win_ns = win["median_ns"] if win["median_ns"] is not None else 2 ** 64 - 1
    entry = {"timestamp": format_rfc3339_utc(), "git_sha": ctx.git_sha,
             "source_xxh3": hex16(_t.xxh3_64(key.encode())),
             "grid_search": {"winner_variant_id": win["variant_id"],
                             "winner_assignments": win["assignments"],
                             "winner_median_ns": win_ns, "ranked": ranked,
                             "machine": ctx.machine()}}
    try:
        append_history_entry(path, entry)
    except OSError as e:
        raise McpToolError(IO_ERROR, "io_error", str(e))
    return {"winner": {"ordinal": win["ordinal"], "variant_id": win["variant_id"],
                       "assignments": win["assignments"],
                       "kernel_entry": win.get("kernel_entry")},
            "winner_median_ns": win_ns, "ranked": ranked, "fallback_used": fallback,
            "warnings": warnings, "history_path": str(path), "machine": ctx.machine(),
            "weight_copies": copies}


def optimization_history(params: dict, ctx: McpContext) -> dict:
    kernel, shape = _kernel_and_shape(params)
    path = history_path(ctx.history_dir, source_key(kernel, shape))
    entries = []
    if path.is_file():
        try:
            for ln in path.read_text(encoding="utf-8").splitlines():
                if ln.strip():
                    entries.append(json.loads(ln))
        except (OSError, ValueError) as e:
            raise McpToolError(IO_ERROR, "io_error", str(e))
    limit = params.get("limit")
    if limit is not None:
        entries = entries[-int(limit):]
    return {"history_path": str(path), "entries": entries}


def _initialize(params: dict, ctx: McpContext) -> dict:
    return {"server": "axiom-compute_amd", "protocol": "jsonrpc-2.0", "methods": list(METHODS),
            "kernels": list(KERNELS)}


_HANDLERS = {"initialize": _initialize, "enumerate_variants": enumerate_variants,
             "bench_variant": bench_variant, "grid_search": grid_search,
             "optimization_history": optimization_history}


# ---- JSON-RPC 2.0 --------------------------------------------------------------------
def handle_line(line: str, ctx: McpContext) -> Optional[dict]:
    """One request line -> one response object, or None for a notification."""
    try:
        env = json.loads(line)
    except ValueError as e:
        return {"jsonrpc": "2.0", "id": None,
                "error": {"code": PARSE_ERROR, "message": f"parse error: {e}"}}
    if not isinstance(env, dict) or env.get("jsonrpc") != "2.0" or \
            not isinstance(env.get("method"), str):
        return {"jsonrpc": "2.0", "id": env.get("id") if isinstance(env, dict) else None,
                "error": {"code": INVALID_REQUEST, "message": "invalid request"}}
    notification = "id" not in env
    rid = env.get("id")
    method = env["method"]
    params = env.get("params") or {}
    if method not in _HANDLERS:
        resp = {"jsonrpc": "2.0", "id": rid,
                "error": {"code": METHOD_NOT_FOUND, "message": f"method not found: {method}",
                          "data": {"category": "method_not_found", "available": list(METHODS)}}}
    elif not isinstance(params, dict):
        resp = {"jsonrpc": "2.0", "id": rid,
                "error": invalid("params must be an object").rpc()}
    else:
        try:
            resp = {"jsonrpc": "2.0", "id": rid, "result": _HANDLERS[method](params, ctx)}
        except McpToolError as e:
            resp = {"jsonrpc": "2.0", "id": rid, "error": e.rpc()}
        except Exception as e:  # keep serving
            resp = {"jsonrpc": "2.0", "id": rid,
                    "error": McpToolError(INTERNAL_ERROR, "internal_error", repr(e)).rpc()}
    return None if notification else resp


def serve(inp=None, out=None, ctx: Optional[McpContext] = None) -> None:
    """Line-delimited JSON-RPC 2.0 over stdio until EOF."""
    inp = inp or sys.stdin
    out = out or sys.stdout
    ctx = ctx or McpContext(history_dir=Path(os.environ.get("AXH_HISTORY_DIR",
                                                            ".pipeline/history")))
    for line in inp:
        if not line.strip():
            continue
        resp = handle_line(line, ctx)
        if resp is not None:
            out.write(json.dumps(resp) + "\n")
            out.flush()


if __name__ == "__main__":
    serve()
