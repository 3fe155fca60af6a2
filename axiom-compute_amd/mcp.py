"""Tuning tools for LLM-driven search over the HIP kernels' strategy holes.

Mirrors the reference's MCP tool surface (crates/axc-driver/src/mcp/):
JSON-RPC 2.0 over stdio (dispatch.rs), `enumerate_variants`, `bench_variant`
(tools/bench_variant.rs) and `grid_search` (tools/grid_search.rs) with the
JSONL optimisation history, and `optimization_history`.  Where the reference
compiles `.axc` source with `@strategy` holes, the kernels here are the
library's compiled Q4 operations, named like the reference kernels:

  q4km_dequant_matvec  holes rows_per_wave, waves_per_workgroup, prefetch, nontemporal
  q4_0_dequant_matvec  holes rows_per_wave, waves_per_workgroup
  q4k_matmul_f16       holes kind, waves_per_workgroup, col_tiles, prefetch, row_tiles

and a request names a shape ({"n_rows", "units_per_row", "batch"}) instead of
input byte sizes.  Correctness is a real verdict for every kernel (the
reference reports its Q4 kernel "not_checked", bench_variant.rs:395-400):
the device result is compared with an f64 accumulation of the reference's
dequantised weights by the library's host checker (include/axh_check.h).

Timing samples are HIP-event times on resident buffers (each sample the mean
of `launches_per_sample` back-to-back launches), not host round trips.
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
def default_holes(kernel: str) -> dict:
    """Candidate values of every hole, from the compiled variants (sorted)."""
    if kernel == "q4k_matmul_f16":
        vs = [(v.kind, v.waves_per_workgroup, v.col_tiles, v.prefetch, v.row_tiles)
              for v in _axh.compiled_matmul_variants()]
        names = ("kind", "waves_per_workgroup", "col_tiles", "prefetch", "row_tiles")
    else:
        kind = "q4k" if kernel == "q4km_dequant_matvec" else "q4_0"
        vs = [(v.rows_per_wave, v.waves_per_workgroup, v.prefetch, v.nontemporal)
              for v in _axh.compiled_variants(kind)]
        names = ("rows_per_wave", "waves_per_workgroup", "prefetch", "nontemporal")
        if kind == "q4_0":
            names, vs = names[:2], [v[:2] for v in vs]
    return {n: sorted({v[i] for v in vs}) for i, n in enumerate(names)}


def _variant_obj(kernel: str, a: dict):
    g = lambda k: int(a.get(k, 0))
    if kernel == "q4k_matmul_f16":
        return _axh.MatmulVariant(g("kind"), g("waves_per_workgroup"), g("col_tiles"),
                                  g("prefetch"), g("row_tiles"))
    return _axh.Variant(g("rows_per_wave"), g("waves_per_workgroup"), g("prefetch"),
                        g("nontemporal"))


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


def _holes(params: dict, kernel: str) -> dict:
    """`holes_override` REPLACES the kernel's hole map when present, even if
    empty (grid_search.rs:268-272); otherwise the compiled hole space."""
    h = params.get("holes_override")
    if h is None:
        return default_holes(kernel)
    if not isinstance(h, dict) or not all(isinstance(v, list) for v in h.values()):
        raise invalid("holes_override must map hole names to lists of integers")
    return {k: [int(x) for x in v] for k, v in h.items()}


def enumerate_variants(params: dict, ctx: McpContext) -> dict:
    from . import tune
    kernel, _ = _kernel_and_shape({**params, "shape": params.get("shape") or
                                   {"n_rows": 1, "units_per_row": 1}})
    holes = _holes(params, kernel)
    try:
        vs = tune.enumerate_strategy(holes)
    except tune.TuneError as e:
        raise McpToolError(ENUMERATE_ERROR, "enumerate_error", str(e))
    return {"variants": [{"ordinal": v.ordinal, "variant_id": v.variant_id,
                          "assignments": v.assignments} for v in vs],
            "count": len(vs)}


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
    rows, units = shape["n_rows"], shape["units_per_row"]
    batch = shape.get("batch", 1)
    variant = _variant_obj(kernel, assignments)
    y_bytes = rows * batch * 4
    bufs = [hip.alloc(max(q.nbytes, 16)), hip.alloc(max(x.nbytes, 16)), hip.alloc(y_bytes)]
    try:
        hip.upload(bufs[0], q)
        hip.upload(bufs[1], x)

        def launch():
            if kernel == "q4km_dequant_matvec":
                hip.q4k_matvec(bufs[0], bufs[1], bufs[2], rows, units, variant)
            elif kernel == "q4_0_dequant_matvec":
                hip.q4_0_matvec(bufs[0], bufs[1], bufs[2], rows, units, variant)
            else:
                hip.q4k_matmul(bufs[0], bufs[1], bufs[2], rows, units, batch, variant)

        try:
            launch()
            hip.synchronize()
        except _axh.DispatchError as e:
            raise McpToolError(DEVICE_UNAVAILABLE, "dispatch_failed",
                               f"{e.variant}: {e}")
        y = np.frombuffer(hip.download(bufs[2], y_bytes), dtype=np.float32).copy()
        samples = []
        e0, e1 = hip.event(), hip.event()
        for _ in range(samples_n):
            e0.record()
            for _ in range(per):
                launch()
            e1.record()
            e1.synchronize()
            samples.append(int(round(e0.elapsed_ms(e1) * 1e6 / per)))
    finally:
        for b in bufs:
            b.close()
    if params.get("correctness", "check") == "none":
        verdict = {"status": "not_checked", "reason": "correctness policy `none`"}
    else:
        rep = check_result(kernel, shape, q, x, y, float(params.get("rel_tol", DEFAULT_REL_TOL)))
        verdict = {"status": "ok"} if rep["ok"] else {
            "status": "failed",
            "reason": f"{rep['rows_failed']} of {rep['rows_checked']} outputs outside tolerance; "
                      f"worst output {rep['worst_row']} at {rep['worst_over_allowed']:.3g} x allowed; "
                      f"norm error {rep['norm_rel_err']:.3g}"}
    srt = sorted(samples)
    name = (_axh.q4k_matmul_kernel_name(rows, units, batch, variant)
            if kernel == "q4k_matmul_f16" else
            _axh.q4k_matvec_kernel_name(rows, units, variant)
            if kernel == "q4km_dequant_matvec" else
            _axh.q4_0_matvec_kernel_name(rows, units, variant))
    return {"median_ns": srt[len(srt) // 2], "samples": samples, "correctness": verdict,
            "machine": ctx.machine(), "kernel_entry": name, "variant_id": vid}


def grid_search(params: dict, ctx: McpContext) -> dict:
    from . import tune
    kernel, shape = _kernel_and_shape(params)
    sample_count = int(params.get("sample_count", 5))
    if sample_count < 1:
        raise invalid("sample_count must be >= 1")
    holes = _holes(params, kernel)
    try:
        variants = tune.enumerate_strategy(holes)
    except tune.TuneError as e:
        raise McpToolError(ENUMERATE_ERROR, "enumerate_error", str(e))
    warnings = []
    if len(variants) > CARTESIAN_WARN_THRESHOLD:
        warnings.append(f"Cartesian product ({len(variants)}) exceeds CARTESIAN_WARN_THRESHOLD "
                        f"({CARTESIAN_WARN_THRESHOLD}); search may take a long time")
    ctx.hip()
    ranked = []
    for v in variants:
        req = {"kernel": kernel, "shape": shape, "assignments": v.assignments,
               "sample_count": sample_count, "correctness": params.get("correctness", "check"),
               "launches_per_sample": params.get("launches_per_sample", 10)}
        try:
            r = bench_variant(req, ctx)
            st = r["correctness"]["status"]
            outcome = ("ok" if st == "ok" else "not_checked" if st == "not_checked" else
                       f"correctness_rejected: {r['correctness']['reason']}")
            median = None if st == "failed" else r["median_ns"]
            ranked.append({"ordinal": v.ordinal, "variant_id": v.variant_id,
                           "assignments": v.assignments, "median_ns": median,
                           "correctness": r["correctness"], "outcome": outcome})
        except McpToolError as e:
            ranked.append({"ordinal": v.ordinal, "variant_id": v.variant_id,
                           "assignments": v.assignments, "median_ns": None,
                           "correctness": {"status": "not_checked", "reason": e.message},
                           "outcome": f"failed: {e.message}"})
    ranked.sort(key=lambda r: (r["median_ns"] is None, r["median_ns"] or 0, r["ordinal"]))
    win = next((r for r in ranked if r["median_ns"] is not None), ranked[0])
    fallback = win["median_ns"] is None
    key = source_key(kernel, shape)
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
                       "assignments": win["assignments"]},
            "winner_median_ns": win_ns, "ranked": ranked, "fallback_used": fallback,
            "warnings": warnings, "history_path": str(path), "machine": ctx.machine()}


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
