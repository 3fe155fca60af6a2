"""Benchmark of the MI355X Q4_0 / Q4_K_M dequant-matvec hot path.

Default (the headline metric): one step = one Q4_K_M matvec of the
4096 x 14336 down-projection over weights already
resident in HBM.  Weights rotate over enough distinct copies (> 512 MiB)
that every call reads HBM instead of the 256 MiB Infinity Cache.  Prints ONE
JSON line.  Other BASELINE configs are measured with --workload:

  c1    Q4_0 matvec 256 x 4096                 (GB/s of weights)
  c2    Q4_K matvec 1 x 32768                  (GB/s of weights)
  c3    Q4_K matvec 4096 x 4096
  c3b   Q4_K matvec 14336 x 4096
  c4    Q4_K matvec 4096 x 14336               (default)
  head  Q4_K matvec 128256 x 4096              (output head)
  c5    Q4_K matmul 14336 x 4096, --batch B    (f16 activations; GB/s for B <= 32,
                                                TFLOP/s for larger B)
  down  Q4_K matmul 4096 x 14336, --batch B    (the c4 weights against B activation
                                                vectors: batched decode; not a config)

  python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--workload c4] [--batch 128]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0        # MI355X published HBM3E bandwidth
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16 MFMA
COPIES_MIN_BYTES = 512 << 20
COPY_ALIGN = 256

# name: (kind, rows, units per row, x sigma, config label)
WORKLOADS = {
    "c1": ("q4_0", 256, 128, 1.0, "BASELINE config 1"),
    "c2": ("q4k", 1, 128, 1.0, "BASELINE config 2"),
    "c3": ("q4k", 4096, 16, 1.0, "BASELINE config 3"),
    "c3b": ("q4k", 14336, 16, 1.0, "BASELINE config 3"),
    "c4": ("q4k", 4096, 56, 0.5, "BASELINE config 4, down-projection"),
    "head": ("q4k", 128256, 16, 1.0, "BASELINE config 4, output head"),
    "c5": ("matmul", 14336, 16, 1.0, "BASELINE config 5"),
    # the c4 down-projection against several activation vectors (batched decode)
    "down": ("matmul", 4096, 56, 1.0, "Llama-3-8B ffn_down batched, not a BASELINE config"),
    # fused SwiGLU gate/up projections of a Llama-3-8B decode step (two
    # 14336 x 4096 Q4_K_M matrices against one x)
    "ffn": ("gate_up", 14336, 16, 0.5, "Llama-3-8B gate/up, not a BASELINE config"),
    # ggml k-quants that Q4_K_M / Q5_K_M checkpoints store next to Q4_K
    "head6": ("q6k", 128256, 16, 1.0, "Llama-3-8B output head as Q4_K_M stores it (Q6_K), "
                                        "not a BASELINE config"),
    "down6": ("q6k", 4096, 56, 0.5, "Llama-3-8B ffn_down as Q6_K, not a BASELINE config"),
    "v6": ("q6k", 1024, 16, 1.0, "Llama-3-8B attn_v (8 KV heads) as Q6_K, not a BASELINE config"),
    "up5": ("q5k", 14336, 16, 1.0, "Llama-3-8B ffn_up as Q5_K, not a BASELINE config"),
    # Q4_0 checkpoints store every projection in it: the same shapes as Q4_0
    "down0": ("q4_0", 4096, 448, 0.5, "Llama-3-8B ffn_down as Q4_0, not a BASELINE config"),
    "head0": ("q4_0", 128256, 128, 1.0, "Llama-3-8B output head as Q4_0, not a BASELINE config"),
    "ffn0": ("gate_up0", 14336, 128, 0.5, "Llama-3-8B gate/up as Q4_0, not a BASELINE config"),
    "ffn5": ("gate_up5", 14336, 16, 0.5, "Llama-3-8B gate/up as Q5_K, not a BASELINE config"),
}
GATE_UP_KINDS = ("gate_up", "gate_up0", "gate_up5")
KQ_IDS = {"q5k": 13, "q6k": 14}


def cpu_model() -> str:
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _time_cpu(fn, budget_s: float):
    fn()  # warm caches / page in
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            return n, el


def profiled_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` at `workload`, as recorded by the
    FETCH_SIZE / WRITE_SIZE counter summary under profiles/ (None if that
    kernel has no recorded summary)."""
    pat = re.compile(r"^traffic_per_launch kernel=(\S+) workload=(\S+) bytes=(\d+) "
                     r"source=(\S+)")
    for f in sorted((ROOT / "profiles").glob("*.md")):
        for ln in f.read_text().splitlines():
            m = pat.match(ln.strip().strip("`"))
            if m and m.group(1) == kernel and m.group(2) == workload:
                return int(m.group(3)), f"profiles/{f.name}"
    return None, None


def profiled_mfma_busy(kernel: str, workload: str):
    """Fraction of the dispatch's cycles the MFMA units were busy, summed over
    every SIMD (SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x SIMDs)), as
    recorded by the counter summary under profiles/ (None if absent)."""
    pat = re.compile(r"^mfma_busy kernel=(\S+) workload=(\S+) frac=([0-9.]+) source=(\S+)")
    for f in sorted((ROOT / "profiles").glob("*.md")):
        for ln in f.read_text().splitlines():
            m = pat.match(ln.strip().strip("`"))
            if m and m.group(1) == kernel and m.group(2) == workload:
                return float(m.group(3)), f"profiles/{f.name}"
    return None, None


class Case:
    """One workload: device buffers, the launch of step i, parity, CPU baseline."""

    def __init__(self, pkg, O, np, ctx, name, batch, variant, x_f32=False):
        kind, rows, units, sigma, label = WORKLOADS[name]
        self.kind, self.rows, self.units, self.label = kind, rows, units, label
        self.ctx, self.O, self.np, self.pkg = ctx, O, np, pkg
        self.batch = batch if kind == "matmul" else 1
        unit_bytes = {"q4_0": 18, "gate_up0": 18, "q5k": 176, "gate_up5": 176,
                      "q6k": 210}.get(kind, 144)
        self.cols = units * (32 if kind in ("q4_0", "gate_up0") else 256)
        self.weight_bytes = rows * units * unit_bytes
        seed = 20241 if name == "c4" else 30000 + rows + units
        self.up_off = 0
        if kind == "q4_0":
            self.q = O.gen_q4_0_weights(seed, rows * units)
        elif kind in KQ_IDS:
            self.q = O.gen_kq_weights(KQ_IDS[kind], seed, rows * units)
        elif kind in GATE_UP_KINDS:
            # gate rows, then the up rows at the next COPY_ALIGN boundary
            gen = {"gate_up": O.gen_q4k_weights, "gate_up0": O.gen_q4_0_weights,
                   "gate_up5": lambda sd, n: O.gen_kq_weights(KQ_IDS["q5k"], sd, n)}[kind]
            self.qg = gen(seed, rows * units)
            self.qu = gen(seed + 7, rows * units)
            self.up_off = -(-self.weight_bytes // COPY_ALIGN) * COPY_ALIGN
            self.q = np.zeros(self.up_off + self.weight_bytes, dtype=np.uint8)
            self.q[: self.weight_bytes] = self.qg
            self.q[self.up_off:] = self.qu
            self.weight_bytes *= 2
        else:
            self.q = O.gen_q4k_weights(seed, rows * units)
        self.x_f32 = kind == "matmul" and x_f32
        if kind == "matmul":
            self.x = O.gen_normal_f32(seed + 1, self.cols * self.batch, sigma)
            if not self.x_f32:
                self.x = self.x.astype(np.float16)
            self.y_bytes = self.batch * rows * 4
        else:
            self.x = O.gen_normal_f32(seed + 1, self.cols, sigma)
            self.y_bytes = rows * 4
        self.variant = variant
        stride = -(-self.q.nbytes // COPY_ALIGN) * COPY_ALIGN
        self.n_copies = max(2, -(-COPIES_MIN_BYTES // stride))
        self.stride = stride
        # tail room of x's size: the weights-and-x read floor reads weight + x
        # bytes from the last copy
        self.wbuf = ctx.alloc(stride * self.n_copies + self.x.nbytes + COPY_ALIGN)
        one = np.zeros(stride, dtype=np.uint8)
        one[: self.q.nbytes] = self.q
        ctx.upload(self.wbuf, np.tile(one, self.n_copies))
        self.dx = ctx.alloc(self.x.nbytes)
        ctx.upload(self.dx, self.x)
        self.dy = ctx.alloc(self.y_bytes)
        self.dx16 = ctx.alloc(self.x.size * 2) if self.x_f32 else None

    def launch(self, i: int) -> None:
        w = self.wbuf.ptr + (i % self.n_copies) * self.stride
        if self.kind == "q4k":
            self.ctx.q4k_matvec(w, self.dx, self.dy, self.rows, self.units, self.variant)
        elif self.kind == "q4_0":
            self.ctx.q4_0_matvec(w, self.dx, self.dy, self.rows, self.units, self.variant)
        elif self.kind == "q5k":
            self.ctx.q5k_matvec(w, self.dx, self.dy, self.rows, self.units, self.variant)
        elif self.kind == "q6k":
            self.ctx.q6k_matvec(w, self.dx, self.dy, self.rows, self.units, self.variant)
        elif self.kind == "gate_up":
            self.ctx.q4k_gate_up(w, w + self.up_off, self.dx, self.dy, self.rows, self.units,
                                 self.variant)
        elif self.kind == "gate_up0":
            self.ctx.q4_0_gate_up(w, w + self.up_off, self.dx, self.dy, self.rows, self.units,
                                  self.variant)
        elif self.kind == "gate_up5":
            self.ctx.q5k_gate_up(w, w + self.up_off, self.dx, self.dy, self.rows, self.units,
                                 self.variant)
        elif self.x_f32:
            self.ctx.q4k_matmul_f32(w, self.dx, self.dx16, self.dy, self.rows, self.units,
                                    self.batch, self.variant)
        else:
            self.ctx.q4k_matmul(w, self.dx, self.dy, self.rows, self.units, self.batch,
                                self.variant)

    def bench_op(self) -> dict:
        """Arguments of ctx.bench_loop for this workload (call i reads copy i)."""
        op = {"q4k": "q4k", "q4_0": "q4_0", "q5k": "q5k", "q6k": "q6k",
              "gate_up": "gate_up", "gate_up0": "gate_up_q4_0",
              "gate_up5": "gate_up_q5k"}.get(self.kind)
        if op is None:
            op = "matmul_f32" if self.x_f32 else "matmul_f16"
        return dict(op=op, q=self.wbuf, q_stride=self.stride, n_copies=self.n_copies, x=self.dx,
                    y=self.dy, n_rows=self.rows, units=self.units, batch=self.batch,
                    variant=self.variant, q2_offset=self.up_off, x16=self.dx16)

    def kernel(self) -> str:
        if self.kind == "q4k":
            return self.pkg.q4k_matvec_kernel_name(self.rows, self.units, self.variant)
        if self.kind == "q4_0":
            return self.pkg.q4_0_matvec_kernel_name(self.rows, self.units, self.variant)
        if self.kind == "gate_up":
            return self.pkg.q4k_gate_up_kernel_name(self.rows, self.units, self.variant)
        if self.kind == "gate_up0":
            return self.pkg.q4_0_gate_up_kernel_name(self.rows, self.units, self.variant)
        if self.kind == "gate_up5":
            return self.pkg.q5k_gate_up_kernel_name(self.rows, self.units, self.variant)
        if self.kind == "q5k":
            return self.pkg.q5k_matvec_kernel_name(self.rows, self.units, self.variant)
        if self.kind == "q6k":
            return self.pkg.q6k_matvec_kernel_name(self.rows, self.units, self.variant)
        return self.pkg.q4k_matmul_kernel_name(self.rows, self.units, self.batch, self.variant)

    def parity(self) -> dict:
        """Checks this exact workload against the oracle before timing."""
        np, O = self.np, self.O
        self.launch(0)
        self.ctx.synchronize()
        y = np.frombuffer(self.ctx.download(self.dy, self.y_bytes), dtype=np.float32)
        if self.kind == "q4k":
            ref = O.q4k_matvec(self.q, self.x, self.rows, self.units)
            yf, ad = O.q4k_matvec_f64(self.q, self.x, self.rows, self.units)
            rep = O.matvec_tolerance_report(y, ref, yf, ad, self.cols)
            return {k: rep[k] for k in ("ok", "rows_failed", "norm_rel_err",
                                        "gpu_err_vs_f64_norm", "cpu_err_vs_f64_norm")}
        if self.kind == "q4_0":
            ref = O.q4_0_matvec(self.q, self.x, self.rows, self.units)
            yf, ad = O.q4_0_matvec_f64(self.q, self.x, self.rows, self.units)
            rep = O.matvec_tolerance_report(y, ref, yf, ad, self.cols)
            return {k: rep[k] for k in ("ok", "rows_failed", "norm_rel_err",
                                        "gpu_err_vs_f64_norm", "cpu_err_vs_f64_norm")}
        if self.kind in KQ_IDS:
            kid = KQ_IDS[self.kind]
            ref = O.kq_matvec(kid, self.q, self.x, self.rows, self.units)
            yf, ad = O.kq_matvec_f64(kid, self.q, self.x, self.rows, self.units)
            rep = O.matvec_tolerance_report(y, ref, yf, ad, self.cols)
            return {k: rep[k] for k in ("ok", "rows_failed", "norm_rel_err",
                                        "gpu_err_vs_f64_norm", "cpu_err_vs_f64_norm")}
        if self.kind in GATE_UP_KINDS:
            f64 = {"gate_up": O.q4k_gate_up_f64, "gate_up0": O.q4_0_gate_up_f64,
                   "gate_up5": lambda *a: O.kq_gate_up_f64(KQ_IDS["q5k"], *a)}[self.kind]
            _, g, ag, u, au = f64(self.qg, self.qu, self.x, self.rows, self.units)
            rep = O.gate_up_tolerance_report(y, g, ag, u, au, self.cols)
            return {k: rep[k] for k in ("ok", "rows_failed", "worst_over_bound", "norm_rel_err")}
        # batched: against the f64 product of the same RN_f16 weights
        w16 = O.q4k_dequant(self.q, self.rows * self.units).reshape(self.rows, self.cols)
        w16 = w16.astype(np.float16).astype(np.float64)
        xf = self.x.astype(np.float16).astype(np.float64).reshape(self.batch, self.cols)
        ref = xf @ w16.T
        yy = y.reshape(self.batch, self.rows)
        err = float(np.linalg.norm(yy - ref) / max(np.linalg.norm(ref), 1e-30))
        return {"ok": err <= 1e-5, "norm_rel_err_vs_f16_weight_f64": err}

    def flops(self) -> float:
        return 2.0 * self.rows * self.cols * self.batch

    def cpu_baseline(self, budget_s: float, unit: str) -> dict:
        """The oracle (scalar C restatement of the reference's CPU function, its
        order) on this workload for about `budget_s` seconds on one core, then
        row-parallel on the host's cores for a quarter of that.  The batched
        case times a slice of rows (rows are independent) and scales up."""
        O = self.O
        threads = max(1, min(os.cpu_count() or 1, 16))
        if self.kind == "q4k":
            one = lambda: O.q4k_matvec_single(self.q, self.x, self.rows, self.units)
            many = lambda: O.q4k_matvec(self.q, self.x, self.rows, self.units, threads=threads)
            frac, what = 1.0, f"full {self.rows}x{self.cols} Q4_K matvecs"
        elif self.kind in KQ_IDS:
            kid = KQ_IDS[self.kind]
            one = lambda: O.kq_matvec(kid, self.q, self.x, self.rows, self.units, threads=1)
            many = lambda: O.kq_matvec(kid, self.q, self.x, self.rows, self.units,
                                       threads=threads)
            frac, what = 1.0, f"full {self.rows}x{self.cols} {self.kind.upper()} matvecs"
        elif self.kind in GATE_UP_KINDS:
            mv = {"gate_up": O.q4k_matvec, "gate_up0": O.q4_0_matvec,
                  "gate_up5": lambda *a, **k: O.kq_matvec(KQ_IDS["q5k"], *a, **k)}[self.kind]
            fmt = {"gate_up": "Q4_K", "gate_up0": "Q4_0", "gate_up5": "Q5_K"}[self.kind]

            def two(threads):
                g = mv(self.qg, self.x, self.rows, self.units, threads=threads)
                u = mv(self.qu, self.x, self.rows, self.units, threads=threads)
                return O.silu(g) * u

            one = lambda: two(1)
            many = lambda: two(threads)
            frac, what = 1.0, f"gate+up {self.rows}x{self.cols} {fmt} matvec pairs + silu*mul"
        elif self.kind == "q4_0":
            one = lambda: O.q4_0_matvec(self.q, self.x, self.rows, self.units, threads=1)
            many = lambda: O.q4_0_matvec(self.q, self.x, self.rows, self.units, threads=threads)
            frac, what = 1.0, f"full {self.rows}x{self.cols} Q4_0 matvecs"
        else:
            sl = max(1, min(self.rows, 16384 // self.batch))
            qs = self.q[: sl * self.units * 144]
            xb = self.x.astype(self.np.float16).view(self.np.uint16)
            one = lambda: O.q4k_matmul_f16x(qs, xb, sl, self.units, self.batch, threads=1)
            many = lambda: O.q4k_matmul_f16x(qs, xb, sl, self.units, self.batch,
                                             threads=threads)
            frac = sl / self.rows
            what = f"{sl}-row slices (of {self.rows}) of the B={self.batch} matmul"
        n, el = _time_cpu(one, budget_s)
        nm, elm = _time_cpu(many, max(1.0, budget_s / 4))
        per_call, per_call_m = el / n / frac, elm / nm / frac

        def rate(t):
            if unit == "TFLOP/s":
                return round(self.flops() / t / 1e12, 6)
            return round(self.weight_bytes / t / 1e9, 4)

        return {
            "value": rate(per_call), "unit": unit, "cores": 1, "kind": "port",
            "sample": f"{n} {what} in {el:.1f}s, one thread ({cpu_model()}, "
                      f"nproc={os.cpu_count()}); {per_call * 1e6:.0f} us per full call",
            "all_cores": {
                "value": rate(per_call_m), "cores": threads,
                "sample": f"{nm} in {elm:.1f}s over {threads} threads (bit-identical per row); "
                          f"{per_call_m * 1e6:.0f} us per full call",
            },
        }

    def close(self) -> None:
        for b in (self.wbuf, self.dx, self.dy, self.dx16):
            if b is not None:
                b.close()


def parse_variant(pkg, kind: str, text: str):
    if not text:
        return None
    vals = [int(t) for t in text.split(",")]
    return pkg.MatmulVariant(*vals) if kind == "matmul" else pkg.Variant(*vals)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c4", choices=sorted(WORKLOADS))
    ap.add_argument("--batch", type=int, default=128, help="activation vectors (c5 and down only)")
    ap.add_argument("--x-f32", action="store_true",
                    help="c5 only: f32 activations (cast to f16 by a separate pass, then the "
                         "f16 matmul; both timed)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--variant", default="",
                    help="matvec: rows_per_wave,waves,prefetch[,nontemporal[,family,sb_per_lane]]; "
                         "c5: kind,waves,col_tiles,prefetch")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run device-to-device copies of the weight size (counter calibration)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build runs the matvec on one MI355X "
              "(across GPUs the rows would be split into contiguous blocks, one per GPU, with "
              "x replicated and no collective until the consumer of y).", file=sys.stderr)
        return 2

    import numpy as np

    import __graft_entry__
    from oracle import oracle as O

    pkg = __graft_entry__.load_package()
    kind = WORKLOADS[args.workload][0]
    variant = parse_variant(pkg, kind, args.variant)
    ctx = pkg.HipContext.new()
    case = Case(pkg, O, np, ctx, args.workload, args.batch, variant, args.x_f32)

    par = case.parity()
    if not par["ok"]:
        print(json.dumps({"error": "parity failure", "report": par}), file=sys.stderr)
        return 1

    # Timed region (the reported value): K back-to-back calls of the operation
    # launched by the library's own loop (axh_bench_loop) on the context
    # stream through the public entry point, between exactly two HIP events on
    # that stream, with device synchronisation on both sides.  The W warmup
    # calls are queued right before the first event (no synchronisation in
    # between), so the first timed call starts behind queued work like the
    # others.  The spread (p10/p50/p90) comes from REPEATS more runs of the
    # same W + K loop, each between its own two events.  The same K calls
    # launched from this Python loop through ctypes, and replayed from one
    # captured HIP graph, are reported next to it.  The repeats run first: the
    # loop right after the pre-warm's long burst runs a few % slower than the
    # loops that follow (clocks), and the timed loop is meant to be a typical one.
    REPEATS = 11
    # Matvec workloads: the read kernel's launch-shape sweep that names the
    # best single-launch read of the weights (for the floors below).  It runs
    # before the pre-warm: after a burst of pure-read launches the matvec runs
    # ~5 % slower until some milliseconds of matvec load have passed (measured:
    # 7.73 -> 8.08-8.15 us per call at C4, back to 7.70 after ~5000 calls, not
    # after 0.5 s idle), and the pre-warm supplies that load.
    if kind != "matmul":
        nb = case.weight_bytes // 16 * 16
        fout = ctx.alloc(2048 * 1024 // 64 * 4)
        words = 8 * ctx.cu_count()
        per_round = max(20, args.steps)  # the headline's loop length

        def floor_op(op, **kw):
            return dict(op=op, q=case.wbuf, q_stride=case.stride, n_copies=case.n_copies, x=None,
                        y=fout, units=nb // 16, **kw)

        def shape_op(threads, loads, grid):
            return floor_op("read_shape", n_rows=grid, batch=grid * threads // 64,
                            variant=pkg.Variant(0, threads // 64, loads))

        def us(op, calls):
            return sum(ctx.bench_loop(**op, warmup=20, groups=1, calls_per_group=calls)) * 1e3 / calls

        # The read kernel at every shape of 256/512/1024 threads, 2/4/8 16-byte
        # loads in flight per lane and 256-2048 workgroups.
        sweep = []
        for threads in (256, 512, 1024):
            for loads in (2, 4, 8):
                for grid in (256, 512, 1024, 2048):
                    sweep.append((us(shape_op(threads, loads, grid), args.steps), threads, loads,
                                  grid))
        sweep.sort()
        _, bt, bl, bg = sweep[0]
    # Pre-warm, untimed: the same calls for at least 100 ms, so the clocks have
    # ramped up under load (a few warmup calls are a fraction of a millisecond,
    # and the first loop of a cold start runs ~10 % slower).
    prewarm_ms, n = 0.0, 20
    while prewarm_ms < 100.0 and n <= (1 << 20):
        prewarm_ms += sum(ctx.bench_loop(**case.bench_op(), warmup=0, groups=1,
                                         calls_per_group=n))
        n *= 2
    ctx.device_synchronize()
    per_call = sorted(ctx.bench_loop(**case.bench_op(), warmup=args.warmup, groups=1,
                                     calls_per_group=args.steps)[0] * 1000.0 / args.steps
                      for _ in range(REPEATS))
    ctx.device_synchronize()
    total_ms = ctx.bench_loop(**case.bench_op(), warmup=args.warmup, groups=1,
                              calls_per_group=args.steps)[0]
    ctx.device_synchronize()
    us_per_call = total_ms * 1000.0 / args.steps
    t = us_per_call * 1e-6
    # Sustained rate: 1000 back-to-back calls in one loop (milliseconds of
    # continuous load, where the clocks settle lower than in a short burst).
    SUSTAINED = 1000
    us_sustained = ctx.bench_loop(**case.bench_op(), warmup=args.warmup, groups=1,
                                  calls_per_group=SUSTAINED)[0] * 1000.0 / SUSTAINED
    ctx.device_synchronize()
    pct = {p: round(per_call[min(len(per_call) - 1, int(p / 100 * len(per_call)))], 3)
           for p in (10, 50, 90)}

    ev0, ev1 = ctx.event(), ctx.event()
    for i in range(args.warmup):
        case.launch(i)
    ctx.device_synchronize()
    ev0.record()
    for i in range(args.steps):
        case.launch(i)
    ev1.record()
    ev1.synchronize()
    ctx.device_synchronize()
    us_python = ev0.elapsed_ms(ev1) * 1000.0 / args.steps

    graph = ctx.capture(lambda: [case.launch(i) for i in range(args.steps)])
    graph.launch()  # warm replay
    ctx.device_synchronize()
    ev0.record()
    graph.launch()
    ev1.record()
    ev1.synchronize()
    ctx.device_synchronize()
    us_graph = ev0.elapsed_ms(ev1) * 1000.0 / args.steps
    graph.close()

    # The floor of the launch-per-call protocol on this box, for matvec
    # workloads: the same number of bytes read from the same rotated copies by
    # a kernel of the same launch shape that only reads (one store per wave),
    # the best of the read kernel's launch shapes (swept above), and an empty
    # kernel, all launched by the same loop.
    floor = None
    if kind != "matmul":
        # Ratios from interleaved rounds (the matvec, the read of its launch
        # shape, the best read shape, the empty kernel, one after another, each
        # max(20, K) back-to-back calls, the headline's loop length, 5 rounds),
        # so that clock drift
        # between runs cancels.
        ops = {"matvec": case.bench_op(), "read": floor_op("read_floor", batch=words),
               "best": shape_op(bt, bl, bg), "empty": floor_op("launch_empty", batch=words)}
        # The bytes a call cannot avoid are the weights and x: a read of as
        # many bytes (from the same rotated copies, starting at each copy; the
        # contents do not matter to a read) at the best read shape.  For C1
        # and C2 x outweighs the weights (C2: 128 KiB of x, 18 KiB of weights).
        nbx = (case.weight_bytes + case.x.nbytes + 15) // 16 * 16
        ops["read_wx"] = dict(op="read_shape", q=case.wbuf, q_stride=case.stride,
                              n_copies=case.n_copies, x=None, y=fout, units=nbx // 16, n_rows=bg,
                              batch=bg * bt // 64, variant=pkg.Variant(0, bt // 64, bl))
        rounds = {k: [] for k in ops}
        for _ in range(5):
            for k, op in ops.items():
                rounds[k].append(us(op, per_round))
        med = {k: sorted(v)[len(v) // 2] for k, v in rounds.items()}
        fout.close()
        read_us, best_us, empty_us = med["read"], med["best"], med["empty"]
        floor = {
            "read_same_bytes_us": round(read_us, 3),
            "read_same_bytes_GBps": round(nb / read_us / 1e3, 1),
            "empty_launch_us": round(empty_us, 3),
            "kernel_interleaved_us": round(med["matvec"], 3),
            "kernel_vs_read_floor": round(read_us / med["matvec"], 4),
            "best_read_us": round(best_us, 3),
            "best_read_GBps": round(nb / best_us / 1e3, 1),
            "best_read_shape": f"axh_read_floor_t{bt}_u{bl}, {bg} workgroups",
            "kernel_vs_best_read": round(best_us / med["matvec"], 4),
            "read_weights_and_x_us": round(med["read_wx"], 3),
            "weights_and_x_bytes": nbx,
            "kernel_vs_read_weights_and_x": round(med["read_wx"] / med["matvec"], 4),
            "read_sweep_us": [[t_, l_, g_, round(u_, 3)] for u_, t_, l_, g_ in sweep],
            "what": "back-to-back launches, by the same loop, of a kernel of the matvec's "
                    "launch shape (one 512-thread workgroup per CU) that only reads the same "
                    "bytes from the same rotated copies (one store per wave), of the fastest of "
                    "that read kernel's 36 launch shapes (read_sweep_us rows: threads, loads "
                    "in flight per lane, workgroups, us per call), of that best shape reading "
                    "the weights and x together (read_weights_and_x_us), and of an empty "
                    "kernel; the ratios are medians of 5 interleaved rounds of max(20, K) "
                    "calls of the matvec and of each floor",
        }
    kernel = case.kernel()
    shape = (("2x" if kind in GATE_UP_KINDS else "") + f"{case.rows}x{case.cols}"
             + (f"xB{case.batch}" if kind == "matmul" else ""))
    traffic, traffic_src = profiled_traffic(kernel, shape)

    if args.calibrate_copy:
        # A plain copy of exactly the weight bytes (hipMemcpy device-to-device
        # through the runtime's copy kernel), for scaling FETCH_SIZE/WRITE_SIZE.
        dst = ctx.alloc(case.weight_bytes)
        for _ in range(10):
            ctx.copy_device(dst, case.wbuf, case.weight_bytes)
        ctx.device_synchronize()
        dst.close()

    mfma_bound = kind == "matmul" and case.batch > 32
    if mfma_bound:
        unit, peak = "TFLOP/s", MFMA_F16_PEAK_TFLOPS
        value = case.flops() / t / 1e12
        algo = case.flops()
        metric = (f"Q4_K_M x f16 matmul TFLOP/s at {case.rows}x{case.cols}, B={case.batch}; "
                  "us/call")
    else:
        unit, peak = "GB/s", HBM_PEAK_GBS
        algo = case.weight_bytes
        value = algo / t / 1e9
        qname = {"q4_0": "Q4_0", "q5k": "Q5_K", "q6k": "Q6_K"}.get(kind, "Q4_K_M")
        if kind == "matmul":
            metric = (f"Q4_K_M x f16 matmul weight-bytes HBM GB/s at {case.rows}x{case.cols}, "
                      f"B={case.batch}; us/call")
        elif kind in GATE_UP_KINDS:
            fmt = {"gate_up": "Q4_K_M", "gate_up0": "Q4_0", "gate_up5": "Q5_K"}[kind]
            metric = (f"{fmt} fused gate+up (silu(g)*u) weight-bytes HBM GB/s at {shape}; "
                      "us/call")
        else:
            metric = f"{qname} matvec weight-bytes HBM GB/s (% of peak) at {shape}; us/call"

    cpu = case.cpu_baseline(args.cpu_seconds, unit) if args.cpu_seconds > 0 else None
    out = {
        "metric": metric,
        "value": round(value, 2),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms / args.steps, 6),
        "us_per_call": round(us_per_call, 3),
        "timing": f"{args.steps} back-to-back calls launched by the library's loop "
                  f"(axh_bench_loop) between two HIP events, behind {args.warmup} queued warmup "
                  f"calls, after an untimed pre-warm of {prewarm_ms:.0f} ms; the same calls "
                  f"launched from Python through ctypes: {us_python:.3f} us/call; replayed from "
                  f"one HIP graph: {us_graph:.3f} us/call",
        "us_per_call_p10_p50_p90": [pct[10], pct[50], pct[90]],
        "us_per_call_sustained": round(us_sustained, 3),
        "distribution": f"{REPEATS} more runs of the same {args.warmup} warmup + {args.steps} "
                        f"timed calls, each between its own two events; us_per_call_sustained: "
                        f"{SUSTAINED} calls in one loop",
        "kernel": kernel,
        "pct_of_peak": round(100.0 * value / peak, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("f32 in (cast to f16, RN), f32 accumulate" if case.x_f32
                  else "f16 in, f32 accumulate") if kind == "matmul" else "f32",
        "data": "synthetic",
        "config": {
            "workload": f"{args.workload}: {kind} {shape} ({case.label})",
            "rows": case.rows,
            "cols": case.cols,
            "batch": case.batch,
            "weight_bytes": case.weight_bytes,
            "x_bytes": case.x.nbytes,
            "y_bytes": case.y_bytes,
            "weight_copies_rotated": case.n_copies,
            "variant": args.variant or "default",
            "parallelism": "single GPU",
        },
        "parity": par,
        "roofline": {
            "bound": "mfma" if mfma_bound else "hbm",
            "achieved": round(value, 2),
            "peak": peak,
            "unit": unit,
            "frac": round(value / peak, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "algorithmic_bytes" if not mfma_bound else "algorithmic_flops": algo,
        },
        "cpu_baseline": cpu,
        "launch_floor": floor,
    }
    if mfma_bound:
        busy, busy_src = profiled_mfma_busy(kernel, shape)
        out["roofline"]["mfma_busy"] = busy
        out["roofline"]["mfma_busy_source"] = busy_src
    print(json.dumps(out), flush=True)
    case.close()
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
