"""Benchmark of the MI355X Q4_K_M dequant-matvec hot path.

One step = one Q4_K_M matvec of the 4096 x 14336 down-projection (BASELINE
config 4, the north-star shape) over weights already resident in HBM.
Weights rotate over enough distinct copies (> 256 MiB) that every call reads
HBM instead of the Infinity Cache.  Prints ONE JSON line.

  python bench.py [--gpus 1] [--steps 200] [--warmup 20]
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

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth
ROWS, SB = 4096, 56     # 4096 x 14336 Q4_K_M
COPIES_MIN_BYTES = 512 << 20


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


def cpu_baseline(O, q, x, rows, sb, budget_s: float) -> dict:
    """The oracle (C restatement of q4km_dequant_matvec_cpu: scalar, the
    reference's order) on the full matrix for about `budget_s` seconds on one
    core, then row-parallel over the host's cores for a quarter of that."""
    weight_bytes = rows * sb * 144
    n, el = _time_cpu(lambda: O.q4k_matvec_single(q, x, rows, sb), budget_s)
    threads = max(1, min(os.cpu_count() or 1, 16))
    nm, elm = _time_cpu(lambda: O.q4k_matvec(q, x, rows, sb, threads=threads),
                        max(1.0, budget_s / 4))
    return {
        "value": round(weight_bytes * n / el / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{n} full {rows}x{sb * 256} Q4_K matvecs in {el:.1f}s, one thread "
                  f"({cpu_model()}, nproc={os.cpu_count()}); {el / n * 1e6:.0f} us/call",
        "all_cores": {
            "value": round(weight_bytes * nm / elm / 1e9, 4),
            "cores": threads,
            "sample": f"{nm} full matvecs in {elm:.1f}s, rows split over {threads} threads "
                      f"(bit-identical to one thread); {elm / nm * 1e6:.0f} us/call",
        },
    }


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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--variant", default="", help="rows_per_wave,waves,prefetch[,nontemporal]")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run device-to-device copies of the weight size (counter calibration)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build runs the matvec on one MI355X; "
              "see DESIGN.md for how the path shards across GPUs.", file=sys.stderr)
        return 2

    import numpy as np

    import __graft_entry__
    from oracle import oracle as O

    pkg = __graft_entry__.load_package()
    variant = None
    if args.variant:
        variant = pkg.Variant(*(int(t) for t in args.variant.split(",")))

    rows, sb = ROWS, SB
    weight_bytes = rows * sb * 144
    q = O.gen_q4k_weights(20241, rows * sb)
    x = O.gen_normal_f32(20242, sb * 256, 0.5)

    ctx = pkg.HipContext.new()
    n_copies = max(2, -(-COPIES_MIN_BYTES // weight_bytes))
    copies = []
    for _ in range(n_copies):
        b = ctx.alloc(weight_bytes)
        ctx.upload(b, q)
        copies.append(b)
    dx = ctx.alloc(x.nbytes)
    ctx.upload(dx, x)
    dy = ctx.alloc(rows * 4)

    # parity of this exact workload before timing
    ctx.q4k_matvec(copies[0], dx, dy, rows, sb, variant)
    ctx.synchronize()
    y = np.frombuffer(ctx.download(dy, rows * 4), dtype=np.float32)
    ref = O.q4k_matvec(q, x, rows, sb)
    yf, absdot = O.q4k_matvec_f64(q, x, rows, sb)
    rep = O.matvec_tolerance_report(y, ref, yf, absdot, sb * 256)
    if not rep["ok"]:
        print(json.dumps({"error": "parity failure", "report": rep}), file=sys.stderr)
        return 1

    # Timed region: K back-to-back calls on the context stream, bracketed by
    # device synchronisation and HIP events recorded on that same stream.
    for i in range(args.warmup):
        ctx.q4k_matvec(copies[i % n_copies], dx, dy, rows, sb, variant)
    ctx.device_synchronize()
    ev0, ev1 = ctx.event(), ctx.event()
    ev0.record()
    for i in range(args.steps):
        ctx.q4k_matvec(copies[i % n_copies], dx, dy, rows, sb, variant)
    ev1.record()
    ev1.synchronize()
    ctx.device_synchronize()
    total_ms = ev0.elapsed_ms(ev1)
    us_per_call = total_ms * 1000.0 / args.steps
    gbs = weight_bytes / (us_per_call * 1e-6) / 1e9

    # Distribution: the same back-to-back stream cut into groups of 10 calls
    # by events (an event between every call would add its own gap).
    group = 10
    n_groups = max(1, args.steps // group)
    evs = [ctx.event() for _ in range(n_groups + 1)]
    evs[0].record()
    for g in range(n_groups):
        for i in range(group):
            ctx.q4k_matvec(copies[(g * group + i) % n_copies], dx, dy, rows, sb, variant)
        evs[g + 1].record()
    evs[-1].synchronize()
    per_call = sorted(evs[g].elapsed_ms(evs[g + 1]) * 1000.0 / group for g in range(n_groups))
    pct = {p: round(per_call[min(len(per_call) - 1, int(p / 100 * len(per_call)))], 3)
           for p in (10, 50, 90)}
    kernel = pkg.q4k_matvec_kernel_name(rows, sb, variant)
    traffic, traffic_src = profiled_traffic(kernel, f"{rows}x{sb * 256}")

    if args.calibrate_copy:
        # A plain copy of exactly weight_bytes (hipMemcpy device-to-device
        # through the runtime's copy kernel), for scaling FETCH_SIZE/WRITE_SIZE.
        dst = ctx.alloc(weight_bytes)
        for _ in range(10):
            ctx.copy_device(dst, copies[0], weight_bytes)
        ctx.device_synchronize()
        dst.close()

    cpu = cpu_baseline(O, q, x, rows, sb, args.cpu_seconds) if args.cpu_seconds > 0 else None
    out = {
        "metric": "Q4_K_M matvec weight-bytes HBM GB/s (% of peak) at 4096x14336; us/call",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms / args.steps, 6),
        "us_per_call": round(us_per_call, 3),
        "us_per_call_p10_p50_p90_of_10call_groups": [pct[10], pct[50], pct[90]],
        "kernel": kernel,
        "pct_of_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "q4k_matvec 4096x14336 (Q4_K_M down-projection, config 4)",
            "rows": rows,
            "cols": sb * 256,
            "weight_bytes": weight_bytes,
            "x_bytes": sb * 256 * 4,
            "y_bytes": rows * 4,
            "weight_copies_rotated": n_copies,
            "variant": args.variant or "default",
            "parallelism": "single GPU",
        },
        "parity": {k: rep[k] for k in ("rows_failed", "norm_rel_err", "gpu_err_vs_f64_norm",
                                       "cpu_err_vs_f64_norm")},
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "algorithmic_bytes": weight_bytes,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    for b in copies + [dx, dy]:
        b.close()
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
