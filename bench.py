#!/usr/bin/env python3
"""Benchmark of the MI355X backend's FusedQuantizedDense hot path.

Headline workload (the config the metric is quoted on): decode GEMV,
x bf16 [1,4096], Int4 weights [4096,11008] (reference packing), group-128 bf16 scales along K,
no bias.  A step is one Execute of the compiled graph over one batch, with every input already
resident in HBM.  Weight sets are rotated (> 512 MB of distinct copies) so each step reads its
weights from HBM rather than the 256 MB Infinity Cache.

Output: one JSON line (see `--help`).  `value` is algorithmic bytes per step / wall time per
step over K back-to-back steps (host launch overhead included); `roofline` prices the dominant
kernel's average duration from HIP events on the backend's stream; `cpu_baseline` times the
CPU restatement of the reference loop (oracle/, the reference itself is Go and cannot be built
here) on a bounded sample on this host.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
MALL_BYTES = 256 << 20


def measure(backend, wl, steps: int, warmup: int, rotate_bytes: int = 2 * MALL_BYTES):
    exe = wl.compile(backend)
    n_sets = max(1, math.ceil(rotate_bytes / max(1, wl.weight_bytes())))
    n_sets = min(n_sets, 64)
    sets = [wl.upload(backend) for _ in range(n_sets)]
    backend.SetProfiling(False)
    exe.ExecuteLoop(sets, warmup)
    backend.Synchronize()
    # Timed region: K back-to-back steps (no per-step host sync), then one sync.
    t0 = time.perf_counter()
    exe.ExecuteLoop(sets, steps)
    backend.Synchronize()
    wall = time.perf_counter() - t0
    # Same K steps with a HIP event pair around every kernel launch (the kernel durations).
    backend.SetProfiling(True)
    backend.ProfileReset()
    exe.ExecuteLoop(sets, steps)
    backend.Synchronize()
    prof = backend.Profile()
    backend.SetProfiling(False)
    for s in sets:
        for b in s:
            b.Finalize()
    exe.Finalize()
    kname, (launches, total_ms) = max(prof.items(), key=lambda kv: kv[1][1])
    return {
        "ms_per_step": wall / steps * 1e3,
        "kernel": kname,
        "kernel_us": total_ms / launches * 1e3,
        "kernel_launches_per_step": launches / steps,
        "profile": {k: {"launches": v[0], "avg_us": v[1] / v[0] * 1e3} for k, v in prof.items()},
        "weight_sets": n_sets,
    }


def cpu_baseline(wl, seconds: float):
    """The oracle (plain-C restatement of quantizedDenseLinearInt, parallel like the reference's
    quantizedDenseParallel) timed on this host over a bounded sample of the same workload."""
    from oracle import oracle as O

    dtmap = {"Int8": O.DT_INT8, "Int4": O.DT_INT4, "Float32": O.DT_FLOAT32, "BFloat16": O.DT_BFLOAT16}
    p = O.QDenseProblem(M=wl.M, K=wl.K, N=wl.N, x=wl.x, x_dtype=dtmap[str(wl.x_dtype)], w=wl.w,
                        w_dtype=dtmap[str(wl.w_dtype)], scale=wl.scale, scale_dtype=dtmap[str(wl.scale_dtype)],
                        scale_shape=wl.scale_shape, block_axis=wl.block_axis, block_size=wl.block_size,
                        bias=wl.bias, bias_dtype=dtmap[str(wl.bias_dtype)] if wl.bias is not None else O.DT_FLOAT32,
                        act=wl.act)
    threads = min(16, os.cpu_count() or 1)
    O.qdense_f32(p, threads=threads)  # warm up
    calls, t0 = 0, time.perf_counter()
    while True:
        O.qdense_f32(p, threads=threads)
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    gbs = wl.algorithmic_bytes() * calls / el / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{calls} full calls of {wl.name} in {el:.1f} s ({el / calls * 1e3:.2f} ms/call)"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--extra", default="C1,C3", help="comma list of other configs to report under 'extra'")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build targets one MI355X; --gpus {args.gpus} is not supported "
              "(the quantized-dense path shards by output columns with no collective on one GPU)", file=sys.stderr)
        sys.exit(2)

    import compute_amd as ca
    from compute_amd import workloads

    backend = ca.New("mi355x")
    wl = workloads.make("C2")
    r = measure(backend, wl, args.steps, args.warmup)
    nbytes = wl.algorithmic_bytes()
    value = nbytes / (r["ms_per_step"] * 1e-3) / 1e9
    achieved = nbytes / (r["kernel_us"] * 1e-6) / 1e9
    out = {
        "metric": "QuantizedDense GB/s & TFLOP/s vs MI355X roofline; us/call at decode+prefill",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded; weights rotated over %d distinct HBM copies)" % r["weight_sets"],
        "config": {"workload": wl.name, "M": wl.M, "K": wl.K, "N": wl.N, "weights": "Int4 reference packing",
                   "group_size": wl.block_size, "scales": "bf16 [32,11008]", "bias": None, "activation": "none",
                   "algorithmic_bytes": nbytes, "us_per_call": round(r["ms_per_step"] * 1e3, 2),
                   "kernel_us": round(r["kernel_us"], 3), "kernel": r["kernel"],
                   "tflops": round(wl.flops() / (r["ms_per_step"] * 1e-3) / 1e12, 3)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None},
    }
    extra = {}
    for name in [n for n in args.extra.split(",") if n]:
        w2 = workloads.make(name)
        steps = max(3, min(args.steps, 50))
        r2 = measure(backend, w2, steps, 2)
        b2 = w2.algorithmic_bytes()
        extra[w2.name] = {
            "us_per_call": round(r2["ms_per_step"] * 1e3, 2), "kernel": r2["kernel"],
            "kernel_us": round(r2["kernel_us"], 3),
            "GBps_kernel": round(b2 / (r2["kernel_us"] * 1e-6) / 1e9, 1),
            "TFLOPs_kernel": round(w2.flops() / (r2["kernel_us"] * 1e-6) / 1e12, 3),
        }
    if extra:
        out["extra"] = extra
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(wl, args.cpu_seconds)
    backend.Finalize()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
