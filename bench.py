#!/usr/bin/env python3
"""Benchmark of the MI355X backend's FusedQuantizedDense hot path.

Headline workload (the config the metric is quoted on): decode GEMV,
x bf16 [1,4096], Int4 weights [4096,11008] (reference packing), group-128 bf16 scales along K,
no bias.  A step is one Execute of the compiled graph over one batch, with every input already
resident in HBM.  Weight sets are rotated (> 512 MB of distinct copies) so each step reads its
weights from HBM rather than the 256 MB Infinity Cache.

The JSON line also reports, under "extra", the other BASELINE configurations measured the same
way: C3 batched decode (HBM roofline), C4 prefill (bf16 MFMA roofline) and C5, the quantized MLP
graph built through the Builder API (microseconds per Execute, 100 resident calls); G1 / G2,
the GGML block-format decode GEMV (Q4_0 / Q4_K rows, f32 x [1,4096], 11008 rows; HBM roofline);
R1, the reference's own layout at the C2 shape (f32 x, Int4, scales [4096, 86]; HBM roofline);
and D1, bf16 DotGeneral at the C4 shape (bf16 MFMA roofline).

`value` is algorithmic bytes per step / wall time per step over K back-to-back steps (host
launch overhead included: the wall clock starts as the first Execute is issued and stops when
the host has seen the last step complete).  `roofline` prices the dominant kernel's average
duration: where one kernel is the whole step, the device time per step of the same timed region
(a HIP event pair on the backend's stream around the K launches); otherwise HIP events recorded
around every launch over K more steps (`kernel_us_source` says which; per-launch events add work
between kernels and read longer, so they are used only to split a multi-kernel step).
Weight sets are handed out in one rotation across the warm-up, timed and event-timed loops, so
no loop starts on a set that is still in the Infinity Cache.  Before the warm-up, every copy is
read once by a read-only pass (the GPU's first access to freshly uploaded memory walks its page
tables) and a pass over a separate 512 MB buffer then leaves none of them in the cache.
`traffic` (HBM bytes per launch) is read from profiles/traffic.json, which is produced from
rocprofv3 FETCH_SIZE / WRITE_SIZE passes over this script (see --copy-calibration).
`stream_floor` is a read-only pass over the headline's weight bytes (same rotation, same region
timing): the HBM floor that the decode kernel's time is set beside.
`cpu_baseline` times the CPU restatement of the reference loop (oracle/, the reference itself is
Go and cannot be built here) on a bounded sample on this host.
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
F32_PEAK_TFLOPS = 157.3
MALL_BYTES = 256 << 20
METRIC = "QuantizedDense GB/s & TFLOP/s vs MI355X roofline; µs/call at decode+prefill"


class Rotation:
    """The weight sets of a workload, handed out in one continuous rotation across the warm-up,
    timed and profiled loops, so that no loop starts on a set read shortly before (each set is
    read again only after every other set, more than the 256 MB Infinity Cache in between)."""

    def __init__(self, sets):
        self.sets, self.next = sets, 0

    def take(self, n: int):
        """The sets of the next n steps, in order (ExecuteLoop runs step i on set i % len)."""
        k = len(self.sets)
        order = [self.sets[(self.next + i) % k] for i in range(min(n, k))]
        self.next = (self.next + n) % k
        return order


_FLUSH = {}


def prime(backend, sets):
    """Touches every input copy on the device once and then leaves none of them in the Infinity
    Cache: a read-only pass over each buffer (the GPU's first access to freshly uploaded memory
    walks its page tables, which added ~2.5 us per step to the first 20 C2 steps), then a pass over
    a separate buffer of twice the cache's size.  Nothing is executed; the warm-up steps follow."""
    import numpy as np
    import compute_amd as ca

    bufs = [b for s in sets for b in s if b.Shape().byte_size() >= 16]
    if bufs:
        backend.DebugStreamRead(bufs, len(bufs))
    key = id(backend)
    if key not in _FLUSH:
        n = 2 * MALL_BYTES // 4
        _FLUSH[key] = backend.BufferFromFlatData(0, np.zeros(n, np.float32), ca.Shape(ca.Float32, n))
    backend.DebugStreamRead([_FLUSH[key]], 1)
    backend.Synchronize()


def measure(backend, wl, steps: int, warmup: int, rotate_bytes: int = 2 * MALL_BYTES):
    """Wall time per step over `steps` back-to-back Executes, then the same steps again with a
    HIP event pair around every kernel launch (per-kernel average durations)."""
    exe = wl.compile(backend)
    n_sets = max(1, math.ceil(rotate_bytes / max(1, wl.weight_bytes())))
    capped = n_sets > 64  # tiny weights (C1): 64 sets still fit the cache; such a case is latency-bound
    n_sets = min(n_sets, 64)
    if rotate_bytes and not capped:
        # A set is read again only after the other n_sets - 1 sets: more than the MALL apart.
        assert (n_sets - 1) * wl.weight_bytes() > MALL_BYTES, (wl.name, n_sets)
    rot = Rotation([wl.upload(backend) for _ in range(n_sets)])
    backend.SetProfiling(False)
    prime(backend, rot.sets)
    exe.ExecuteLoop(rot.take(warmup), warmup)
    backend.Synchronize()
    timed = exe.LoopSets(rot.take(steps))
    backend.RegionBegin()  # the device-side start event; the wall clock starts with the first Execute
    t0 = time.perf_counter()
    exe.ExecuteLoop(timed, steps)
    region_ms = backend.RegionEnd()  # waits for the stream: the timed region ends here
    wall = time.perf_counter() - t0
    backend.SetProfiling(True)
    backend.ProfileReset()
    exe.ExecuteLoop(rot.take(steps), steps)
    backend.Synchronize()
    prof = backend.Profile()
    backend.SetProfiling(False)
    for s in rot.sets:
        for b in s:
            b.Finalize()
    exe.Finalize()
    kernels = {k: {"launches_per_step": v[0] / steps, "avg_us": v[1] / v[0] * 1e3} for k, v in prof.items()}
    kname = max(prof.items(), key=lambda kv: kv[1][1])[0]
    kernel_us_per_step = sum(v[1] for v in prof.values()) / steps * 1e3
    region_us = region_ms / steps * 1e3
    if len(prof) == 1 and kernels[kname]["launches_per_step"] == 1:
        # One kernel per step: its average duration is the device time of the timed region per
        # step (an event pair on the backend's stream around the back-to-back launches; the
        # inter-dispatch gap is included, so this errs low on the achieved rate).  Per-launch
        # events add work between the kernels and read longer.
        kernel_us, source = region_us, "hip_events_region (per-launch events read %.3f us)" % kernels[kname]["avg_us"]
        kernel_us_per_step = region_us
    else:
        kernel_us, source = kernels[kname]["avg_us"], "hip_events_per_launch"
    return {"ms_per_step": wall / steps * 1e3, "kernel": kname, "kernel_us": kernel_us, "kernel_us_source": source,
            "kernels": kernels, "kernel_us_per_step": kernel_us_per_step, "region_us_per_step": region_us,
            "weight_sets": n_sets}


def stream_floor(backend, wl, steps: int, warmup: int, rotate_bytes: int = 2 * MALL_BYTES):
    """The HBM streaming floor for the workload's weight bytes: read-only passes
    (mx_backend_debug_stream_read, 16-byte loads, nothing written) over as many distinct weight
    copies as the timed loop rotates through, `steps` passes timed as one region like the kernel."""
    import compute_amd as ca

    n_sets = max(1, math.ceil(rotate_bytes / wl.weight_bytes()))
    bufs = [backend.BufferFromFlatData(0, wl.w.ravel(), ca.Shape(wl.w_dtype, wl.K, wl.N)) for _ in range(n_sets)]
    prime(backend, [[b] for b in bufs])
    backend.DebugStreamRead(bufs, warmup)
    backend.Synchronize()
    k = warmup % n_sets  # continue the rotation: the first timed pass reads the least recent copy
    backend.RegionBegin()
    backend.DebugStreamRead(bufs[k:] + bufs[:k], steps)
    us = backend.RegionEnd() / steps * 1e3
    for b in bufs:
        b.Finalize()
    nbytes = wl.weight_bytes()
    return {"kernel": "stream_read_kernel", "bytes": nbytes, "us": round(us, 3),
            "GBps": round(nbytes / (us * 1e-6) / 1e9, 1), "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "us_at_algorithmic_bytes": round(us * wl.algorithmic_bytes() / nbytes, 3), "copies": n_sets,
            "source": "hip_events_region"}


def traffic_for(name: str):
    """HBM bytes per launch of the workload's dominant kernel from profiles/traffic.json."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        v = t.get(name)
        return None if v is None else int(v["hbm_bytes_per_launch"])
    except (OSError, ValueError, KeyError, TypeError):
        return None


def hbm_roofline(nbytes: float, us: float, traffic):
    achieved = nbytes / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic}


def mfma_roofline(flops: float, us: float, traffic, peak: float = None):
    peak = peak or BF16_PEAK_TFLOPS
    achieved = flops / (us * 1e-6) / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 1), "peak": peak, "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4), "traffic": traffic}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _oracle_problems(wl):
    """The workload as oracle problems: one for a FusedQuantizedDense workload, the three
    projections (gate, up, down) for the MLP, whose other ops are a few KB of elementwise work."""
    import numpy as np
    from oracle import oracle as O

    dtmap = {"Int8": O.DT_INT8, "Int4": O.DT_INT4, "Uint4": O.DT_UINT4, "Float32": O.DT_FLOAT32,
             "BFloat16": O.DT_BFLOAT16}
    if hasattr(wl, "weights"):
        h = wl.x  # RMSNorm output stand-in of the same shape and dtype (timing only)
        return [O.QDenseProblem(M=wl.M, K=K, N=N, x=h if K == wl.D else np.zeros((wl.M, K), np.uint16),
                                x_dtype=O.DT_BFLOAT16, w=w, w_dtype=O.DT_INT4, scale=sc, scale_dtype=O.DT_BFLOAT16,
                                scale_shape=(K // wl.G, N), block_axis=0, block_size=wl.G, bias=None,
                                bias_dtype=O.DT_FLOAT32, act=0)
                for w, sc, K, N in wl.weights]
    return [O.QDenseProblem(M=wl.M, K=wl.K, N=wl.N, x=wl.x, x_dtype=dtmap[str(wl.x_dtype)], w=wl.w,
                            w_dtype=dtmap[str(wl.w_dtype)], scale=wl.scale, scale_dtype=dtmap[str(wl.scale_dtype)],
                            scale_shape=wl.scale_shape, block_axis=wl.block_axis, block_size=wl.block_size,
                            bias=wl.bias,
                            bias_dtype=dtmap[str(wl.bias_dtype)] if wl.bias is not None else O.DT_FLOAT32,
                            act=wl.act, scheme=wl.scheme)]


def cpu_time_per_call(wl, seconds: float, threads: int):
    """Seconds per full call of the oracle on `threads` threads, from a bounded sample: whole
    calls, or for large M a block of rows scaled up to M (the loop is row-independent)."""
    import numpy as np
    from oracle import oracle as O

    probs = _oracle_problems(wl)
    rows = None
    if wl.M > 64:
        rows = np.arange(0, wl.M, wl.M // 16, dtype=np.int64)[:16]
    for p in probs:  # warm up
        O.qdense_f32(p, rows=rows, threads=threads)
    calls, t0 = 0, time.perf_counter()
    while True:
        for p in probs:
            O.qdense_f32(p, rows=rows, threads=threads)
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per = el / calls
    if rows is not None:
        per *= wl.M / len(rows)
    what = f"{calls} calls" + (f" of {len(rows)} of {wl.M} rows, scaled to all rows" if rows is not None else "")
    return per, what


def cpu_baseline(headline, others, seconds: float):
    """The oracle (plain-C restatement of quantizedDenseLinearInt, quantizeddense.go:616-650, run
    in parallel over output rows and columns like quantizedDenseParallel) timed on this host's
    cores, since the reference's Go toolchain is absent: the headline config gives `value`, every
    config its own entry."""
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    per, what = cpu_time_per_call(headline, seconds, threads)
    out = {"value": round(headline.algorithmic_bytes() / per / 1e9, 3), "unit": "GB/s", "cores": threads,
           "nproc": os.cpu_count(), "cpu_model": _cpu_model(), "kind": "port",
           "reference": "CPU baseline unavailable (no Go toolchain): gobackend is Go and cannot be built or "
                        "run in this image; the figures are the oracle's C restatement (a port)",
           "sample": f"{what} of {headline.name} in the C oracle ({per * 1e3:.2f} ms/call); Go (gobackend) "
                     "is absent from this image, so the oracle's restatement of quantizeddense.go:616-650 "
                     "stands in for it",
           "configs": {}}
    for wl in [headline] + list(others):
        p2, w2 = (per, what) if wl is headline else cpu_time_per_call(wl, seconds / 3, threads)
        e = {"us_per_call": round(p2 * 1e6, 1), "sample": w2}
        if wl.name.startswith("C4"):
            e["GFLOPs"] = round(wl.flops() / p2 / 1e9, 1)
        else:
            e["GBps"] = round(wl.algorithmic_bytes() / p2 / 1e9, 3)
        out["configs"][wl.name] = e
    return out


def copy_calibration(mib: int, iters: int):
    """A plain device-to-device copy of known size (for scaling the FETCH_SIZE / WRITE_SIZE
    counters to bytes): `iters` copies of `mib` MiB."""
    import torch

    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(iters):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": n, "launches": iters}), flush=True)


def extra_entry(wl, r):
    nbytes = wl.algorithmic_bytes()
    e = {"us_per_call": round(r["ms_per_step"] * 1e3, 2), "kernel": r["kernel"], "kernel_us": round(r["kernel_us"], 3),
         "kernel_us_source": r["kernel_us_source"], "kernel_us_per_call": round(r["kernel_us_per_step"], 3),
         "device_us_per_call": round(r["region_us_per_step"], 3)}
    if wl.name.startswith("C4") or wl.name.startswith("D1") or wl.name.startswith("Q"):
        e["TFLOPs_kernel"] = round(wl.flops() / (r["kernel_us"] * 1e-6) / 1e12, 1)
        e["roofline"] = mfma_roofline(wl.flops(), r["kernel_us"], traffic_for(wl.name))
    elif wl.name.startswith("R3"):
        # f32 x: the dequantised weights are contracted on the f32 matrix cores; the whole call
        # (dequantisation, contraction, epilogue) priced against the dense f32 MFMA peak.
        e["TFLOPs_call"] = round(wl.flops() / (r["kernel_us_per_step"] * 1e-6) / 1e12, 1)
        e["kernels"] = {k: {"per_call": round(v["launches_per_step"], 2), "avg_us": round(v["avg_us"], 3)}
                        for k, v in r["kernels"].items()}
        e["roofline"] = mfma_roofline(wl.flops(), r["kernel_us_per_step"], traffic_for(wl.name), F32_PEAK_TFLOPS)
    elif wl.name.startswith("C5"):
        # Whole graph per call: the three quantized projections dominate; price one call's device
        # time (the timed region per call, all kernels and the gaps between them) against HBM.
        e["GBps_call"] = round(nbytes / (r["ms_per_step"] * 1e-3) / 1e9, 1)
        e["kernels"] = {k: {"per_call": round(v["launches_per_step"], 2), "avg_us": round(v["avg_us"], 3)}
                        for k, v in r["kernels"].items()}
        e["roofline"] = hbm_roofline(nbytes, r["region_us_per_step"], traffic_for(wl.name))
    else:
        e["GBps_kernel"] = round(nbytes / (r["kernel_us"] * 1e-6) / 1e9, 1)
        e["roofline"] = hbm_roofline(nbytes, r["kernel_us"], traffic_for(wl.name))
    return e


def dot_table(ca):
    """The reference's BenchmarkDotGeneral model shapes (support/backendtest/bench_dotgeneral.go,
    float32 there) on this backend, in float32 and bfloat16: microseconds per Execute (wall, launch
    included), the kernels that ran and their time per call."""
    from compute_amd import workloads
    backend = ca.New("")
    for case in workloads.DOT_MODEL_CASES:
        for dt in (ca.Float32, ca.BFloat16):
            wl = workloads.DotCaseWorkload(case, dt)
            r = measure(backend, wl, 50, 5, rotate_bytes=0)
            e = {"case": case[0], "dtype": dt.name, "us_per_call": round(r["ms_per_step"] * 1e3, 2),
                 "kernel_us_per_call": round(r["kernel_us_per_step"], 2),
                 "GFLOPs_call": round(wl.flops() / (r["ms_per_step"] * 1e-3) / 1e9, 1),
                 "kernels": {k: round(v["avg_us"], 2) for k, v in r["kernels"].items()}}
            print(json.dumps(e), flush=True)
    backend.Finalize()


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--extra", default="C1,C3,C4,C5,Q1,Q2,G1,G2,R1,R3,D1",
                    help="comma list of other configs to report under 'extra' (C1's wall time per call, with a "
                         "kernel of a few microseconds, bounds the host time of one Execute)")
    ap.add_argument("--only", default="", help="run only this config (profiling passes); prints its entry")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-crossover", dest="crossover", action="store_false",
                    help="skip the 32/64-row GEMM-vs-GEMV comparison")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--dot-table", action="store_true",
                    help="only time the reference's BenchmarkDotGeneral model shapes (f32 and bf16), one line each")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build targets one MI355X; --gpus {args.gpus} is not supported "
              "(the quantized-dense path shards by output columns with no collective on one GPU)", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration, 20)
        return

    import compute_amd as ca
    if args.dot_table:
        dot_table(ca)
        return
    from compute_amd import workloads

    backend = ca.New("mi355x")
    if args.only:
        wl = workloads.make(args.only)
        r = measure(backend, wl, args.steps, args.warmup)
        print(json.dumps({"workload": wl.name, **extra_entry(wl, r)}), flush=True)
        backend.Finalize()
        return

    wl = workloads.make("C2")
    r = measure(backend, wl, args.steps, args.warmup)
    nbytes = wl.algorithmic_bytes()
    value = nbytes / (r["ms_per_step"] * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights, bf16 activations, f32 accumulate",
        "data": "synthetic (seeded; weights rotated over %d distinct HBM copies)" % r["weight_sets"],
        "config": {"workload": wl.name, "M": wl.M, "K": wl.K, "N": wl.N, "weights": "Int4 reference packing",
                   "group_size": wl.block_size, "scales": "bf16 [32,11008]", "bias": None, "activation": "none",
                   "algorithmic_bytes": nbytes, "us_per_call": round(r["ms_per_step"] * 1e3, 2),
                   "kernel_us": round(r["kernel_us"], 3), "kernel_us_source": r["kernel_us_source"],
                   "kernel": r["kernel"],
                   "tflops": round(wl.flops() / (r["ms_per_step"] * 1e-3) / 1e12, 3)},
        "roofline": hbm_roofline(nbytes, r["kernel_us"], traffic_for(wl.name)),
        "stream_floor": stream_floor(backend, wl, args.steps, args.warmup),
    }
    extra = {}
    for name in [n for n in args.extra.split(",") if n]:
        w2 = workloads.make(name)
        steps = 100 if name == "C5" else max(3, min(args.steps, 50))
        extra[w2.name] = extra_entry(w2, measure(backend, w2, steps, 5))
    if args.crossover:
        # Rows 17..64 with per-channel int8: the default plan (skinny row groups at 32 rows, the
        # GEMM at 64) against the GEMV they replaced.
        b2 = ca.New("mi355x,gemv_over_gemm")
        for name in ("P32", "P64"):
            w2 = workloads.make(name)
            e = {}
            for label, bk in (("default", backend), ("gemv", b2)):
                r2 = measure(bk, w2, max(3, min(args.steps, 50)), 5)
                e[label] = {"us_per_call": round(r2["ms_per_step"] * 1e3, 2), "kernel": r2["kernel"],
                            "kernel_us_per_call": round(r2["kernel_us_per_step"], 3)}
            extra[w2.name] = e
        b2.Finalize()
    if extra:
        out["extra"] = extra
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(wl, [workloads.make(n) for n in ("C1", "C3", "C4", "C5")],
                                           args.cpu_seconds)
    backend.Finalize()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
