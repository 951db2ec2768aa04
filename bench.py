#!/usr/bin/env python3
"""Benchmark of the fused cyclic-convolution hot path on one MI355X.

A "step" is one launch of the fused convolution over one batch of 2^27
points held in HBM: N = 4096, batch 32768, one shared filter (BASELINE.json
metric and configs[1]; the other configs are parity-test cases).  Prints ONE
JSON line.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]

Timing: W untimed launches, then exactly K launches bracketed by
torch.cuda.synchronize(), measured with HIP events recorded on the stream the
kernels are launched on.  Inputs are resident in HBM before the timed region.

roofline.achieved uses the reference's bandwidth model, 3 passes x 8 B = 24
bytes per point for fp32 (bench_fufft.cu:314-317), over the average launch
duration; with a shared filter one of those passes is served from cache, so
the physical minimum is 16 B/pt and `physical` reports that figure too.
roofline.traffic is the HBM bytes per launch measured by rocprofv3 PMC
(FETCH_SIZE + WRITE_SIZE) for this same command, read from the committed
summary profiles/conv_f32_n4096.md when present.

The cpu_baseline leg times the reference's own fp64 CPU conv path
(cpu_mixed.cpp, built into oracle/_ref) -- or, where that was not built, this
build's restatement of it -- on a bounded sample of the same workload, one
thread per host core.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import threading
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
HBM_PEAK_GBS = 8000.0
METRIC = json.loads((ROOT / "BASELINE.json").read_text())["metric"] if (ROOT / "BASELINE.json").exists() \
    else "Gpoints/s + % HBM peak, fused conv N=4096 fp32 & int16-BFP, 2^27-pt batch"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--n", type=int, default=4096)
    p.add_argument("--points-log2", type=int, default=27)
    p.add_argument("--variant", default="v16")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    return p.parse_args()


def spectrum_from_taps(rng, n):
    taps = (rng.standard_normal(n) + 1j * rng.standard_normal(n)).astype(np.complex64)
    return taps


def time_launches(torch, fn, steps, warmup, stream):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / 1e3          # seconds for `steps` launches


def measured_traffic(n, pts):
    """HBM bytes per launch from the committed rocprofv3 PMC summary."""
    f = ROOT / "profiles" / f"conv_f32_n{n}.md"
    if not f.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)\s+points:\s*(\d+)", f.read_text())
    if not m or int(m.group(2)) != pts:
        return None
    return float(m.group(1))


def cpu_baseline(n, seconds, threads):
    """Reference CPU conv path on a bounded sample, `threads` host threads."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as O                     # the checker library, CPU leg only
    ref = O.load_ref()
    rng = np.random.default_rng(3)
    per_thread = 64
    a = (rng.standard_normal((threads, per_thread, n)) + 1j * rng.standard_normal((threads, per_thread, n)))
    s = (rng.standard_normal(n) + 1j * rng.standard_normal(n)) / n
    s_full = np.ascontiguousarray(np.broadcast_to(s, (per_thread, n)))
    out = np.empty_like(a)
    counts = [0] * threads
    deadline = [0.0]

    def work(t):
        at = np.ascontiguousarray(a[t])
        ot = out[t]
        while time.perf_counter() < deadline[0]:
            if ref is not None:
                ref.ref_mixed_conv_f64(n, 16, at.ctypes.data, s_full.ctypes.data, n, ot.ctypes.data, per_thread)
            else:
                O.mixed_conv_f64(at, s_full, n, 16)
            counts[t] += per_thread

    deadline[0] = time.perf_counter() + seconds
    t0 = time.perf_counter()
    ths = [threading.Thread(target=work, args=(t,)) for t in range(threads)]
    for th in ths:
        th.start()
    for th in ths:
        th.join()
    el = time.perf_counter() - t0
    pts = sum(counts) * n
    return {
        "value": round(pts / el / 1e9, 6),
        "unit": "Gpoints/s",
        "cores": threads,
        "kind": "reference" if ref is not None else "port",
        "sample": (f"{sum(counts)} signals of N={n} (fp64 mixed-radix DIF -> multiply -> DIT with "
                   f"per-twiddle cos/sin, cpu_mixed.cpp) in {el:.1f} s on {threads} threads"),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the path shards along the batch with no exchange, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    import torch
    import fufft_amd as ff

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ff.init(0)
    n = args.n
    pts = 1 << args.points_log2
    batch = pts // n
    rng = np.random.default_rng(1)

    # synthetic workload: signal and taps i.i.d. N(0,1) from a seed
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    x = torch.randn(pts, dtype=torch.complex64, device=dev, generator=gen)
    out = torch.empty_like(x)
    taps = spectrum_from_taps(rng, n)
    filt = torch.from_numpy(ff.plan_filter(taps, n, variant=args.variant, kind=ff.FILTER_TAPS)).to(dev)
    stream = torch.cuda.current_stream()

    # correctness before timing: fp64 numpy on a sample of signals
    ff.conv(x, filt, out, n=n, batch=batch, variant=args.variant, stream=stream)
    torch.cuda.synchronize()
    idx = np.linspace(0, batch - 1, 16).astype(np.int64)
    xs = x.view(batch, n)[torch.from_numpy(idx).to(dev)].cpu().numpy().astype(np.complex128)
    ys = out.view(batch, n)[torch.from_numpy(idx).to(dev)].cpu().numpy()
    want = np.fft.ifft(np.fft.fft(xs, axis=1) * np.fft.fft(taps.astype(np.complex128))[None, :], axis=1)
    rel = float(np.linalg.norm(ys - want) / np.linalg.norm(want))
    if not rel <= 2e-6:
        print(json.dumps({"error": f"accuracy check failed: rel L2 {rel:.3e}"}))
        sys.exit(1)

    def step():
        ff.conv(x, filt, out, n=n, batch=batch, variant=args.variant, stream=stream)

    torch.cuda.synchronize()
    secs = time_launches(torch, step, args.steps, args.warmup, stream)
    torch.cuda.synchronize()
    avg = secs / args.steps
    gpts = pts / avg / 1e9
    achieved = 24.0 * pts / avg / 1e9
    physical = 16.0 * pts / avg / 1e9
    traffic = measured_traffic(n, pts)

    line = {
        "metric": METRIC,
        "value": round(gpts, 3),
        "unit": "Gpoints/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(avg * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"fused fp32 cyclic conv, N={n}, batch {batch} (2^{args.points_log2} points), "
                               f"one shared filter, mid=multiply, variant={args.variant}",
                   "n": n, "batch": batch, "points": pts},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "model_bytes_per_point": 24,
                     "physical": {"bytes_per_point": 16, "achieved": round(physical, 1),
                                  "frac": round(physical / HBM_PEAK_GBS, 4)}},
        "accuracy": {"rel_l2_vs_fp64_sample": rel},
    }
    if not args.no_cpu_baseline:
        threads = min(16, os.cpu_count() or 1)
        line["cpu_baseline"] = cpu_baseline(n, args.cpu_seconds, threads)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
