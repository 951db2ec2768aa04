#!/usr/bin/env python3
"""Benchmark of the fused cyclic-convolution hot path on one MI355X.

A "step" is one launch of the fused convolution over one batch of 2^27
points held in HBM: N = 4096, batch 32768, one shared filter (BASELINE.json
metric, configs[1]).  The metric names fp32 AND int16-BFP, so the same JSON
line carries the fp32 figure as `value` and the int16-BFP figure for the same
N and batch under "bfp", plus a short fp32 sweep over the other
configs[1] sizes under "sweep".  Prints ONE JSON line.

The filter is planned once on the host (--layout lane: the library's
lane-major pair layout, at the variant fufft_fastest_variant picks for it --
radix 16 at N = 4096; --layout dr: the reference's digit order).  The line
also carries the headline workload with the other layout ("dr_layout").

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]

Timing, the same for the headline and every other leg: a correctness check
against fp64 first, then --settle seconds of untimed launches (after an idle
gap the part runs 8-13% slow for the first tens of milliseconds while its
clocks ramp), then W untimed launches, then exactly K launches bracketed by
torch.cuda.synchronize(), measured with HIP events recorded on the stream the
kernels are launched on.  Inputs are resident in HBM before the timed region.

roofline.achieved counts the bytes the workload must move across HBM: the
signal read and the result written once, 16 bytes per point, plus the shared
filter once (8N bytes), over the average launch duration; rocprofv3's
FETCH_SIZE + WRITE_SIZE for this same command (roofline.traffic, read from
the committed summary profiles/conv_f32_n4096.md) measure 16.003 B/pt, so
roofline.frac is the fraction of MI355X's 8 TB/s the kernel really moves.
The reference's own model, 3 passes x 8 B = 24 B/pt (bench_fufft.cu:314-317),
counts the filter as a third pass; with one shared filter that pass is served
from cache, so it is reported apart (roofline.model_24B) and can exceed 1.
Every other leg likewise gives `frac` on the bytes it must move and the
reference-model figure under a `model_` key.  roofline.stream_ceiling_gbs is
the best of a sweep of copy shapes of the library's buffer-instruction stream
copy (fufft_stream_f32) over the same bytes, the measured HBM ceiling.

The cpu_baseline leg times the reference's own CPU conv paths (cpu_mixed.cpp
fp64, and verify_kernel.cpp's fp32 and int16-BFP transcriptions of the device
dataflow, built into oracle/_ref) per N, on bounded samples of the same
workloads, one thread per usable host core.
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
    p.add_argument("--variant", default="fastest",
                   help="r8 | v16 | auto | fastest (fufft_fastest_variant for --layout)")
    p.add_argument("--layout", default="lane", choices=["lane", "dr"],
                   help="filter layout of the fp32 and BFP legs: the library's lane-major pairs "
                        "(fastest) or the reference's digit order")
    p.add_argument("--sweep", default="512,1024,2048",
                   help="extra fp32 sizes timed with --sweep-steps launches each ('' for none)")
    p.add_argument("--sweep-steps", type=int, default=50)
    p.add_argument("--no-bfp", action="store_true")
    p.add_argument("--bfp-sizes", default="4096,512")
    p.add_argument("--large-sizes", default="32768,65536",
                   help="four-step sizes timed with --sweep-steps calls each ('' for none)")
    p.add_argument("--no-2d", action="store_true")
    p.add_argument("--no-c2c", action="store_true", help="skip the natural-order C2C line")
    p.add_argument("--no-vendor", action="store_true", help="skip the rocFFT chain comparison")
    p.add_argument("--per-signal-sizes", default="",
                   help="comma list of further N for the one-filter-per-signal legs (both filter layouts)")
    p.add_argument("--no-per-signal", action="store_true",
                   help="skip the one-filter-per-signal legs (fp32 and reference-format BFP at N)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=20.0,
                   help="wall seconds for all CPU-baseline rows together")
    p.add_argument("--settle", type=float, default=0.1,
                   help="seconds of untimed launches before each secondary figure (0 under PMC runs)")
    p.add_argument("--no-stream-sweep", action="store_true",
                   help="skip the sweep of copy shapes (the ceiling is then the best fixed shape; for PMC runs)")
    p.add_argument("--copy-sweep", action="store_true",
                   help="time every copy shape of the stream-ceiling sweep and print one line per shape")
    p.add_argument("--copy-only", action="store_true",
                   help="time only the stream copy of the workload's bytes (HBM ceiling, and the copy "
                        "of known size that scales rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return p.parse_args()


def stream_ceiling(torch, ff, dev, pts, steps, warmup, stream, nontemporal):
    """GB/s (read + write) of the library's buffer-instruction stream copy
    (fufft_stream_f32) over pts complex64 points, and seconds per copy."""
    x = torch.empty(pts, dtype=torch.complex64, device=dev).fill_(1.0)
    y = torch.empty_like(x)
    secs = time_launches(torch, lambda: ff.stream_copy(x, y, pts * 8, nontemporal, stream=stream),
                         steps, warmup, stream, SETTLE_S)
    torch.cuda.synchronize()
    if not torch.equal(x, y):
        raise RuntimeError("stream copy produced a wrong result")
    del x, y
    return 2.0 * pts * 8 * steps / secs / 1e9, secs / steps


# The copy shapes of the ceiling sweep (fufft_stream_shape_f32): lanes per
# workgroup, bytes per load and loads in flight per lane, consecutive tiles per
# workgroup or a persistent grid of workgroups (0 = one launch-wide grid), and
# the cache policies of loads and stores (SC0 = 1, NT = 2).
SWEEP_SHAPES = [(lanes, w, loads) for lanes in (256, 64, 1024) for w in (16, 8) for loads in (1, 2, 4, 8, 16, 32)
                if lanes * w * loads <= 256 * 1024]
SWEEP_GRID = ((1, 0), (2, 0), (4, 0), (1, 1024), (1, 2048), (1, 4096))
SWEEP_POLICY = ((0, 0), (2, 2), (2, 0), (0, 2), (3, 3))


def stream_sweep(torch, ff, dev, pts, steps, warmup, stream):
    """Every shape of the sweep over the same 2^k points: a list of
    (GB/s, shape dict), the whole sweep settled once (the launches run back to
    back), each shape checked for an exact copy."""
    x = torch.empty(pts, dtype=torch.complex64, device=dev).fill_(1.0)
    x.view(torch.float32)[::7].fill_(-3.5)
    y = torch.empty_like(x)
    nbytes = pts * 8
    rows = []
    time_launches(torch, lambda: ff.stream_copy(x, y, nbytes, True, stream=stream), 1, 1, stream, SETTLE_S)
    for lanes, width, loads in SWEEP_SHAPES:
        for per, groups in SWEEP_GRID:
            for pld, pst in SWEEP_POLICY:
                y.zero_()

                def copy():
                    ff.stream_copy_shape(x, y, nbytes, loads, per, groups, pld, pst, width=width, lanes=lanes,
                                         stream=stream)
                secs = time_launches(torch, copy, steps, warmup, stream, 0.0)
                torch.cuda.synchronize()
                if not torch.equal(x, y):
                    raise RuntimeError(f"stream copy shape {(lanes, width, loads, per, groups, pld, pst)} "
                                       "copied wrongly")
                rows.append((2.0 * nbytes * steps / secs / 1e9,
                             {"lanes": lanes, "load_bytes": width, "loads_per_lane": loads, "tiles_per_group": per,
                              "groups": groups, "load_policy": pld, "store_policy": pst}))
    del x, y
    return rows


SETTLE_S = 0.1          # set from --settle in main()


def time_launches(torch, fn, steps, warmup, stream, settle_s=0.0):
    """Seconds for `steps` launches of fn after `warmup` untimed ones.  With
    settle_s > 0 (every leg passes --settle; PMC runs pass 0) untimed launches
    continue until settle_s seconds have passed: after an idle gap -- host-side
    input generation or a correctness check -- the part runs 8-13% slow for
    the first tens of milliseconds while its clocks ramp."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t_end = time.perf_counter() + settle_s
    while time.perf_counter() < t_end:
        for _ in range(4):
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


def frac(bytes_per_launch, secs):
    """Fraction of MI355X's HBM peak: bytes per launch over seconds per launch."""
    return round(bytes_per_launch / secs / 1e9 / HBM_PEAK_GBS, 4)


def rel_l2(got, want):
    return float(np.linalg.norm(got - want) / np.linalg.norm(want))


def per_launch_us(torch, fn, count, stream):
    """Durations of `count` launches timed one by one (an event pair around
    each), in microseconds -- after the timed region, so that region's own
    timing is untouched."""
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(count)]
    for a, b in ev:
        a.record(stream)
        fn()
        b.record(stream)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) * 1e3 for a, b in ev]


def pick_variant(ff, n, variant, layout):
    """The variant a leg runs: --variant as given, "fastest" through the library."""
    return ff.fastest_variant(n, layout) if variant == "fastest" else ff.resolve_variant(n, variant)


def bench_fp32(torch, ff, dev, n, pts, variant, steps, warmup, stream, seed, settle_s=0.0, per_launch=0,
               layout="dr", per_signal=False):
    """fp32 fused conv at size n over pts points, the filter planned in
    `layout`: (seconds per launch, rel L2 of a sample), plus the one-by-one
    launch durations in us when per_launch > 0.  per_signal: one filter per
    signal (filt_stride = n, random natural-order spectra planned on the
    device), the reference bench's own protocol (bench_fufft.cu:160-170),
    where the filter is a third pass over HBM."""
    batch = pts // n
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    x = torch.randn(pts, dtype=torch.complex64, device=dev, generator=gen)
    out = torch.empty_like(x)
    rng = np.random.default_rng(seed)
    idx = torch.from_numpy(np.linspace(0, batch - 1, 16).astype(np.int64)).to(dev)
    if per_signal:
        spec = torch.randn(pts, dtype=torch.complex64, device=dev, generator=gen)
        filt = torch.empty_like(spec)
        ff.plan_filter_device(spec, filt, n, count=batch, variant=variant, layout=layout, stream=stream)
        spec_s = spec.view(batch, n)[idx].cpu().numpy().astype(np.complex128)
        del spec
        stride = n
    else:
        taps = (rng.standard_normal(n) + 1j * rng.standard_normal(n)).astype(np.complex64)
        filt = torch.from_numpy(ff.plan_filter(taps, n, variant=variant, layout=layout, kind=ff.FILTER_TAPS)).to(dev)
        spec_s = np.fft.fft(taps.astype(np.complex128))[None, :]
        stride = 0

    def step():
        ff.conv(x, filt, out, n=n, batch=batch, filt_stride=stride, variant=variant, layout=layout, stream=stream)

    # correctness before timing: fp64 numpy on a sample of signals
    step()
    torch.cuda.synchronize()
    xs = x.view(batch, n)[idx].cpu().numpy().astype(np.complex128)
    ys = out.view(batch, n)[idx].cpu().numpy()
    want = np.fft.ifft(np.fft.fft(xs, axis=1) * spec_s, axis=1)
    rel = rel_l2(ys, want)
    secs = time_launches(torch, step, steps, warmup, stream, settle_s)
    each = per_launch_us(torch, step, per_launch, stream) if per_launch else []
    del x, out, filt
    if per_launch:
        return secs / steps, rel, each
    return secs / steps, rel


def bench_vendor_chain(torch, dev, n, pts, steps, warmup, stream, seed, uniform=False):
    """The vendor-library chain the reference compares against (cuFFT fwd ->
    pointwise -> inv, bench_fufft.cu:201-213, and beside the four-step at
    453-478), on MI355X: torch.fft, which calls rocFFT, forward -> multiply ->
    inverse on the same workload (Re/Im N(0,1), or U[-1,1) with uniform)."""
    batch = pts // n
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    if uniform:
        x = (torch.rand(2 * pts, device=dev, generator=gen) * 2 - 1).view(torch.complex64).view(batch, n)
    else:
        x = torch.randn(pts, dtype=torch.complex64, device=dev, generator=gen).view(batch, n)
    rng = np.random.default_rng(seed)
    taps = (rng.standard_normal(n) + 1j * rng.standard_normal(n)).astype(np.complex64)
    spec = torch.fft.fft(torch.from_numpy(taps).to(dev))

    def step():
        return torch.fft.ifft(torch.fft.fft(x, dim=1) * spec, dim=1)

    y = step()
    torch.cuda.synchronize()
    want = np.fft.ifft(np.fft.fft(x[:4].cpu().numpy().astype(np.complex128), axis=1)
                       * np.fft.fft(taps.astype(np.complex128))[None, :], axis=1)
    rel = rel_l2(y[:4].cpu().numpy(), want)
    del y
    secs = time_launches(torch, step, steps, warmup, stream, SETTLE_S)
    del x
    torch.cuda.empty_cache()
    return secs / steps, rel


def bench_c2c(torch, ff, dev, n, pts, steps, warmup, stream, seed):
    """Natural-order batched forward C2C (fufft_c2c_f32) and rocFFT's
    (torch.fft.fft) on the same 2^27-point batch: 16 B/pt, read + write."""
    batch = pts // n
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    x = torch.randn(pts, dtype=torch.complex64, device=dev, generator=gen)
    out = torch.empty_like(x)

    def ours():
        ff.c2c(x, out, n=n, batch=batch, direction=ff.FORWARD, variant="auto", stream=stream)

    ours()
    torch.cuda.synchronize()
    idx = torch.from_numpy(np.linspace(0, batch - 1, 16).astype(np.int64)).to(dev)
    want = np.fft.fft(x.view(batch, n)[idx].cpu().numpy().astype(np.complex128), axis=1)
    rel = rel_l2(out.view(batch, n)[idx].cpu().numpy(), want)
    t_ours = time_launches(torch, ours, steps, warmup, stream, SETTLE_S) / steps
    xv = x.view(batch, n)

    def vendor():
        return torch.fft.fft(xv, dim=1)

    y = vendor()
    torch.cuda.synchronize()
    vrel = rel_l2(y.view(batch, n)[idx].cpu().numpy(), want)
    del y
    t_vendor = time_launches(torch, vendor, steps, warmup, stream, SETTLE_S) / steps
    del x, out, xv
    torch.cuda.empty_cache()
    return {"n": n, "batch": batch, "direction": "forward", "variant": ff.resolve_variant(n, "auto"),
            "gpoints_s": round(pts / t_ours / 1e9, 3), "ms": round(t_ours * 1e3, 5),
            "bytes_per_point": 16, "achieved_gbs": round(16.0 * pts / t_ours / 1e9, 1),
            "frac": frac(16.0 * pts, t_ours), "rel_l2": rel,
            "rocfft": {"what": "torch.fft.fft (rocFFT), same batch", "gpoints_s": round(pts / t_vendor / 1e9, 3),
                       "ms": round(t_vendor * 1e3, 5), "rel_l2": vrel},
            "speedup_vs_rocfft": round(t_vendor / t_ours, 3)}


def bench_r2(torch, ff, dev, n, pts, steps, warmup, stream, seed):
    """Real two-for-one 1D conv (fufft_conv_r2_f32): pts complex points are
    2 pts real samples, x and y U[0,1) each convolved with one shared real
    filter (taps U[0,1), planned as a spectrum) and written to u and v; 4 bytes
    per real sample read and written, 16 per complex point."""
    batch = pts // n
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    x = torch.rand(pts, device=dev, generator=gen)
    y = torch.rand(pts, device=dev, generator=gen)
    u, v = torch.empty_like(x), torch.empty_like(y)
    rng = np.random.default_rng(seed)
    taps = rng.uniform(0, 1, n).astype(np.complex64)
    layout = "lane"
    var = ff.fastest_variant(n, layout)
    filt = torch.from_numpy(ff.plan_filter(taps, n, variant=var, layout=layout, kind=ff.FILTER_TAPS)).to(dev)

    def step():
        ff.conv_r2(x, y, filt, u, v, n=n, batch=batch, variant=var, layout=layout, stream=stream)

    step()
    torch.cuda.synchronize()
    idx = torch.from_numpy(np.linspace(0, batch - 1, 16).astype(np.int64)).to(dev)
    spec = np.fft.fft(taps.real.astype(np.float64))
    got, want = [], []
    for a, b in ((x, u), (y, v)):
        xs = a.view(batch, n)[idx].cpu().numpy().astype(np.float64)
        want.append(np.fft.ifft(np.fft.fft(xs, axis=1) * spec[None, :], axis=1).real)
        got.append(b.view(batch, n)[idx].cpu().numpy())
    rel = rel_l2(np.stack(got), np.stack(want))
    secs = time_launches(torch, step, steps, warmup, stream, SETTLE_S) / steps
    del x, y, u, v, filt
    return {"n": n, "batch": batch, "variant": var, "filter_layout": layout,
            "gsamples_s": round(2 * pts / secs / 1e9, 3), "gpoints_s": round(pts / secs / 1e9, 3),
            "ms": round(secs * 1e3, 5), "bytes_per_sample": 8, "frac": frac(16.0 * pts + 8.0 * n, secs),
            "rel_l2": rel}


def bench_large(torch, ff, dev, n, pts, steps, warmup, stream, seed, variant="auto", per_transform=False):
    """Four-step conv: batch pts/n of U[-1,1) signals, one
    shared filter in the chain order of the middle `variant` ("auto" = "v16",
    the reference's run_large middle), in place.  per_transform: one chained
    filter per transform, as the reference's run_large feeds it
    (bench_fufft.cu:410-428; fufft::ref::run_large), planned on the device from
    random natural-order spectra.  Returns (seconds per call, rel L2 of a
    sample)."""
    batch = pts // n
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    x = (torch.rand(2 * pts, device=dev, generator=gen) * 2 - 1).view(torch.complex64)
    rng = np.random.default_rng(seed)
    idx = torch.from_numpy(np.linspace(0, batch - 1, 8).astype(np.int64)).to(dev)
    xs = x.view(batch, n)[idx].cpu().numpy().astype(np.complex128)
    if per_transform:
        spec = torch.randn(pts, dtype=torch.complex64, device=dev, generator=gen)
        filt = torch.empty_like(spec)
        ff.plan_filter_large_device(spec, filt, n, count=batch, variant=variant, stream=stream)
        spec_s = spec.view(batch, n)[idx].cpu().numpy().astype(np.complex128)
        stride = n
    else:
        taps = (rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)).astype(np.complex64)
        filt = torch.from_numpy(ff.plan_filter_large(taps, n, kind=ff.FILTER_TAPS, variant=variant)).to(dev)
        spec_s = np.fft.fft(taps.astype(np.complex128))[None, :]
        stride = 0
    ff.conv_large(x, filt, n=n, batch=batch, filt_stride=stride, variant=variant, stream=stream)
    torch.cuda.synchronize()
    ys = x.view(batch, n)[idx].cpu().numpy()
    want = np.fft.ifft(np.fft.fft(xs, axis=1) * spec_s, axis=1)
    rel = rel_l2(ys, want)
    # the call is in place, so the timed launches re-convolve their own output;
    # they use all-pass filters (unit-modulus spectra, random phase) of the
    # same cost, which keep the data's norm fixed over any number of launches
    if per_transform:
        spec = torch.polar(torch.ones(pts, device=dev), torch.rand(pts, device=dev, generator=gen) * (2 * np.pi))
        ff.plan_filter_large_device(spec, filt, n, count=batch, variant=variant, stream=stream)
        del spec
    else:
        phase = np.exp(2j * np.pi * rng.uniform(0, 1, n)).astype(np.complex64)
        filt = torch.from_numpy(ff.plan_filter_large(phase, n, kind=ff.FILTER_SPECTRUM, variant=variant)).to(dev)
    secs = time_launches(torch, lambda: ff.conv_large(x, filt, n=n, batch=batch, filt_stride=stride,
                                                      variant=variant, stream=stream),
                         steps, warmup, stream, SETTLE_S)
    del x, filt
    return secs / steps, rel


def bench_2d(torch, ff, dev, pts, steps, warmup, stream, seed):
    """BASELINE configs[4] at 512 x 512: (a) two real images per complex
    transform, 2^27 real pixels U[0,1), one real filter U[0,1); (b) the split
    path: one image transformed once, applied against 256 filters with
    Gaussian spectra.  Returns a dict for the JSON line."""
    h = w = 512
    np_img = h * w
    nimg = pts // np_img // 2                    # packed complex transforms
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    x = torch.rand(nimg * np_img, device=dev, generator=gen)
    y = torch.rand(nimg * np_img, device=dev, generator=gen)
    u, v = torch.empty_like(x), torch.empty_like(y)
    work = torch.empty(nimg * np_img, dtype=torch.complex64, device=dev)
    taps = rng.uniform(0, 1, np_img).astype(np.complex64)
    filt = torch.from_numpy(ff.plan_filter2d(taps, h, w, kind=ff.FILTER_TAPS, layout="lane")).to(dev)

    def r2():
        ff.conv2d_r2(x, y, filt, u, v, work, h, w, nimg, layout="lane", stream=stream)

    r2()
    torch.cuda.synchronize()
    xs = x.view(nimg, h, w)[0].cpu().numpy().astype(np.float64)
    want = np.real(np.fft.ifft2(np.fft.fft2(xs) * np.fft.fft2(taps.real.reshape(h, w).astype(np.float64))))
    rel_r2 = rel_l2(u.view(nimg, h, w)[0].cpu().numpy(), want)
    t_r2 = time_launches(torch, r2, steps, warmup, stream, SETTLE_S) / steps
    del x, y, u, v, work

    nf = 256
    a = torch.rand(2 * np_img, device=dev, generator=gen).view(torch.complex64)
    spec = torch.empty_like(a)
    spec_nat = (rng.standard_normal((nf, np_img)) + 1j * rng.standard_normal((nf, np_img))).astype(np.complex64)
    filters = torch.from_numpy(np.concatenate([ff.plan_filter2d(spec_nat[i], h, w, layout="lane")
                                               for i in range(nf)])).to(dev)
    out = torch.empty(nf * np_img, dtype=torch.complex64, device=dev)
    ff.fwd2d(a, spec, h, w, 1, stream=stream)

    def apply():
        ff.apply2d(spec, filters, out, h, w, nf, spec_stride=0, filt_stride=np_img, layout="lane", stream=stream)

    apply()
    torch.cuda.synchronize()
    fa = np.fft.fft2(a.cpu().numpy().reshape(h, w).astype(np.complex128))
    rel_ap = rel_l2(out.view(nf, np_img)[5].cpu().numpy(),
                    np.fft.ifft2(fa * spec_nat[5].reshape(h, w)).reshape(-1))
    t_ap = time_launches(torch, apply, steps, warmup, stream, SETTLE_S) / steps
    del a, spec, filters, out
    return {
        "real_two_for_one_512x512": {
            "gpixels_s": round(2 * nimg * np_img / t_r2 / 1e9, 3), "ms": round(t_r2 * 1e3, 5),
            "images": 2 * nimg, "rel_l2": rel_r2,
            # three launches, each reading and writing 4 B per real pixel (a complex
            # point packs two pixels); the filter is cache-resident
            "bytes_per_pixel": 24, "frac": frac(24.0 * 2 * nimg * np_img, t_r2)},
        "split_apply_512x512_x256": {
            "gpoints_s": round(nf * np_img / t_ap / 1e9, 3), "ms": round(t_ap * 1e3, 5), "rel_l2": rel_ap,
            # filter read + result written by the column apply, the row inverse's read
            # and write; the shared spectrum is cache-resident
            "bytes_per_point": 32, "frac": frac(32.0 * nf * np_img, t_ap)},
    }


def bench_bfp(torch, ff, dev, n, pts, steps, warmup, stream, seed, block=64, variant="auto", layout="dr"):
    """int16-BFP fused conv: Gaussian x 10^u per signal (u ~ U[-3, 3]), quantised on
    the host by the library codec (one exponent per `block` points), one shared
    fp32 filter spectrum planned in `layout`."""
    batch = pts // n
    rng = np.random.default_rng(seed)
    x = np.empty((batch, n), dtype=np.complex64)
    chunk = max(1, (1 << 22) // n)
    for b0 in range(0, batch, chunk):
        b1 = min(batch, b0 + chunk)
        re = rng.standard_normal((b1 - b0, n), dtype=np.float32)
        im = rng.standard_normal((b1 - b0, n), dtype=np.float32)
        s = (10.0 ** rng.uniform(-3, 3, (b1 - b0, 1))).astype(np.float32)
        x[b0:b1].real = re * s
        x[b0:b1].imag = im * s
    q, e = ff.bfp_quantize(x, block=block)
    taps = (rng.standard_normal(n) + 1j * rng.standard_normal(n)).astype(np.complex64)
    filt = torch.from_numpy(ff.plan_filter(taps, n, variant=variant, layout=layout, kind=ff.FILTER_TAPS)).to(dev)
    dq, de = torch.from_numpy(q).to(dev), torch.from_numpy(e).to(dev)
    qo, eo = torch.empty_like(dq), torch.empty_like(de)

    def step():
        ff.conv_bfp16(dq, de, filt, qo, eo, n=n, batch=batch, stream=stream, block=block, variant=variant,
                      layout=layout)

    step()
    torch.cuda.synchronize()
    idx = np.linspace(0, batch - 1, 16).astype(np.int64)
    qs = qo.view(batch, 2 * n)[torch.from_numpy(idx).to(dev)].cpu().numpy()
    es = eo.view(batch, n // block)[torch.from_numpy(idx).to(dev)].cpu().numpy()
    got = ff.bfp_dequantize(qs, es, block=block).reshape(16, n)
    want = np.fft.ifft(np.fft.fft(x[idx].astype(np.complex128), axis=1)
                       * np.fft.fft(taps.astype(np.complex128))[None, :], axis=1)
    per_sig = np.linalg.norm(got - want, axis=1) / np.linalg.norm(want, axis=1)
    del x
    secs = time_launches(torch, step, steps, warmup, stream, SETTLE_S)
    del dq, de, qo, eo
    return secs / steps, rel_l2(got, want), float(per_sig.max())


def bench_bfp_scaled(torch, ff, dev, n, pts, steps, warmup, stream, seed, variant="v16", layout="dr",
                     per_signal=False):
    """int16-BFP conv in the reference's own format (fufft_conv_bfp16_scaled: one
    fp32 scale per transform, an int16 filter with one scale, in the given
    filter layout), on the same Gaussian x 10^u input as bench_bfp, quantised
    by the reference's rule.  per_signal: one int16 filter per signal (random
    natural-order spectra, planned on the device, quantised per filter), as
    the reference's bench feeds fufft_pipeline_v16_bfp (bench_fufft.cu:172-178)."""
    batch = pts // n
    rng = np.random.default_rng(seed)
    q = np.empty(2 * pts, dtype=np.int16)
    sc = np.empty(batch, dtype=np.float32)
    chunk = max(1, (1 << 22) // n)
    x16 = None
    for b0 in range(0, batch, chunk):
        b1 = min(batch, b0 + chunk)
        s = (10.0 ** rng.uniform(-3, 3, (b1 - b0, 1))).astype(np.float32)
        xc = (rng.standard_normal((b1 - b0, n), dtype=np.float32) * s
              + 1j * (rng.standard_normal((b1 - b0, n), dtype=np.float32) * s)).astype(np.complex64)
        if b0 == 0:
            x16 = xc[:16].copy()
        q[2 * n * b0: 2 * n * b1], sc[b0:b1] = ff.bfp_scaled_quantize(xc, n)
    if per_signal:
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        spec = torch.randn(pts, dtype=torch.complex64, device=dev, generator=gen)
        planned = torch.empty_like(spec)
        ff.plan_filter_device(spec, planned, n, count=batch, variant=variant, layout=layout, stream=stream)
        spec16 = spec[: 16 * n].cpu().numpy().astype(np.complex128).reshape(16, n)
        del spec
        fq = np.empty(2 * pts, dtype=np.int16)
        fs = np.empty(batch, dtype=np.float32)
        for b0 in range(0, batch, chunk):
            b1 = min(batch, b0 + chunk)
            fq[2 * n * b0: 2 * n * b1], fs[b0:b1] = ff.bfp_scaled_quantize(planned[n * b0: n * b1].cpu().numpy(), n)
        del planned
        stride = n
    else:
        taps = (rng.standard_normal(n) + 1j * rng.standard_normal(n)).astype(np.complex64)
        fq, fs = ff.bfp_scaled_quantize(ff.plan_filter(taps, n, variant=variant, layout=layout, kind=ff.FILTER_TAPS), n)
        spec16 = np.fft.fft(taps.astype(np.complex128))[None, :]
        stride = 0
    dq, ds = torch.from_numpy(q).to(dev), torch.from_numpy(sc).to(dev)
    dfq, dfs = torch.from_numpy(fq).to(dev), torch.from_numpy(fs).to(dev)
    qo, so = torch.empty_like(dq), torch.empty_like(ds)
    del q

    def step():
        ff.conv_bfp16_scaled(dq, ds, dfq, dfs, qo, so, n=n, batch=batch, filt_stride=stride, variant=variant,
                             layout=layout, stream=stream)

    step()
    torch.cuda.synchronize()
    got = ff.bfp_scaled_dequantize(qo[: 32 * n].cpu().numpy(), so[:16].cpu().numpy(), n).reshape(16, n)
    want = np.fft.ifft(np.fft.fft(x16.astype(np.complex128), axis=1) * spec16, axis=1)
    secs = time_launches(torch, step, steps, warmup, stream, SETTLE_S)
    del dq, ds, dfq, dfs, qo, so
    return secs / steps, rel_l2(got, want)


def usable_cores():
    """(cores, affinity, quota): host cores this process may run on -- its CPU
    affinity (os.sched_getaffinity), capped by a cgroup CPU quota where one is
    set (cgroup v2 cpu.max, else v1 cfs_quota_us / cfs_period_us)."""
    affinity = len(os.sched_getaffinity(0))
    quota = None
    try:
        q, per = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if q != "max":
            quota = int(q) / int(per)
    except (OSError, ValueError):
        try:
            q = int(Path("/sys/fs/cgroup/cpu/cpu.cfs_quota_us").read_text())
            per = int(Path("/sys/fs/cgroup/cpu/cpu.cfs_period_us").read_text())
            if q > 0:
                quota = q / per
        except (OSError, ValueError):
            pass
    cores = affinity if quota is None else max(1, min(affinity, int(quota)))
    return cores, affinity, quota


def _timed_threads(threads, seconds, per_call, call):
    """Run call(t) on `threads` host threads until `seconds` have passed; each
    call processes per_call signals.  Returns (signals done, elapsed seconds)."""
    counts = [0] * threads
    deadline = time.perf_counter() + seconds

    def work(t):
        while time.perf_counter() < deadline:
            call(t)
            counts[t] += per_call

    t0 = time.perf_counter()
    ths = [threading.Thread(target=work, args=(t,)) for t in range(threads)]
    for th in ths:
        th.start()
    for th in ths:
        th.join()
    return sum(counts), time.perf_counter() - t0


def cpu_baseline(sizes, bfp_sizes, head_n, seconds, threads, lanes):
    """The reference's CPU conv paths on the GPU box's host cores, on bounded
    samples of the bench workloads (Re/Im N(0,1) signals, one shared filter),
    one thread per usable core, each thread looping over its own batch:

    - fp64: cpu_mixed.cpp's V=16 fp64 DIF -> multiply -> DIT with per-twiddle
      cos/sin (cpu_mixed.cpp:121-174, 260-266), per N in `sizes`; the headline
      `value` is this row at head_n;
    - fp32 transcription: verify_kernel.cpp's CPU transcription of the device
      dataflow at the plan the GPU runs in this bench (lanes[n] values per
      lane: kernel_pipeline_ip for radix 8, kernel_pipeline_v16 for radix 16;
      verify_kernel.cpp:211-244, 1051-1082);
    - BFP transcription: verify_kernel.cpp's kernel_v16_bfp (1111-1135), the
      int16-BFP dataflow with one fp32 scale per transform, per N in bfp_sizes.

    The reference's sources are built into oracle/_ref; where that library is
    missing, this build's restatement (oracle/) stands in ("port")."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as O                     # the checker library, CPU leg only
    ref = O.load_ref()
    kind = "reference" if ref is not None else "port"
    per_row = seconds / (2 * len(sizes) + len(bfp_sizes))
    rng = np.random.default_rng(3)
    rows = {"fp64_cpu_mixed": {}, "fp32_transcription": {}, "bfp16_transcription": {}}

    def gpts(done, el, n):
        return round(done * n / el / 1e9, 6)

    for n in sizes:
        per = max(1, 16384 // n)                       # signals per call and thread
        a = rng.standard_normal((threads, per, n)) + 1j * rng.standard_normal((threads, per, n))
        spec = (rng.standard_normal(n) + 1j * rng.standard_normal(n)) / n
        s_full = np.ascontiguousarray(np.broadcast_to(spec, (per, n)))
        out = np.empty_like(a)

        def f64(t):
            if ref is not None:
                ref.ref_mixed_conv_f64(n, 16, a[t].ctypes.data, s_full.ctypes.data, n, out[t].ctypes.data, per)
            else:
                O.mixed_conv_f64(a[t], s_full, n, 16)
        done, el = _timed_threads(threads, per_row, per, f64)
        rows["fp64_cpu_mixed"][str(n)] = {"gpoints_s": gpts(done, el, n), "signals": done, "seconds": round(el, 2)}

        v = lanes[n]                                   # the plan the GPU legs run
        plan = O.ref_plan(n, v)
        lead = plan.radices[0] if plan.radices[0] != v else 1
        nv = sum(1 for r in plan.radices if r == v)
        a32 = a.astype(np.complex64)
        f32 = np.ascontiguousarray(np.broadcast_to(spec[O.mixedrev(plan)].astype(np.complex64), (per, n)))
        o32 = np.empty_like(a32)

        def tr32(t):
            if ref is not None:
                fn = ref.ref_vk_pipeline_ip if v == 8 else ref.ref_vk_pipeline_v16
                fn(n, lead, nv, 1, a32[t].ctypes.data, f32.ctypes.data, o32[t].ctypes.data, per)
            else:
                O.conv(a32[t], f32[0], n, plan, tw=O.TW_LIBM)
        done, el = _timed_threads(threads, per_row, per, tr32)
        rows["fp32_transcription"][str(n)] = {"gpoints_s": gpts(done, el, n), "plan": plan.radices,
                                              "signals": done, "seconds": round(el, 2)}

    for n in bfp_sizes:
        plan = O.ref_plan(n, 16)                       # kernel_v16_bfp runs the radix-16 plan
        lead = plan.radices[0] if plan.radices[0] != 16 else 1
        nrv = sum(1 for r in plan.radices if r == 16)
        per = max(1, 16384 // n)
        x = (rng.standard_normal((threads, per, n)) + 1j * rng.standard_normal((threads, per, n))).astype(np.complex64)
        spec = ((rng.standard_normal(n) + 1j * rng.standard_normal(n)) / n).astype(np.complex64)
        qb = np.empty(2 * n, np.int16)
        qa = np.empty((threads, per, 2 * n), np.int16)
        sa = np.empty((threads, per), np.float32)
        qo = np.empty_like(qa)
        so = np.empty_like(sa)
        if ref is not None:
            sb = ref.ref_vk_bfp_quantize(np.ascontiguousarray(spec[O.mixedrev(plan)]).ctypes.data, n, qb.ctypes.data)
            for t in range(threads):
                for i in range(per):
                    sa[t, i] = ref.ref_vk_bfp_quantize(x[t, i].ctypes.data, n, qa[t, i].ctypes.data)
        qe, ee = O.bfp_quantize(x.reshape(-1), block=n)

        def bfp(t):
            if ref is not None:
                ref.ref_vk_v16_bfp(n, lead, nrv, qa[t].ctypes.data, sa[t].ctypes.data, qb.ctypes.data, sb,
                                   qo[t].ctypes.data, so[t].ctypes.data, per)
            else:
                O.bfp_conv(qe[2 * n * per * t:2 * n * per * (t + 1)], ee[per * t:per * (t + 1)],
                           spec[O.mixedrev(plan)], n, plan, block=n)
        done, el = _timed_threads(threads, per_row, per, bfp)
        rows["bfp16_transcription"][str(n)] = {"gpoints_s": gpts(done, el, n), "plan": plan.radices,
                                               "signals": done, "seconds": round(el, 2)}

    head = rows["fp64_cpu_mixed"][str(head_n)]
    total = sum(r["seconds"] for g in rows.values() for r in g.values())
    return {
        "value": head["gpoints_s"],
        "unit": "Gpoints/s",
        "cores": threads,
        "kind": kind,
        "sample": (f"N={head_n}: {head['signals']} signals of the fp64 cpu_mixed conv (mixed-radix DIF -> "
                   f"multiply -> DIT, per-twiddle cos/sin) in {head['seconds']} s on {threads} threads, one per "
                   f"usable host core; all rows below together {total:.0f} s of wall time"),
        "rows": rows,
    }


def main():
    global SETTLE_S
    args = parse()
    SETTLE_S = max(0.0, args.settle)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the path shards along the batch with no exchange between GPUs)", file=sys.stderr)
        sys.exit(2)

    import torch
    import fufft_amd as ff

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ff.init(0)
    n = args.n
    pts = 1 << args.points_log2
    batch = pts // n
    stream = torch.cuda.current_stream()

    if args.copy_only:
        gbs, t = stream_ceiling(torch, ff, dev, pts, args.steps, args.warmup, stream, False)
        print(json.dumps({"copy_bytes": 2 * pts * 8, "ms": round(t * 1e3, 5), "gb_s": round(gbs, 1)}))
        return
    if args.copy_sweep:
        rows = stream_sweep(torch, ff, dev, pts, args.steps, args.warmup, stream)
        for g, shape in sorted(rows, key=lambda r: -r[0]):
            print(json.dumps({"gb_s": round(g, 1), **shape}))
        return
    # the headline is timed first, like every other leg: correctness check, then
    # SETTLE_S of untimed launches, then exactly --warmup and --steps launches
    var = pick_variant(ff, n, args.variant, args.layout)
    avg, rel, each = bench_fp32(torch, ff, dev, n, pts, var, args.steps, args.warmup, stream, 1234,
                                SETTLE_S, per_launch=50, layout=args.layout)
    if not rel <= 2e-6:
        print(json.dumps({"error": f"fp32 accuracy check failed at N={n}: rel L2 {rel:.3e}"}))
        sys.exit(1)
    # then the measured ceiling: the two fixed copies and the sweep of copy shapes
    plain_gbs, _ = stream_ceiling(torch, ff, dev, pts, 20, 3, stream, False)
    nt_gbs, _ = stream_ceiling(torch, ff, dev, pts, 20, 3, stream, True)
    sweep_rows = [] if args.no_stream_sweep else stream_sweep(torch, ff, dev, pts, 20, 3, stream)
    best_gbs, best_shape = max(sweep_rows, key=lambda r: r[0]) if sweep_rows else (0.0, None)
    ceiling = max(best_gbs, plain_gbs, nt_gbs)
    gpts = pts / avg / 1e9
    # the bytes the workload must move across HBM: each point read and written
    # once, the shared filter once
    alg_bytes = 16.0 * pts + 8.0 * n
    achieved = alg_bytes / avg / 1e9
    model24 = 24.0 * pts / avg / 1e9
    traffic = measured_traffic(n, pts)

    line = {
        "metric": METRIC,
        "value": round(gpts, 3),
        "unit": "Gpoints/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(avg * 1e3, 5),
        "settle_s": SETTLE_S,
        # median / min / max of 50 further launches timed one by one (event pair
        # around each), after the timed region
        "launch_us": {"median": round(float(np.median(each)), 2), "min": round(min(each), 2),
                      "max": round(max(each), 2), "count": len(each)},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"fused fp32 cyclic conv, N={n}, batch {batch} (2^{args.points_log2} points), "
                               f"one shared filter planned on the host, mid=multiply, variant={var}, "
                               f"filter layout={args.layout}",
                   "n": n, "batch": batch, "points": pts, "variant": var, "filter_layout": args.layout},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     # achieved counts these bytes per launch: 16 B per point plus the filter once
                     "bytes_per_launch": int(alg_bytes), "bytes_per_point": 16,
                     "traffic_bytes_per_point": round(traffic / pts, 4) if traffic else None,
                     "frac_of_stream_ceiling": round(achieved / ceiling, 4),
                     # the measured HBM ceiling: the best of the sweep of copy shapes of
                     # fufft_stream_shape_f32 over the same 2^27 points, and the two fixed
                     # shapes of fufft_stream_f32
                     "stream_ceiling_gbs": {"best": round(ceiling, 1), "best_shape": best_shape,
                                            "shapes_timed": len(sweep_rows),
                                            "fixed_plain": round(plain_gbs, 1), "fixed_nt": round(nt_gbs, 1)},
                     "model_24B": {"what": "the reference's 3-pass model (bench_fufft.cu:314-317): it counts the "
                                           "shared filter as a third pass, which the caches serve here, so this "
                                           "figure can exceed the HBM peak",
                                   "bytes_per_point": 24, "achieved": round(model24, 1),
                                   "frac": round(model24 / HBM_PEAK_GBS, 4)}},
        "accuracy": {"rel_l2_vs_fp64_sample": rel},
    }

    # the same workload with the other filter layout.  In digit order that is
    # the reference's own kernel and filter at this N: fufft_pipeline_v16 with
    # mixedrev_host's radix-16 order (bench_fufft.cu:164-165, 218-219), i.e.
    # FUFFT_V16 -- and, when it differs, the plan FUFFT_AUTO takes for a
    # digit-order filter (radix 8 at N = 512, 4096, 8192, the split apply's
    # faster plan) beside it
    other = "dr" if args.layout == "lane" else "lane"
    ovar = "v16" if other == "dr" else pick_variant(ff, n, "fastest", other)
    a, r = bench_fp32(torch, ff, dev, n, pts, ovar, args.sweep_steps, 3, stream, 1234, SETTLE_S, layout=other)
    if not r <= 2e-6:
        print(json.dumps({"error": f"fp32 accuracy check failed at N={n} ({other}): rel L2 {r:.3e}"}))
        sys.exit(1)
    line[f"{other}_layout"] = {"gpoints_s": round(pts / a / 1e9, 3), "ms": round(a * 1e3, 5),
                               "variant": ovar, "frac": frac(16.0 * pts + 8.0 * n, a), "rel_l2": r}
    if other == "dr":
        line["dr_layout"]["plan"] = "the reference's fufft_pipeline_v16 plan and filter order"
        avar = ff.resolve_variant(n, "auto")
        if avar != ovar:
            a, r = bench_fp32(torch, ff, dev, n, pts, avar, args.sweep_steps, 3, stream, 1234, SETTLE_S,
                              layout=other)
            if not r <= 2e-6:
                print(json.dumps({"error": f"fp32 accuracy check failed at N={n} (dr, auto): rel L2 {r:.3e}"}))
                sys.exit(1)
            line["dr_layout"]["auto"] = {"gpoints_s": round(pts / a / 1e9, 3), "ms": round(a * 1e3, 5),
                                         "variant": avar, "rel_l2": r}

    # the reference bench's protocol: one filter per signal, so the filter is a
    # third pass over HBM (24 B/pt physical, the model's bytes)
    if not args.no_per_signal:
        a, r = bench_fp32(torch, ff, dev, n, pts, var, args.sweep_steps, 3, stream, 4321, SETTLE_S,
                          layout=args.layout, per_signal=True)
        if not r <= 2e-6:
            print(json.dumps({"error": f"fp32 per-signal-filter accuracy check failed at N={n}: rel L2 {r:.3e}"}))
            sys.exit(1)
        line["per_signal_filter"] = {
            "what": "one filter per signal (filt_stride = n), the reference bench's own protocol",
            "fp32": {"gpoints_s": round(pts / a / 1e9, 3), "ms": round(a * 1e3, 5), "variant": var,
                     "filter_layout": args.layout, "bytes_per_point": 24,
                     "achieved_gbs": round(24.0 * pts / a / 1e9, 1), "frac": frac(24.0 * pts, a), "rel_l2": r}}
        # the same protocol in the reference's own format as well: its plan
        # (fufft_pipeline_v16) and its digit-order filters, what
        # fufft::ref::fufft_pipeline_v16 runs (bench_fufft.cu:166-169, 218-219)
        a, r = bench_fp32(torch, ff, dev, n, pts, "v16", args.sweep_steps, 3, stream, 4322, SETTLE_S,
                          layout="dr", per_signal=True)
        if not r <= 2e-6:
            print(json.dumps({"error": f"fp32 per-signal digit-order accuracy check failed at N={n}: "
                                       f"rel L2 {r:.3e}"}))
            sys.exit(1)
        line["per_signal_filter"]["fp32_reference_plan"] = {
            "what": "the reference's plan and digit-order filters, one per signal",
            "gpoints_s": round(pts / a / 1e9, 3), "ms": round(a * 1e3, 5), "variant": "v16", "filter_layout": "dr",
            "bytes_per_point": 24, "achieved_gbs": round(24.0 * pts / a / 1e9, 1), "frac": frac(24.0 * pts, a),
            "rel_l2": r}
        # the same two legs at further sizes (the reference's bench runs this
        # protocol at every N, bench_fufft.cu:156-221)
        by_size = {}
        for s in [int(v) for v in args.per_signal_sizes.split(",") if v.strip()]:
            if s == n:
                continue
            legs = {}
            for key, lay, sv in (("lane", "lane", ff.fastest_variant(s, "lane")), ("reference_plan", "dr", "v16")):
                a, r = bench_fp32(torch, ff, dev, s, pts, sv, args.sweep_steps, 3, stream, 4323 + s, SETTLE_S,
                                  layout=lay, per_signal=True)
                if not r <= 2e-6:
                    print(json.dumps({"error": f"fp32 per-signal accuracy check failed at N={s} ({lay}): "
                                               f"rel L2 {r:.3e}"}))
                    sys.exit(1)
                legs[key] = {"gpoints_s": round(pts / a / 1e9, 3), "ms": round(a * 1e3, 5), "variant": sv,
                             "filter_layout": lay, "frac": frac(24.0 * pts, a), "rel_l2": r}
            by_size[str(s)] = legs
        if by_size:
            line["per_signal_filter"]["by_size"] = by_size

    # seconds per call of the rocFFT chain by N: the reference's published
    # ratios are against the vendor chain (README.md:12-13, bench_fufft.cu:201-246)
    chain_s = {}
    if not args.no_vendor:
        vt, vrel = bench_vendor_chain(torch, dev, n, pts, args.sweep_steps, 3, stream, 1234)
        chain_s[n] = vt
        line["vendor_chain"] = {"what": "torch.fft (rocFFT) forward -> multiply -> inverse, same workload",
                                "gpoints_s": round(pts / vt / 1e9, 3), "ms": round(vt * 1e3, 5),
                                "rel_l2": vrel, "fused_speedup": round(vt / avg, 3)}

    sweep = {}
    for s in [int(v) for v in args.sweep.split(",") if v.strip()]:
        if s == n:
            continue
        sv = pick_variant(ff, s, args.variant, args.layout)
        a, r = bench_fp32(torch, ff, dev, s, pts, sv, args.sweep_steps, 3, stream, 77 + s, SETTLE_S,
                          layout=args.layout)
        sweep[str(s)] = {"gpoints_s": round(pts / a / 1e9, 3), "ms": round(a * 1e3, 5),
                         "frac": frac(16.0 * pts + 8.0 * s, a),
                         "model_frac_24B": round(24.0 * pts / a / 1e9 / HBM_PEAK_GBS, 4),
                         "variant": sv, "filter_layout": args.layout, "rel_l2": r}
        if not r <= 2e-6:
            print(json.dumps({"error": f"fp32 accuracy check failed at N={s}: rel L2 {r:.3e}"}))
            sys.exit(1)
        if not args.no_vendor:
            vt_s, vrel_s = bench_vendor_chain(torch, dev, s, pts, args.sweep_steps, 3, stream, 1234 + s)
            chain_s[s] = vt_s
            sweep[str(s)]["rocfft_chain"] = {"gpoints_s": round(pts / vt_s / 1e9, 3), "ms": round(vt_s * 1e3, 5),
                                             "rel_l2": vrel_s}
            sweep[str(s)]["speedup_vs_rocfft"] = round(vt_s / a, 3)
    if sweep:
        line["sweep"] = sweep

    if not args.no_bfp:
        bfp = {}
        for s in [int(v) for v in args.bfp_sizes.split(",") if v.strip()]:
            bv = pick_variant(ff, s, args.variant, args.layout)
            a, r, worst = bench_bfp(torch, ff, dev, s, pts, args.steps if s == n else args.sweep_steps,
                                    args.warmup if s == n else 3, stream, 99 + s, variant=bv, layout=args.layout)
            if not r <= 1e-4:
                print(json.dumps({"error": f"BFP accuracy check failed at N={s}: rel L2 {r:.3e}"}))
                sys.exit(1)
            g = pts / a / 1e9
            # 4 B per point in and out, one exponent byte per 64-point block in and out,
            # the fp32 filter once
            bb = 8.0 * pts + 2.0 * pts / 64 + 8.0 * s
            bfp[str(s)] = {"gpoints_s": round(g, 3), "ms": round(a * 1e3, 5),
                           "bytes_per_point": round(bb / pts, 4), "achieved_gbs": round(bb / a / 1e9, 1),
                           "frac": frac(bb, a), "model_frac_12B": round(12.0 * pts / a / 1e9 / HBM_PEAK_GBS, 4),
                           "rel_l2_vs_fp64_unquantised": r, "worst_signal_rel_l2": worst,
                           "variant": bv, "filter_layout": args.layout}
            if s in chain_s:
                # against the fp32 rocFFT chain at this N (the reference: 4.3-4.5x against cuFFT's)
                bfp[str(s)]["speedup_vs_rocfft"] = round(chain_s[s] / a, 3)
            if s == n:
                # both legs timed the same way: check, SETTLE_S, --warmup, --steps
                bfp[str(s)]["speedup_vs_fp32"] = round(g / gpts, 3)
                # one exponent per signal: the reference's per-transform scale
                a, r, worst = bench_bfp(torch, ff, dev, s, pts, args.sweep_steps, 3, stream, 99 + s, block=s,
                                        variant=bv, layout=args.layout)
                if not r <= 1e-4:
                    print(json.dumps({"error": f"BFP (block = N) accuracy check failed at N={s}: rel L2 {r:.3e}"}))
                    sys.exit(1)
                bfp[str(s)]["block_n"] = {"gpoints_s": round(pts / a / 1e9, 3), "ms": round(a * 1e3, 5),
                                          "rel_l2_vs_fp64_unquantised": r, "worst_signal_rel_l2": worst}
            # the reference's own format (fp32 scale per transform, int16 filter), same plan and layout
            a, r = bench_bfp_scaled(torch, ff, dev, s, pts, args.sweep_steps, 3, stream, 199 + s, variant=bv,
                                    layout=args.layout)
            if not r <= 1e-4:
                print(json.dumps({"error": f"BFP (reference format) accuracy check failed at N={s}: "
                                           f"rel L2 {r:.3e}"}))
                sys.exit(1)
            # 4 B per point in and out, one fp32 scale per transform in and out, the int16 filter once
            rb = 8.0 * pts + 8.0 * pts / s + 4.0 * s
            bfp[str(s)]["reference_format"] = {"gpoints_s": round(pts / a / 1e9, 3), "ms": round(a * 1e3, 5),
                                               "frac": frac(rb, a),
                                               "model_frac_12B": round(12.0 * pts / a / 1e9 / HBM_PEAK_GBS, 4),
                                               "rel_l2_vs_fp64_unquantised": r, "variant": bv,
                                               "filter_layout": args.layout, "filter": "int16, one scale"}
            if s == n and not args.no_per_signal:
                a, r = bench_bfp_scaled(torch, ff, dev, s, pts, args.sweep_steps, 3, stream, 299 + s, variant=bv,
                                        layout=args.layout, per_signal=True)
                if not r <= 1e-4:
                    print(json.dumps({"error": f"BFP (reference format, filter per signal) accuracy check failed "
                                               f"at N={s}: rel L2 {r:.3e}"}))
                    sys.exit(1)
                line.setdefault("per_signal_filter", {})["bfp_reference_format"] = {
                    "gpoints_s": round(pts / a / 1e9, 3), "ms": round(a * 1e3, 5), "variant": bv,
                    "filter_layout": args.layout, "bytes_per_point": 12,
                    "achieved_gbs": round(12.0 * pts / a / 1e9, 1), "frac": frac(12.0 * pts, a),
                    "rel_l2_vs_fp64_unquantised": r}
                # and the reference's own call: its plan and digit-order int16 filters
                # (fufft_pipeline_v16_bfp, bench_fufft.cu:172-178, 220-221)
                a, r = bench_bfp_scaled(torch, ff, dev, s, pts, args.sweep_steps, 3, stream, 399 + s, variant="v16",
                                        layout="dr", per_signal=True)
                if not r <= 1e-4:
                    print(json.dumps({"error": f"BFP (reference call, filter per signal) accuracy check failed "
                                               f"at N={s}: rel L2 {r:.3e}"}))
                    sys.exit(1)
                line["per_signal_filter"]["bfp_reference_plan"] = {
                    "what": "the reference's plan and digit-order int16 filters, one per signal",
                    "gpoints_s": round(pts / a / 1e9, 3), "ms": round(a * 1e3, 5), "variant": "v16",
                    "filter_layout": "dr", "bytes_per_point": 12,
                    "achieved_gbs": round(12.0 * pts / a / 1e9, 1), "frac": frac(12.0 * pts, a),
                    "rel_l2_vs_fp64_unquantised": r}
        line["bfp"] = bfp

    large = {}
    for s in [int(v) for v in args.large_sizes.split(",") if v.strip()]:
        lout, mid = ff.large_plan(s)
        legs = {}
        for lv in ("v16", "r8"):
            a, r = bench_large(torch, ff, dev, s, pts, args.sweep_steps, 3, stream, 5 + s, variant=lv)
            if not r <= 2e-6:
                print(json.dumps({"error": f"four-step accuracy check failed at N={s} ({lv}): rel L2 {r:.3e}"}))
                sys.exit(1)
            model = (4 * lout + 3) * 8
            legs[lv] = {"gpoints_s": round(pts / a / 1e9, 3), "ms": round(a * 1e3, 5),
                        "plan": f"{lout} outer radix-16 level(s) + fused middle N={mid} at "
                                f"{'radix 16 (the reference run_large middle)' if lv == 'v16' else 'radix 8'}",
                        # three passes of 16 B (the two outer levels of a two-level plan
                        # run as one pass); the filter is cache-resident
                        "bytes_per_point": 48, "frac": frac(48.0 * pts, a),
                        # the reference's (4 lout + 3) x 8 B model (bench_fufft.cu:481)
                        "model_bytes_per_point": model,
                        "model_frac": round(model * pts / a / 1e9 / HBM_PEAK_GBS, 4),
                        "rel_l2": r}
        # the default middle (the reference's) with the radix-8 one beside it
        large[str(s)] = {**legs["v16"], "variant": "v16", "r8_middle": legs["r8"]}
        if not args.no_per_signal:
            # the reference's own run_large protocol: one chained filter per
            # transform, a fourth 8 B/pt stream (its 56 B/pt model is then the
            # physical bytes)
            a, r = bench_large(torch, ff, dev, s, pts, args.sweep_steps, 3, stream, 7 + s, variant="v16",
                               per_transform=True)
            if not r <= 2e-6:
                print(json.dumps({"error": f"four-step (filter per transform) accuracy check failed at N={s}: "
                                           f"rel L2 {r:.3e}"}))
                sys.exit(1)
            large[str(s)]["per_transform_filter"] = {
                "what": "one chained filter per transform, as the reference's run_large (fufft::ref::run_large)",
                "gpoints_s": round(pts / a / 1e9, 3), "ms": round(a * 1e3, 5), "bytes_per_point": 56,
                "frac": frac(56.0 * pts, a), "rel_l2": r}
        if not args.no_vendor:
            # the reference times its four-step against the cuFFT chain at this N
            # (bench_fufft.cu:453-478); here rocFFT through torch.fft, same batch
            vt, vrel = bench_vendor_chain(torch, dev, s, pts, args.sweep_steps, 3, stream, 1234 + s, uniform=True)
            large[str(s)]["rocfft_chain"] = {"what": "torch.fft (rocFFT) forward -> multiply -> inverse, same batch",
                                             "gpoints_s": round(pts / vt / 1e9, 3), "ms": round(vt * 1e3, 5),
                                             "rel_l2": vrel}
            large[str(s)]["speedup_vs_rocfft"] = round(vt * 1e3 / legs["v16"]["ms"], 3)
        if ff.supported(s, "v16"):
            # the same size as one fused conv (N = 32768: a workgroup per
            # transform, 32 values per lane), 16 B/pt, both filter layouts
            single = {}
            for lay in ("lane", "dr"):
                a, r = bench_fp32(torch, ff, dev, s, pts, "v16", args.sweep_steps, 3, stream, 6 + s, SETTLE_S,
                                  layout=lay)
                if not r <= 2e-6:
                    print(json.dumps({"error": f"fused conv accuracy check failed at N={s} ({lay}): "
                                               f"rel L2 {r:.3e}"}))
                    sys.exit(1)
                single[lay] = {"gpoints_s": round(pts / a / 1e9, 3), "ms": round(a * 1e3, 5),
                               "bytes_per_point": 16, "frac": frac(16.0 * pts + 8.0 * s, a), "rel_l2": r}
            large[str(s)]["single_launch"] = {
                "what": "fufft_conv_f32 at this N: one launch, the radix-16 plan with 32 values per lane "
                        "(not the reference's four-step chain); N(0,1) signals, one shared filter",
                **single["lane"], "filter_layout": "lane", "dr_filter": single["dr"],
                "speedup_vs_fourstep": round(legs["v16"]["ms"] / single["lane"]["ms"], 3)}
            if "rocfft_chain" in large[str(s)]:
                large[str(s)]["single_launch"]["speedup_vs_rocfft"] = round(
                    large[str(s)]["rocfft_chain"]["ms"] / single["lane"]["ms"], 3)
    if large:
        line["large"] = large

    if not args.no_c2c:
        # the real two-for-one 1D conv at the headline N (two real signals per complex transform)
        r2 = bench_r2(torch, ff, dev, n, pts, args.sweep_steps, 3, stream, 23)
        if not r2["rel_l2"] <= 2e-6:
            print(json.dumps({"error": f"r2 accuracy check failed: rel L2 {r2['rel_l2']:.3e}"}))
            sys.exit(1)
        line["real_two_for_one"] = r2
        c2c = bench_c2c(torch, ff, dev, n, pts, args.sweep_steps, 3, stream, 21)
        if not c2c["rel_l2"] <= 2e-6:
            print(json.dumps({"error": f"C2C accuracy check failed: rel L2 {c2c['rel_l2']:.3e}"}))
            sys.exit(1)
        line["c2c"] = c2c

    if not args.no_2d:
        d2 = bench_2d(torch, ff, dev, pts, args.sweep_steps, 3, stream, 11)
        for k, v in d2.items():
            if not v["rel_l2"] <= 2e-6:
                print(json.dumps({"error": f"2D accuracy check failed ({k}): rel L2 {v['rel_l2']:.3e}"}))
                sys.exit(1)
        line["conv2d"] = d2

    if not args.no_cpu_baseline:
        cores, affinity, quota = usable_cores()
        sizes = sorted({512, 1024, 2048, 4096, n})
        lanes = {s: 8 if pick_variant(ff, s, args.variant, args.layout) == "r8" else 16 for s in sizes}
        cb = cpu_baseline(sizes, [int(v) for v in args.bfp_sizes.split(",") if v.strip()], n,
                          args.cpu_seconds, cores, lanes)
        cb["host"] = {"affinity_cpus": affinity, "cgroup_cpu_quota": quota, "threads": cores}
        line["cpu_baseline"] = cb
    print(json.dumps(line))


if __name__ == "__main__":
    main()
