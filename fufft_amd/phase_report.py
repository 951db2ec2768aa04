"""Phase-timer report of the fused conv (the counterpart of the reference's
in-kernel timer read-out, fufft.cuh:86-176).

Runs fufft_conv_timed_f32 on one batch, decodes every workgroup's record and
prints one JSON object: median cycles per phase and their shares, the shader
clock each workgroup ran at (its cycles over the constant 100 MHz clock across
the same marks), workgroups per XCD, how many workgroups a CU holds at once on
average and the gap between one leaving and the next starting there, and the
cost of the marks themselves (timed / untimed launch time).

    python -m fufft_amd.phase_report [--n 4096] [--points-log2 27] [--variant fastest] [--layout lane]

The filter is planned in --layout (default the lane-major pairs) at
--variant ("fastest": fufft_fastest_variant for that layout, as bench.py).
"""
from __future__ import annotations

import argparse
import json

import numpy as np


def residency(rec: dict) -> tuple[float, float]:
    """(workgroups live on a CU on average over the launch, median cycles from
    the latest end of a workgroup on a CU to the next start there).  A CU is
    (XCD, HW_ID bits 8-15: CU, shader array, shader engine); start and end are
    the workgroup's first and last shader-clock marks."""
    start = rec["start"]
    end = start + rec["total_cycles"]
    cu = rec["xcd"] * 256 + ((rec["hw_id"] >> 8) & 0xFF)
    live, gaps = [], []
    for c in np.unique(cu):
        m = cu == c
        s, e = np.sort(start[m]), np.sort(end[m])
        live.append(float((end[m] - start[m]).sum()) / float(e.max() - s.min()))
        i = np.searchsorted(e, s) - 1
        gaps.append(s[i >= 0] - e[i[i >= 0]])
    return round(float(np.mean(live)), 3), float(np.median(np.concatenate(gaps)))


def run(n: int, points_log2: int, variant: str, mid: str = "mul", reps: int = 20, layout: str = "lane") -> dict:
    import torch
    import fufft_amd as ff

    dev = torch.device("cuda:0")
    ff.init(0)
    if variant == "fastest":
        variant = ff.fastest_variant(n, layout)
    batch = (1 << points_log2) // n
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    a = torch.randn(batch * n, dtype=torch.complex64, device=dev, generator=gen)
    out = torch.empty_like(a)
    rng = np.random.default_rng(3)
    taps = (rng.standard_normal(n) + 1j * rng.standard_normal(n)).astype(np.complex64)
    filt = torch.from_numpy(ff.plan_filter(taps, n, variant=variant, layout=layout, kind=ff.FILTER_TAPS)).to(dev)
    tpw = ff.transforms_per_workgroup(n, variant)
    groups = -(-batch // tpw)
    timing = torch.zeros(groups * ff.TIMER_STRIDE, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream()

    def timed():
        ff.conv_timed(a, filt, out, timing, n=n, batch=batch, timing_groups=groups, mid=mid,
                      variant=variant, layout=layout, stream=stream)

    def plain():
        ff.conv(a, filt, out, n=n, batch=batch, mid=mid, variant=variant, layout=layout, stream=stream)

    def clock(fn):
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3 / reps

    clock(plain)                                   # warm both paths, then measure
    t_timed = clock(timed)
    t_plain = clock(plain)
    t_timed = min(t_timed, clock(timed))
    rec = ff.decode_timing(timing.cpu().numpy().view(np.uint32))

    phases = {k: float(np.median(v)) for k, v in rec["phase_cycles"].items()}
    total = float(np.median(rec["total_cycles"]))
    ok = rec["realtime_ticks"] > 0
    mhz = rec["total_cycles"][ok] / (rec["realtime_ticks"][ok] / 100.0)
    per_xcd = {int(x): int(c) for x, c in zip(*np.unique(rec["xcd"], return_counts=True))}
    live, gap = residency(rec)
    return {
        "what": "fused fp32 conv, in-kernel phase timer (s_memtime after s_waitcnt + workgroup barrier)",
        "n": n, "batch": batch, "variant": ff.resolve_variant(n, variant), "filter_layout": layout, "mid": mid,
        "workgroups": int(groups), "transforms_per_workgroup": int(tpw),
        "median_cycles": {**{k: round(v, 1) for k, v in phases.items()}, "total": total},
        "share": {k: round(v / total, 4) for k, v in phases.items()},
        "shader_clock_mhz": {"median": round(float(np.median(mhz)), 1),
                             "p5": round(float(np.percentile(mhz, 5)), 1),
                             "p95": round(float(np.percentile(mhz, 95)), 1)},
        "median_us_per_workgroup": round(float(np.median(rec["realtime_ticks"])) / 100.0, 3),
        "workgroups_per_xcd": per_xcd,
        "live_workgroups_per_cu": live, "start_gap_cycles": gap,
        "ms_untimed": round(t_plain * 1e3, 5), "ms_timed": round(t_timed * 1e3, 5),
        "timer_overhead": round(t_timed / t_plain, 3),
    }


def main() -> None:
    p = argparse.ArgumentParser()
    p.add_argument("--n", type=int, default=4096)
    p.add_argument("--points-log2", type=int, default=27)
    p.add_argument("--variant", default="fastest")
    p.add_argument("--layout", default="lane", choices=["lane", "dr"])
    p.add_argument("--mid", default="mul")
    a = p.parse_args()
    print(json.dumps(run(a.n, a.points_log2, a.variant, a.mid, layout=a.layout)))


if __name__ == "__main__":
    main()
