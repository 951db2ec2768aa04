"""Seeded random configurations of the 1D entry points against the oracle,
bit for bit: the size, lane width, batch (ragged), mid operation, filter
layout, filter stride and aliasing are drawn per case, so combinations the
targeted tests do not list still run.  Every case prints its parameters first.
"""
import os

import numpy as np
import pytest

from conftest import bits_equal, bperm, crandn, lane_major
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SIZES = {"r8": [512, 1024, 2048, 4096, 8192], "v16": [256, 512, 1024, 2048, 4096, 8192, 16384]}
BFP_SIZES = {"r8": [512, 1024, 2048, 4096, 8192], "v16": [1024, 2048, 4096, 8192, 16384]}
OPS = ["conv", "split", "r2", "c2c", "bfp", "bfp_scaled"]


def draw(seed):
    rng = np.random.default_rng(seed)
    op = OPS[seed % len(OPS)]
    variant = ["r8", "v16"][rng.integers(2)]
    sizes = BFP_SIZES[variant] if op == "bfp" else SIZES[variant]               # bfp_scaled: every size
    if op == "conv" and variant == "v16":
        sizes = sizes + [32768]                 # the fused conv alone runs N = 32768 in one launch
    n = int(rng.choice(sizes))
    batch = int(rng.integers(1, max(2, min(37, (1 << 19) // n))))
    return dict(op=op, variant=variant, n=n, batch=batch,
                mid=["mul", "conj", "none"][rng.integers(3)],
                layout=["dr", "lane", "bperm"][rng.integers(3)],
                per_signal=bool(rng.integers(2)), inplace=bool(rng.integers(2)),
                direction=[-1, 1][rng.integers(2)], block=int(2 ** rng.integers(6, int(np.log2(n)) + 1)),
                seed=seed)


def seeds():
    """40 seeds by default; FUFFT_RANDOM_SEEDS=a:b runs seeds a .. b-1 instead (longer sweeps)."""
    spec = os.environ.get("FUFFT_RANDOM_SEEDS")
    if not spec:
        return range(40)
    lo, hi = (int(x) for x in spec.split(":"))
    return range(lo, hi)


@pytest.mark.parametrize("seed", seeds())
def test_random_config(dev, seed):
    import torch
    import fufft_amd as ff
    c = draw(seed)
    print(f"case random {c}", flush=True)
    rng = np.random.default_rng(1000 + seed)
    n, batch, v = c["n"], c["batch"], (8 if c["variant"] == "r8" else 16)
    plan = O.kernel_plan(n, v)
    nf = batch if c["per_signal"] else 1
    fdr = (crandn(rng, (nf, n)) / n).astype(np.complex64).reshape(-1)
    fdev = {"dr": fdr, "lane": lane_major(fdr, n, v), "bperm": bperm(fdr, n, v)}[c["layout"]]
    stride = n if c["per_signal"] else 0
    dt = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    if c["op"] == "conv":
        a = crandn(rng, batch * n)
        da = dt(a)
        out = da if c["inplace"] else torch.empty_like(da)
        ff.conv(da, dt(fdev), out, n=n, batch=batch, filt_stride=stride, mid=c["mid"],
                variant=c["variant"], layout=c["layout"])
        torch.cuda.synchronize()
        assert bits_equal(out.cpu().numpy(), O.conv(a, fdr, n, plan, filt_stride=stride, mid=c["mid"]))
    elif c["op"] == "split":
        a = crandn(rng, batch * n)
        spec = torch.empty(batch * n, dtype=torch.complex64, device=dev)
        ff.fwd(dt(a), spec, n=n, batch=batch, variant=c["variant"])
        out = spec if c["inplace"] else torch.empty_like(spec)
        ff.apply(spec, dt(fdev), out, n=n, batch=batch, spec_stride=n, filt_stride=stride,
                 mid=c["mid"], variant=c["variant"], layout=c["layout"])
        torch.cuda.synchronize()
        want = O.apply(O.fwd(a, n, plan), fdr, n, batch, plan, spec_stride=n, filt_stride=stride,
                       mid=c["mid"])
        assert bits_equal(out.cpu().numpy(), want)
    elif c["op"] == "r2":
        x = rng.uniform(-1, 1, batch * n).astype(np.float32)
        y = rng.uniform(-1, 1, batch * n).astype(np.float32)
        fr = (rng.uniform(-1, 1, (nf, n)) / n).astype(np.complex64)      # real filter taps' spectrum
        taps_plan = np.concatenate([ff.plan_filter(fr[i], n, variant=c["variant"], kind=ff.FILTER_TAPS)
                                    for i in range(nf)])
        fdev2 = {"dr": taps_plan, "lane": lane_major(taps_plan, n, v), "bperm": bperm(taps_plan, n, v)}[c["layout"]]
        u, w = torch.empty(batch * n, device=dev), torch.empty(batch * n, device=dev)
        ff.conv_r2(dt(x), dt(y), dt(fdev2), u, w, n=n, batch=batch, filt_stride=stride,
                   variant=c["variant"], layout=c["layout"])
        torch.cuda.synchronize()
        ou, ow = O.conv_r2(x, y, taps_plan, n, plan, filt_stride=stride)
        assert bits_equal(u.cpu().numpy(), ou) and bits_equal(w.cpu().numpy(), ow)
    elif c["op"] == "c2c":
        a = crandn(rng, batch * n)
        da = dt(a)
        out = da if c["inplace"] else torch.empty_like(da)
        ff.c2c(da, out, n=n, batch=batch, direction=c["direction"], variant=c["variant"])
        torch.cuda.synchronize()
        assert bits_equal(out.cpu().numpy(), O.c2c(a, n, plan, c["direction"]))
    elif c["op"] == "bfp_scaled":
        # the reference's format: fp32 scale per transform, int16 filter (its
        # digit-order words, moved into the drawn layout's slots)
        x = crandn(rng, batch * n) * np.repeat(10.0 ** rng.uniform(-3, 3, batch), n).astype(np.float32)
        q, s = ff.bfp_scaled_quantize(x, n)
        fq, fs = ff.bfp_scaled_quantize(fdr, n)
        fw = fq.view(np.uint32)
        fqdev = {"dr": fw, "lane": lane_major(fw, n, v), "bperm": bperm(fw, n, v)}[c["layout"]].view(np.int16)
        dq, ds = dt(q), dt(s)
        qo, so = (dq, ds) if c["inplace"] else (torch.empty_like(dq), torch.empty_like(ds))
        nofilt = c["mid"] == "none" and c["per_signal"]            # NULL filter where none is read
        ff.conv_bfp16_scaled(dq, ds, None if nofilt else dt(fqdev), None if nofilt else dt(fs), qo, so, n=n,
                             batch=batch, filt_stride=stride, mid=c["mid"], variant=c["variant"],
                             layout=c["layout"])
        torch.cuda.synchronize()
        oq, os_ = O.bfp_scaled_conv(q, s, fq, fs, n, plan, filt_stride=stride, mid=c["mid"])
        assert np.array_equal(so.cpu().numpy().view(np.uint32), os_.view(np.uint32))
        assert np.array_equal(qo.cpu().numpy(), oq)
    else:
        x = crandn(rng, batch * n) * np.repeat(10.0 ** rng.uniform(-3, 3, batch), n).astype(np.float32)
        q, e = ff.bfp_quantize(x, block=c["block"])
        dq, de = dt(q), dt(e)
        qo = dq if c["inplace"] else torch.empty_like(dq)
        eo = de if c["inplace"] else torch.empty_like(de)
        ff.conv_bfp16(dq, de, dt(fdev), qo, eo, n=n, batch=batch, filt_stride=stride, mid=c["mid"],
                      variant=c["variant"], layout=c["layout"], block=c["block"])
        torch.cuda.synchronize()
        oq, oe = O.bfp_conv(q, e, fdr, n, plan, filt_stride=stride, mid=c["mid"], block=c["block"])
        assert np.array_equal(eo.cpu().numpy(), oe) and np.array_equal(qo.cpu().numpy(), oq)
