"""Seeded random configurations of the 2D and four-step entry points against
the oracle, bit for bit: shape, batch (ragged), mid operation, filter order,
per-item filters, broadcast spectra, aliasing and the four-step middle are drawn per case, so
combinations the targeted tests do not list still run.  Every case prints its
parameters first.  FUFFT_RANDOM_SEEDS=a:b runs seeds a .. b-1 instead of the
default 30 (the same variable as the 1D sweep).
"""
import os

import numpy as np
import pytest

from conftest import bits_equal, cols_to_dr, crandn, cuniform, filt2d_dr
from oracle import oracle as O

pytestmark = pytest.mark.gpu

HEIGHTS = [256, 512, 1024, 2048]                 # the column kernels' lengths
SMALL = [8, 16, 32, 64, 128, 256, 512]            # fused small images: h * w <= 8192
WIDTHS = [256, 512, 1024, 2048, 4096, 8192, 16384]
LARGE = [8192, 16384, 32768, 65536, 131072, 262144]
OPS = ["conv2d", "r2_2d", "split2d", "large", "small2d"]
MAX_IMAGE = 1 << 22                               # points per image (every width occurs)
MAX_POINTS = 1 << 21                              # per case beyond one image: the oracle takes a second or two


def draw(seed):
    rng = np.random.default_rng(seed)
    op = OPS[seed % len(OPS)]
    c = dict(op=op, seed=seed, mid=["mul", "conj", "none"][rng.integers(3)],
             layout=["dr", "lane"][rng.integers(2)], per_item=bool(rng.integers(2)),
             inplace=bool(rng.integers(2)), null_filter=bool(rng.integers(2)))
    if op == "small2d":
        h = int(rng.choice(SMALL))
        w = int(rng.choice([x for x in SMALL if h * x <= 8192]))
        c.update(h=h, w=w, batch=int(rng.integers(1, 40)))
    elif op == "large":
        c["n"] = int(rng.choice(LARGE))
        c["batch"] = int(rng.integers(1, max(2, min(5, MAX_POINTS // c["n"] + 1))))
        c["middle"] = ["v16", "r8"][rng.integers(2)]
    else:
        h = int(rng.choice(HEIGHTS))
        w = int(rng.choice([x for x in WIDTHS if h * x <= MAX_IMAGE]))
        c.update(h=h, w=w, batch=int(rng.integers(1, max(2, min(5, MAX_POINTS // (h * w) + 1)))),
                 broadcast=bool(rng.integers(2)))
    return c


def seeds():
    spec = os.environ.get("FUFFT_RANDOM_SEEDS")
    if not spec:
        return range(30)
    lo, hi = (int(x) for x in spec.split(":"))
    return range(lo, hi)


def plans(h, w):
    import fufft_amd as ff
    vr, vc = ff.plan2d(h, w)
    return O.kernel_plan(h, vc), O.kernel_plan(w, vr)


@pytest.mark.parametrize("seed", seeds())
def test_random_config(dev, seed):
    import torch
    import fufft_amd as ff
    c = draw(seed)
    print(f"case random 2d/large {c}", flush=True)
    rng = np.random.default_rng(2000 + seed)
    dt = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    batch, mid = c["batch"], c["mid"]
    nf = batch if c["per_item"] else 1

    if c["op"] == "large":
        n = c["n"]
        lout, mid_n = ff.large_plan(n)
        # the middle drawn for the case: the reference's radix-16 one or radix 8
        plan = O.large_plan(lout, mid_n, ff.large_middle(c["middle"]))
        a = cuniform(rng, batch * n)
        filt = np.concatenate([ff.plan_filter_large(cuniform(rng, n), n, kind=ff.FILTER_TAPS, variant=c["middle"])
                               for _ in range(nf)])
        stride = n if c["per_item"] else 0
        buf = dt(a)
        gfilt = None if (mid == "none" and c["null_filter"]) else dt(filt)
        ff.conv_large(buf, gfilt, n=n, batch=batch, filt_stride=stride, mid=mid, variant=c["middle"])
        torch.cuda.synchronize()
        assert bits_equal(buf.cpu().numpy(), O.conv(a, filt, n, plan, filt_stride=stride, mid=mid))
        return

    h, w, layout = c["h"], c["w"], c["layout"]
    ph, pw = plans(h, w)
    np_ = h * w
    stride = np_ if c["per_item"] else 0
    if c["op"] in ("conv2d", "small2d"):
        a = crandn(rng, batch * np_)
        filt = np.concatenate([ff.plan_filter2d(cuniform(rng, np_), h, w, kind=ff.FILTER_TAPS, layout=layout)
                               for _ in range(nf)])
        da = dt(a)
        out = da if c["inplace"] else torch.empty_like(da)
        gfilt = None if (mid == "none" and c["null_filter"]) else dt(filt)
        ff.conv2d(da, gfilt, out, h, w, batch=batch, filt_stride=stride, mid=mid, layout=layout)
        torch.cuda.synchronize()
        want = O.conv2d(a, filt2d_dr(filt, h, w, layout), h, w, ph, pw, filt_stride=stride, mid=mid)
        assert bits_equal(out.cpu().numpy(), want)
    elif c["op"] == "r2_2d":
        x = rng.uniform(0, 1, batch * np_).astype(np.float32)
        y = rng.uniform(0, 1, batch * np_).astype(np.float32)
        taps = rng.uniform(0, 1, (nf, np_)).astype(np.float32)
        filt = np.concatenate([ff.plan_filter2d(taps[i].astype(np.complex64), h, w, kind=ff.FILTER_TAPS,
                                                layout=layout) for i in range(nf)])
        dx, dy = dt(x), dt(y)
        u, v = (dx, dy) if c["inplace"] else (torch.empty_like(dx), torch.empty_like(dy))
        work = torch.empty(batch * np_, dtype=torch.complex64, device=dev)
        ff.conv2d_r2(dx, dy, dt(filt), u, v, work, h, w, batch, filt_stride=stride, layout=layout)
        torch.cuda.synchronize()
        z = (x + 1j * y).astype(np.complex64)
        want = O.conv2d(z, filt2d_dr(filt, h, w, layout), h, w, ph, pw, filt_stride=stride)
        assert bits_equal(u.cpu().numpy(), np.ascontiguousarray(want.real))
        assert bits_equal(v.cpu().numpy(), np.ascontiguousarray(want.imag))
    else:
        # one spectrum per item, or one broadcast to every item against per-item filters
        ns = 1 if c["broadcast"] else batch
        a = cuniform(rng, ns * np_)
        spec = torch.empty(ns * np_, dtype=torch.complex64, device=dev)
        ff.fwd2d(dt(a), spec, h, w, batch=ns)
        filt = np.concatenate([ff.plan_filter2d(crandn(rng, np_, 1.0 / np_), h, w, fold_inv_n=False,
                                                layout=layout) for _ in range(nf)])
        spec_stride = 0 if c["broadcast"] else np_
        got_spec = spec.cpu().numpy()
        # the output may alias the spectrum only where each item has its own
        out = spec if (c["inplace"] and not c["broadcast"] and batch == ns) else \
            torch.empty(batch * np_, dtype=torch.complex64, device=dev)
        gfilt = None if (mid == "none" and c["null_filter"]) else dt(filt)
        ff.apply2d(spec, gfilt, out, h, w, batch=batch, spec_stride=spec_stride, filt_stride=stride,
                   mid=mid, layout=layout)
        torch.cuda.synchronize()
        assert bits_equal(cols_to_dr(got_spec, h, w), O.fwd2d(a, h, w, ph, pw))
        want = O.apply2d(cols_to_dr(got_spec, h, w), filt2d_dr(filt, h, w, layout), h, w, batch, ph, pw,
                         spec_stride=spec_stride, filt_stride=stride, mid=mid)
        assert bits_equal(out.cpu().numpy(), want)
