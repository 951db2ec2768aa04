"""GPU parity of the int16 BFP conv in the reference's own format
(fufft_conv_bfp16_scaled: one fp32 scale per transform, an int16 filter with
one scale, in digit order or the lane-major / bperm slots;
fufft_pipeline_v16_bfp, fufft.cuh:1614-1701).

Bar: int16 words and fp32 scales bit-identical to the oracle's restatement of
kernel_v16_bfp (verify_kernel.cpp:1092-1135) at every size, variant and mid
operation; with the reference's base twiddles, bit-identical to the compiled
reference's own outputs on the golden fixtures; and rel L2 <= 1e-4 against
the fp64 convolution of the unquantised input on BASELINE config-3 input
(per-signal N(0,1) x 10^u, u ~ U[-3, 3]).
"""
import numpy as np
import pytest

from conftest import bperm, crandn, lane_major
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL_BFP = 1e-4
SIZES = [("v16", n) for n in (256, 512, 1024, 2048, 4096, 8192, 16384)] + \
        [("r8", n) for n in (512, 1024, 2048, 4096, 8192)]


def to_dev(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def config3_signals(rng, batch, n):
    x = (crandn(rng, (batch, n)) * (10.0 ** rng.uniform(-3, 3, (batch, 1)))).astype(np.complex64)
    return x.reshape(-1)


def run(dev, q, s, fq, fs, n, batch, filt_stride=0, mid="mul", variant="v16", inplace=False, layout="dr"):
    import torch
    import fufft_amd as ff
    dq, ds = to_dev(q, dev), to_dev(s, dev)
    qo, so = (dq, ds) if inplace else (torch.empty_like(dq), torch.empty_like(ds))
    ff.conv_bfp16_scaled(dq, ds, None if fq is None else to_dev(fq, dev), None if fs is None else to_dev(fs, dev),
                         qo, so, n=n, batch=batch, filt_stride=filt_stride, mid=mid, variant=variant, layout=layout)
    torch.cuda.synchronize()
    return qo.cpu().numpy(), so.cpu().numpy()


@pytest.mark.parametrize("variant,n", SIZES)
@pytest.mark.parametrize("mid", ["mul", "conj", "none"])
def test_scaled_bfp_matches_oracle(dev, variant, n, mid, rng):
    import fufft_amd as ff
    batch = max(3, min(64, 65536 // n)) + 1               # ragged: not a multiple of any group
    x = config3_signals(rng, batch, n)
    x[:n] = 0                                             # an all-zero transform: scale 1e-30 / 32767
    q, s = ff.bfp_scaled_quantize(x, n)
    v = 8 if variant == "r8" else 16
    plan = O.kernel_plan(n, v)
    taps = crandn(rng, n)
    fq, fs = ff.bfp_scaled_quantize(ff.plan_filter(taps, n, variant=variant, kind=ff.FILTER_TAPS), n)
    print(f"case bfp_scaled n={n} variant={variant} mid={mid} batch={batch}", flush=True)
    qo, so = run(dev, q, s, None if mid == "none" else fq, None if mid == "none" else fs, n, batch,
                 mid=mid, variant=variant)
    oq, os_ = O.bfp_scaled_conv(q, s, fq, fs, n, plan, mid=mid)
    assert np.array_equal(so.view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(qo, oq)
    if mid == "mul":
        # accuracy against fp64 on the unquantised input, both quantisations included
        spec = np.fft.fft(taps.astype(np.complex128)) / n
        got = ff.bfp_scaled_dequantize(qo, so, n)[n:]
        want = O.conv_spec_f64(x[n:], spec, n)
        assert O.rel_l2(got, want) <= TOL_BFP


@pytest.mark.parametrize("variant,n", SIZES)
def test_scaled_bfp_filter_layouts(dev, variant, n, rng):
    """The int16 filter in the lane-major pair slots and in the reference's
    bperm slots (the digit-order words moved, the scales unchanged) gives the
    digit-order call's words and scales bit for bit, which equal the oracle's;
    a shared filter with the product and per-signal filters with the
    conjugate product."""
    import fufft_amd as ff
    batch = max(3, min(32, 32768 // n)) + 1
    x = config3_signals(rng, batch, n)
    q, s = ff.bfp_scaled_quantize(x, n)
    v = 8 if variant == "r8" else 16
    taps = crandn(rng, n)
    fq, fs = ff.bfp_scaled_quantize(ff.plan_filter(taps, n, variant=variant, kind=ff.FILTER_TAPS), n)
    lq, ls = ff.bfp_scaled_quantize(ff.plan_filter(taps, n, variant=variant, layout="lane", kind=ff.FILTER_TAPS), n)
    # quantising the lane-major fp32 filter gives the digit-order words in lane-major slots
    assert np.array_equal(lq.view(np.uint32), lane_major(fq.view(np.uint32), n, v)) and np.array_equal(ls, fs)
    pf = (crandn(rng, (batch, n)) / n).astype(np.complex64).reshape(-1)
    for stride, mid, (fq, fs) in ((0, "mul", (fq, fs)), (n, "conj", ff.bfp_scaled_quantize(pf, n))):
        print(f"case bfp_scaled layouts n={n} variant={variant} mid={mid} filt_stride={stride}", flush=True)
        wq, ws = run(dev, q, s, fq, fs, n, batch, filt_stride=stride, mid=mid, variant=variant)
        oq, os_ = O.bfp_scaled_conv(q, s, fq, fs, n, O.kernel_plan(n, v), filt_stride=stride, mid=mid)
        assert np.array_equal(wq, oq) and np.array_equal(ws.view(np.uint32), os_.view(np.uint32))
        for layout, move in (("lane", lane_major), ("bperm", bperm)):
            mq = move(fq.view(np.uint32), n, v).view(np.int16)
            gq, gs = run(dev, q, s, mq, fs, n, batch, filt_stride=stride, mid=mid, variant=variant, layout=layout)
            assert np.array_equal(gq, wq), layout
            assert np.array_equal(gs.view(np.uint32), ws.view(np.uint32)), layout


@pytest.mark.parametrize("variant,n", [("v16", 512), ("r8", 4096), ("v16", 16384)])
def test_scaled_bfp_per_signal_filters_in_place(dev, variant, n, rng):
    import fufft_amd as ff
    batch = 5
    x = config3_signals(rng, batch, n)
    q, s = ff.bfp_scaled_quantize(x, n)
    v = 8 if variant == "r8" else 16
    fdr = (crandn(rng, (batch, n)) / n).astype(np.complex64).reshape(-1)
    fq, fs = ff.bfp_scaled_quantize(fdr, n)
    print(f"case bfp_scaled per-signal filters in place n={n} variant={variant}", flush=True)
    qo, so = run(dev, q, s, fq, fs, n, batch, filt_stride=n, variant=variant, inplace=True)
    oq, os_ = O.bfp_scaled_conv(q, s, fq, fs, n, O.kernel_plan(n, v), filt_stride=n)
    assert np.array_equal(qo, oq) and np.array_equal(so.view(np.uint32), os_.view(np.uint32))


@pytest.mark.parametrize("n", [512, 4096])
def test_scaled_bfp_full_batch_config3(dev, n):
    """BASELINE config 3's shape (2^27 points, batch 2^27 / n) in the reference's
    format at its plan (radix 16): sampled transforms bit-identical to the
    oracle, and within 1e-4 of fp64 on the unquantised input."""
    import torch
    import fufft_amd as ff
    rng = np.random.default_rng(3000 + n)
    batch = (1 << 27) // n
    pick = np.unique(np.concatenate([[0, 1, batch - 1], rng.integers(0, batch, 29)]))
    # the batch is generated on the GPU; the sampled transforms are drawn on the host
    dq = torch.randint(-32767, 32767, (2 * n * batch,), dtype=torch.int16, device=dev)
    ds = torch.exp(torch.empty(batch, device=dev).uniform_(-7, 7)).float() / 32767.0
    xs = config3_signals(rng, pick.size, n)
    qs, ss = ff.bfp_scaled_quantize(xs, n)
    idx = torch.from_numpy(pick).to(dev)
    dq.view(batch, 2 * n)[idx] = to_dev(qs.reshape(-1, 2 * n), dev)
    ds[idx] = to_dev(ss, dev)
    taps = crandn(rng, n)
    fq, fs = ff.bfp_scaled_quantize(ff.plan_filter(taps, n, variant="v16", kind=ff.FILTER_TAPS), n)
    qo, so = torch.empty_like(dq), torch.empty_like(ds)
    print(f"case bfp_scaled full batch n={n} batch={batch}", flush=True)
    ff.conv_bfp16_scaled(dq, ds, to_dev(fq, dev), to_dev(fs, dev), qo, so, n=n, batch=batch, variant="v16")
    torch.cuda.synchronize()
    gq = qo.view(batch, 2 * n)[idx].cpu().numpy().reshape(-1)
    gs = so[idx].cpu().numpy()
    oq, os_ = O.bfp_scaled_conv(qs, ss, fq, fs, n, O.kernel_plan(n, 16))
    assert np.array_equal(gq, oq) and np.array_equal(gs.view(np.uint32), os_.view(np.uint32))
    spec = np.fft.fft(taps.astype(np.complex128)) / n
    got = ff.bfp_scaled_dequantize(gq, gs, n)
    assert O.rel_l2(got, O.conv_spec_f64(xs, spec, n)) <= TOL_BFP


def test_scaled_bfp_rejects_bad_arguments(dev):
    import torch
    import fufft_amd as ff
    n = 4096
    q = torch.zeros(2 * n * 2, dtype=torch.int16, device=dev)
    s = torch.ones(2, device=dev)
    fq = torch.zeros(2 * n, dtype=torch.int16, device=dev)
    fs = torch.ones(1, device=dev)
    with pytest.raises(ff.FufftError):                    # radix 8 needs n >= 512
        ff.conv_bfp16_scaled(q, s, fq, fs, q, s, n=256, batch=2, variant="r8")
    with pytest.raises(ff.FufftError):                    # a filter stride neither 0 nor n
        ff.check(ff.lib.fufft_conv_bfp16_scaled(q.data_ptr(), s.data_ptr(), fq.data_ptr(), fs.data_ptr(), 7,
                                                q.data_ptr(), s.data_ptr(), n, 2, 0, 0, 0, None), "stride")
    with pytest.raises(ff.FufftError):                    # a misaligned filter
        ff.check(ff.lib.fufft_conv_bfp16_scaled(q.data_ptr(), s.data_ptr(), fq.data_ptr() + 4, fs.data_ptr(), 0,
                                                q.data_ptr(), s.data_ptr(), n, 2, 0, 0, 0, None), "align")
    # an empty batch is a no-op
    ff.conv_bfp16_scaled(q, s, fq, fs, q, s, n=n, batch=0)
