"""The fused conv at N = 32768 (wide.hip: one workgroup per transform, 32
values per lane, the radix-16 plan LEAD 8 + three radix-16 passes with two
groups per lane): bit for bit the oracle's restatement of that plan
(kernel_plan(32768, 16), the reference's fufft_pipeline_v16 structure,
fufft.cuh:722-800) for every mid operation, every filter layout, shared and
per-signal filters, in place; at 2^27 points on sampled signals, against fp64
within the fp32 bound; and beyond 4 GiB of per-signal filters, where the
launch is split into chunks.  The four-step call at the same N computes the
reference's run_large chain instead; both agree with fp64."""
import numpy as np
import pytest

from conftest import bits_equal, crandn, cuniform
from oracle import oracle as O

pytestmark = pytest.mark.gpu

N = 32768
TOL_F32 = 2e-6
GIB4 = 1 << 32


def _dt(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


@pytest.mark.parametrize("layout", ["dr", "lane", "bperm"])
@pytest.mark.parametrize("mid", ["mul", "conj", "none"])
@pytest.mark.parametrize("per_signal", [False, True])
def test_wide_equals_oracle(dev, layout, mid, per_signal):
    import torch
    import fufft_amd as ff
    rng = np.random.default_rng(["dr", "lane", "bperm"].index(layout) * 10 + ["mul", "conj", "none"].index(mid) * 2
                                + int(per_signal))
    batch = 5
    nf = batch if per_signal else 1
    a = crandn(rng, batch * N)
    taps = [cuniform(rng, N) for _ in range(nf)]
    filt = np.concatenate([ff.plan_filter(t, N, variant="v16", layout=layout, kind=ff.FILTER_TAPS) for t in taps])
    fdr = np.concatenate([ff.plan_filter(t, N, variant="v16", layout="dr", kind=ff.FILTER_TAPS) for t in taps])
    stride = N if per_signal else 0
    print(f"case wide n={N} layout={layout} mid={mid} per_signal={per_signal}", flush=True)
    x = _dt(a, dev)
    out = torch.full_like(x, 7.0)
    ff.conv(x, _dt(filt, dev), out, N, batch, filt_stride=stride, mid=mid, variant="v16", layout=layout)
    torch.cuda.synchronize()
    want = O.conv(a, fdr, N, O.kernel_plan(N, 16), filt_stride=stride, mid=mid)
    assert bits_equal(out.cpu().numpy(), want)


def test_wide_in_place_and_auto(dev):
    import torch
    import fufft_amd as ff
    rng = np.random.default_rng(3)
    batch = 3
    a = crandn(rng, batch * N)
    fdr = ff.plan_filter(cuniform(rng, N), N, variant="auto", kind=ff.FILTER_TAPS)
    print(f"case wide in place n={N} variant=auto", flush=True)
    x = _dt(a, dev)
    ff.conv(x, _dt(fdr, dev), x, N, batch, variant="auto")
    torch.cuda.synchronize()
    assert bits_equal(x.cpu().numpy(), O.conv(a, fdr, N, O.kernel_plan(N, 16)))


def test_wide_full_batch_against_fp64(dev):
    """2^27 points (BASELINE config 4's size), the lane-major filter: sampled
    signals bit-identical to the oracle and within the fp32 bound of the fp64
    convolution; the four-step call on the same input agrees with fp64 too."""
    import torch
    import fufft_amd as ff
    batch = (1 << 27) // N
    rng = np.random.default_rng(4)
    taps = cuniform(rng, N)
    gen = torch.Generator(device=dev)
    gen.manual_seed(44)
    x = torch.rand(batch * N, dtype=torch.complex64, device=dev, generator=gen) * 2 - (1 + 1j)
    out = torch.empty_like(x)
    filt = _dt(ff.plan_filter(taps, N, variant="v16", layout="lane", kind=ff.FILTER_TAPS), dev)
    print(f"case wide full batch n={N} batch={batch}", flush=True)
    ff.conv(x, filt, out, N, batch, variant="v16", layout="lane")
    big = x.clone()
    ff.conv_large(big, _dt(ff.plan_filter_large(taps, N, kind=ff.FILTER_TAPS), dev), n=N, batch=batch)
    torch.cuda.synchronize()
    idx = np.array([0, 1, batch // 2, batch - 1])
    ti = torch.from_numpy(idx).to(dev)
    a_s = x.view(batch, N)[ti].cpu().numpy()
    got = out.view(batch, N)[ti].cpu().numpy()
    four = big.view(batch, N)[ti].cpu().numpy()
    fdr = ff.plan_filter(taps, N, variant="v16", layout="dr", kind=ff.FILTER_TAPS)
    assert bits_equal(got, O.conv(a_s, fdr, N, O.kernel_plan(N, 16)).reshape(len(idx), N))
    spec = np.fft.fft(taps.astype(np.complex128)) / N
    ref = O.conv_spec_f64(a_s.reshape(-1), spec, N).reshape(len(idx), N)
    assert O.rel_l2(got, ref) <= TOL_F32
    assert O.rel_l2(four, ref) <= TOL_F32


def test_wide_per_signal_filters_beyond_4gib(dev):
    """Per-signal filters above 4 GiB: the launch runs in chunks of 16128
    transforms (4 GiB of filter, a multiple of 256); sampled transforms from
    both sides of the boundary are bit-identical to the oracle."""
    import torch
    import fufft_amd as ff
    chunk = ((GIB4 - 1) // (N * 8)) & ~255
    batch = GIB4 // (N * 8) + 5                     # 4 GiB + 1.25 MiB per array
    gen = torch.Generator(device=dev)
    gen.manual_seed(45)
    x = torch.randn(batch * N, dtype=torch.complex64, device=dev, generator=gen)
    f = torch.randn(batch * N, dtype=torch.complex64, device=dev, generator=gen) / N
    out = torch.empty_like(x)
    assert f.numel() * 8 > GIB4
    idx = [0, chunk - 1, chunk, 2 * chunk - 1 if 2 * chunk < batch else batch - 2, batch - 1]
    print(f"case wide per-signal filters beyond 4 GiB n={N} batch={batch} samples={idx}", flush=True)
    ff.conv(x, f, out, n=N, batch=batch, filt_stride=N, variant="v16")
    torch.cuda.synchronize()
    ti = torch.tensor(idx, device=dev)
    a_s = x.view(batch, N)[ti].cpu().numpy()
    f_s = f.view(batch, N)[ti].cpu().numpy()
    got = out.view(batch, N)[ti].cpu().numpy()
    want = O.conv(a_s, f_s, N, O.kernel_plan(N, 16), filt_stride=N).reshape(len(idx), N)
    assert bits_equal(got, want)
    del x, f, out


@pytest.mark.parametrize("layout", ["dr", "lane", "bperm"])
def test_wide_device_planned_spectra(dev, layout):
    """Natural-order spectra planned on the device at N = 32768 (a gather:
    bit-identical to the host planner) drive the fused conv as the host's do;
    taps are refused at this size (the forward transform exists up to 16384)."""
    import torch
    import fufft_amd as ff
    rng = np.random.default_rng(50 + ["dr", "lane", "bperm"].index(layout))
    count = 3
    specs = crandn(rng, count * N)
    host = np.concatenate([ff.plan_filter(specs[i * N:(i + 1) * N], N, variant="v16", layout=layout)
                           for i in range(count)])
    print(f"case wide device planning n={N} layout={layout}", flush=True)
    d_spec = _dt(specs, dev)
    out = torch.empty_like(d_spec)
    ff.plan_filter_device(d_spec, out, N, count=count, variant="v16", layout=layout)
    torch.cuda.synchronize()
    assert bits_equal(out.cpu().numpy(), host)
    with pytest.raises(ff.FufftError):
        ff.plan_filter_device(d_spec, out, N, count=count, variant="v16", layout=layout, kind=ff.FILTER_TAPS)

