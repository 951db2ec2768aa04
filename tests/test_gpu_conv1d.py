"""GPU parity of the 1D fused path (fufft_conv_f32 / fwd / apply / conv_r2).

Bar: bit-identical to the oracle in table-twiddle mode (same operation order,
same twiddle table, -ffp-contract=off on both sides), and rel L2 <= 2e-6
against fp64 (the north_star bound for fp32).
"""
import numpy as np
import pytest

from conftest import bits_equal, bperm, crandn, cuniform, lane_major
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL_F32 = 2e-6
V = {"v16": 16, "r8": 8}
SIZES = [("v16", n) for n in (256, 512, 1024, 2048, 4096, 8192, 16384)] + \
        [("r8", n) for n in (512, 1024, 2048, 4096, 8192)]


def to_dev(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def from_dev(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def run_conv(dev, a, filt, n, filt_stride, mid, variant, layout, inplace=False):
    import torch
    import fufft_amd as ff
    da = to_dev(a, dev)
    df = to_dev(filt, dev)
    dout = da if inplace else torch.empty_like(da)
    ff.conv(da, df, dout, n=n, batch=a.size // n, filt_stride=filt_stride, mid=mid,
            variant=variant, layout=layout)
    return from_dev(dout).reshape(-1)


@pytest.mark.parametrize("variant,n", SIZES)
@pytest.mark.parametrize("mid", ["mul", "conj", "none"])
def test_conv_matches_oracle_bitwise(dev, variant, n, mid, rng):
    batch = max(4, 65536 // n)
    a = crandn(rng, (batch, n))
    spec = crandn(rng, n) / n
    plan = O.kernel_plan(n, V[variant])
    fdr = spec[O.mixedrev(plan)]
    print(f"case conv variant={variant} n={n} mid={mid} batch={batch}", flush=True)
    got = run_conv(dev, a, fdr, n, 0, mid, variant, "dr")
    want = O.conv(a, fdr, n, plan, filt_stride=0, mid=mid)
    assert bits_equal(got, want)
    truth = O.conv_spec_f64(a[:8], spec, n, mid=mid)
    assert O.rel_l2(got[:8 * n], truth) <= TOL_F32


@pytest.mark.parametrize("variant,n", [("v16", 512), ("v16", 1024), ("v16", 2048), ("v16", 4096), ("r8", 512),
                                       ("r8", 1024)])
def test_per_signal_filter_and_lane_layout(dev, variant, n, rng):
    batch = 64
    v = V[variant]
    a = cuniform(rng, (batch, n))
    spec = cuniform(rng, (batch, n)) / n
    plan = O.kernel_plan(n, v)
    fdr = np.ascontiguousarray(spec[:, O.mixedrev(plan)]).reshape(-1)
    want = O.conv(a, fdr, n, plan, filt_stride=n)
    print(f"case per-signal variant={variant} n={n}", flush=True)
    assert bits_equal(run_conv(dev, a, fdr, n, n, "mul", variant, "dr"), want)
    assert bits_equal(run_conv(dev, a, lane_major(fdr, n, v), n, n, "mul", variant, "lane"), want)
    # the reference's own bperm layout (fufft_pipeline_v16f's filter) passes as it is
    assert bits_equal(run_conv(dev, a, bperm(fdr, n, v), n, n, "mul", variant, "bperm"), want)


@pytest.mark.parametrize("mid", ["mul", "conj"])
@pytest.mark.parametrize("inplace", [False, True])
@pytest.mark.parametrize("layout", ["lane", "dr"])
def test_per_signal_filters_n4096_full_batch(dev, mid, inplace, layout):
    """One filter per signal at N = 4096, radix 16 (the reference bench's
    protocol; with the digit-order filter, its exact call): the library runs
    the kernels that issue each signal's filter loads with its signal loads
    (lane-major pairs, or the digit order's 1 KiB runs handed to the lanes
    through LDS).  2^27 points, filters planned on the device from random
    spectra; 16 signals across the batch bit-identical to the oracle, which
    reads the same filters planned in digit order."""
    import torch
    import fufft_amd as ff
    n, batch = 4096, (1 << 27) // 4096
    gen = torch.Generator(device=dev)
    gen.manual_seed(4096 + inplace)
    x = torch.randn(batch * n, dtype=torch.complex64, device=dev, generator=gen)
    spec = torch.randn(batch * n, dtype=torch.complex64, device=dev, generator=gen)
    flane = torch.empty_like(spec)
    ff.plan_filter_device(spec, flane, n, count=batch, variant="v16", layout=layout, kind=ff.FILTER_SPECTRUM)
    idx = torch.from_numpy(np.linspace(0, batch - 1, 16).astype(np.int64)).to(dev)
    a_s = x.view(batch, n)[idx].cpu().numpy()
    s_s = spec.view(batch, n)[idx].contiguous()
    del spec
    fdr_s = torch.empty_like(s_s)
    ff.plan_filter_device(s_s, fdr_s, n, count=16, variant="v16", layout="dr", kind=ff.FILTER_SPECTRUM)
    out = x if inplace else torch.empty_like(x)
    print(f"case per-signal {layout} filters n=4096 full batch mid={mid} inplace={inplace}", flush=True)
    ff.conv(x, flane, out, n=n, batch=batch, filt_stride=n, mid=mid, variant="v16", layout=layout)
    torch.cuda.synchronize()
    got = out.view(batch, n)[idx].cpu().numpy().reshape(-1)
    want = O.conv(a_s, fdr_s.cpu().numpy(), n, O.kernel_plan(n, 16), filt_stride=n, mid=mid)
    assert bits_equal(got, want)
    del x, flane, out


@pytest.mark.parametrize("n", [1024, 4096])
def test_in_place(dev, n, rng):
    a = crandn(rng, (32, n))
    spec = crandn(rng, n) / n
    plan = O.kernel_plan(n, 16)
    fdr = spec[O.mixedrev(plan)]
    print(f"case in-place n={n}", flush=True)
    assert bits_equal(run_conv(dev, a, fdr, n, 0, "mul", "v16", "dr", inplace=True),
                      O.conv(a, fdr, n, plan))


@pytest.mark.parametrize("variant,n", [("v16", 512), ("v16", 2048), ("r8", 512), ("r8", 4096)])
def test_split_fwd_apply_bit_identical_to_fused(dev, variant, n, rng):
    import torch
    import fufft_amd as ff
    batch = 16
    a = crandn(rng, (batch, n))
    spec = crandn(rng, (batch, n)) / n
    plan = O.kernel_plan(n, V[variant])
    fdr = np.ascontiguousarray(spec[:, O.mixedrev(plan)]).reshape(-1)
    print(f"case split variant={variant} n={n}", flush=True)
    da, df = to_dev(a, dev), to_dev(fdr, dev)
    dspec, dout = torch.empty_like(da), torch.empty_like(da)
    ff.fwd(da, dspec, n=n, batch=batch, variant=variant)
    ff.apply(dspec, df, dout, n=n, batch=batch, spec_stride=n, filt_stride=n, variant=variant)
    assert bits_equal(from_dev(dspec).reshape(-1), O.fwd(a, n, plan))
    fused = run_conv(dev, a, fdr, n, n, "mul", variant, "dr")
    assert bits_equal(from_dev(dout).reshape(-1), fused)


def test_split_broadcast_one_spectrum_many_filters(dev, rng):
    """one signal forward once, then applied against 256 filters"""
    import torch
    import fufft_amd as ff
    n, nf = 4096, 256
    a = crandn(rng, (1, n))
    filters = crandn(rng, (nf, n)) / n
    plan = O.kernel_plan(n, 16)
    fdr = np.ascontiguousarray(filters[:, O.mixedrev(plan)]).reshape(-1)
    print("case split broadcast", flush=True)
    da, df = to_dev(a, dev), to_dev(fdr, dev)
    dspec = torch.empty_like(da)
    dout = torch.empty((nf * n,), dtype=torch.complex64, device=dev)
    ff.fwd(da, dspec, n=n, batch=1, variant="v16")
    ff.apply(dspec, df, dout, n=n, batch=nf, spec_stride=0, filt_stride=n, variant="v16")
    got = from_dev(dout)
    spec1 = O.fwd(a, n, plan)
    assert bits_equal(got, O.apply(spec1, fdr, n, nf, plan, spec_stride=0, filt_stride=n))
    truth = O.conv_spec_f64(np.repeat(a, 4, axis=0), filters[:4], n, spec_stride=n)
    assert O.rel_l2(got[:4 * n], truth) <= TOL_F32


@pytest.mark.parametrize("variant,n", [("v16", 512), ("r8", 512), ("v16", 4096)])
def test_conv_r2_two_real_signals(dev, variant, n, rng):
    import torch
    import fufft_amd as ff
    batch = 32
    x = rng.uniform(0, 1, (batch, n)).astype(np.float32)
    y = rng.uniform(0, 1, (batch, n)).astype(np.float32)
    h = rng.uniform(0, 1, n)
    spec = (np.fft.fft(h) / n).astype(np.complex64)           # spectrum of a REAL filter
    plan = O.kernel_plan(n, V[variant])
    fdr = spec[O.mixedrev(plan)]
    print(f"case r2 variant={variant} n={n}", flush=True)
    dx, dy, df = to_dev(x, dev), to_dev(y, dev), to_dev(fdr, dev)
    du, dv = torch.empty_like(dx), torch.empty_like(dy)
    ff.conv_r2(dx, dy, df, du, dv, n=n, batch=batch, variant=variant)
    u, v = from_dev(du).reshape(-1), from_dev(dv).reshape(-1)
    ou, ov = O.conv_r2(x, y, fdr, n, plan)
    assert bits_equal(u, ou) and bits_equal(v, ov)
    # packed-real equals the complex kernel on x + iy
    z = run_conv(dev, (x + 1j * y).astype(np.complex64), fdr, n, 0, "mul", variant, "dr")
    assert bits_equal(u, z.real.copy()) and bits_equal(v, z.imag.copy())
    truth = np.real(np.fft.ifft(np.fft.fft(x[:2].astype(np.float64), axis=1) * np.fft.fft(h)[None], axis=1))
    assert O.rel_l2(u[:2 * n], truth.reshape(-1)) <= TOL_F32


def test_full_size_properties(dev, rng):
    """The bench workload size (2^27 points): every signal is checked through
    linearity against an oracle sample and a checksum of the round trip."""
    import torch
    import fufft_amd as ff
    n, batch = 4096, (1 << 27) // 4096
    torch.manual_seed(7)
    da = torch.randn(batch * n, dtype=torch.complex64, device=dev)
    spec = crandn(rng, n) / n
    plan = O.kernel_plan(n, 16)
    df = to_dev(spec[O.mixedrev(plan)], dev)
    dout = torch.empty_like(da)
    print("case full-size n=4096 batch=32768", flush=True)
    ff.conv(da, df, dout, n=n, batch=batch, variant="v16")
    # sample 64 signals spread over the batch: bit-identical to the oracle
    idx = np.linspace(0, batch - 1, 64).astype(np.int64)
    a_s = da.view(batch, n)[torch.from_numpy(idx).to(dev)].cpu().numpy()
    got_s = dout.view(batch, n)[torch.from_numpy(idx).to(dev)].cpu().numpy()
    assert bits_equal(got_s.reshape(-1), O.conv(a_s, spec[O.mixedrev(plan)], n, plan))
    # round trip with no mid operation returns N * input for every signal
    ff.conv(da, df, dout, n=n, batch=batch, mid="none", variant="v16")
    err = torch.linalg.vector_norm(dout / n - da) / torch.linalg.vector_norm(da)
    assert float(err) < 1e-6


@pytest.mark.parametrize("layout", ["dr", "lane"])
@pytest.mark.parametrize("variant,n", SIZES)
def test_full_batch_every_size(dev, variant, n, layout):
    """2^27 points at every size and both filter layouts: full occupancy, every
    workgroup slot of the GPU busy, where an exchange race would show; 16
    signals spread over the batch (first and last included) bit-identical to
    the oracle."""
    import torch
    import fufft_amd as ff
    batch = (1 << 27) // n
    gen = torch.Generator(device=dev)
    gen.manual_seed(n + 16 * V[variant])
    da = torch.randn(batch * n, dtype=torch.complex64, device=dev, generator=gen)
    rng = np.random.default_rng(n)
    spec = crandn(rng, n) / n
    plan = O.kernel_plan(n, V[variant])
    fdr = spec[O.mixedrev(plan)]
    dout = torch.empty_like(da)
    fdev = lane_major(fdr, n, V[variant]) if layout == "lane" else fdr
    print(f"case full-batch variant={variant} n={n} layout={layout} batch={batch}", flush=True)
    ff.conv(da, to_dev(fdev, dev), dout, n=n, batch=batch, variant=variant, layout=layout)
    idx = torch.from_numpy(np.linspace(0, batch - 1, 16).astype(np.int64)).to(dev)
    a_s = da.view(batch, n)[idx].cpu().numpy()
    got = dout.view(batch, n)[idx].cpu().numpy().reshape(-1)
    assert bits_equal(got, O.conv(a_s, fdr, n, plan))
    del da, dout


def test_empty_batch_is_noop(dev):
    import torch
    import fufft_amd as ff
    d = torch.zeros(4096, dtype=torch.complex64, device=dev)
    ff.conv(d, d, d, n=4096, batch=0)


def test_config1_every_signal_against_fp64(dev):
    """BASELINE config 1 exactly: N = 1024, batch 8192, Re/Im U[-1, 1) from a
    seed, one shared filter of N taps U[-1, 1) planned on the host (fp64
    spectrum, 1/N, digit order), every one of the 8192 outputs bit-identical to
    the oracle and within 2e-6 of the fp64 convolution."""
    import torch
    import fufft_amd as ff
    n, batch = 1024, 8192
    g = np.random.default_rng(1024)
    a = (g.uniform(-1, 1, (batch, n)) + 1j * g.uniform(-1, 1, (batch, n))).astype(np.complex64)
    taps = (g.uniform(-1, 1, n) + 1j * g.uniform(-1, 1, n)).astype(np.complex64)
    filt = ff.plan_filter(taps, n, "auto", kind=ff.FILTER_TAPS)
    print("case config1 n=1024 batch=8192", flush=True)
    got = run_conv(dev, a, filt, n, 0, "mul", "auto", "dr")
    assert bits_equal(got, O.conv(a, filt, n, O.kernel_plan(n, V[ff.resolve_variant(n, "auto")])))
    want = np.fft.ifft(np.fft.fft(a.astype(np.complex128), axis=1)
                       * np.fft.fft(taps.astype(np.complex128))[None, :], axis=1)
    per = np.linalg.norm(got.reshape(batch, n) - want, axis=1) / np.linalg.norm(want, axis=1)
    assert O.rel_l2(got, want.reshape(-1)) <= TOL_F32 and per.max() <= 4 * TOL_F32
