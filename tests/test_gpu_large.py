"""GPU parity of the four-step large-N conv (fufft_conv_large_f32).

Bar: bit-identical to the oracle's monolithic chain with the same radix
sequence (radix-16 outer levels first, then the middle's plan) in table-twiddle
mode -- the reference's own four-step check is "four-step == monolithic"
(verify_kernel.cpp:555) -- and rel L2 <= 2e-6 against fp64.  Both middles run:
"v16" (the default, the reference's run_large middle fufft_pipeline_v16,
bench_fufft.cu:368-386) and "r8".
"""
import numpy as np
import pytest

from conftest import bits_equal, crandn, cuniform
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL_F32 = 2e-6


def to_dev(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def oracle_plan(n, variant="auto"):
    import fufft_amd as ff
    lout, mid = ff.large_plan(n)
    return O.large_plan(lout, mid, ff.large_middle(variant))


def run_large(dev, a, filt, n, filt_stride=0, mid="mul", variant="auto"):
    import torch
    import fufft_amd as ff
    buf = to_dev(a, dev)
    ff.conv_large(buf, to_dev(filt, dev), n=n, batch=a.size // n, filt_stride=filt_stride, mid=mid,
                  variant=variant)
    torch.cuda.synchronize()
    return buf.cpu().numpy().reshape(-1)


@pytest.mark.parametrize("n,batch", [(8192, 4), (16384, 3), (32768, 4), (65536, 2), (131072, 2), (262144, 1), (1048576, 1)])
@pytest.mark.parametrize("mid", ["mul", "conj", "none"])
@pytest.mark.parametrize("variant", ["v16", "r8"])
def test_large_matches_oracle(dev, n, batch, mid, variant, rng):
    import fufft_amd as ff
    a = cuniform(rng, batch * n)
    taps = cuniform(rng, n)
    filt = ff.plan_filter_large(taps, n, kind=ff.FILTER_TAPS, variant=variant)
    plan = oracle_plan(n, variant)
    print(f"case large n={n} batch={batch} mid={mid} variant={variant} plan={plan.radices}", flush=True)
    got = run_large(dev, a, filt, n, mid=mid, variant=variant)
    assert bits_equal(got, O.conv(a, filt, n, plan, mid=mid))
    truth = O.conv_spec_f64(a, np.fft.fft(taps.astype(np.complex128)) / n, n, mid=mid)
    assert O.rel_l2(got, truth) <= TOL_F32


@pytest.mark.parametrize("variant", ["v16", "r8"])
def test_large_per_signal_filter(dev, variant, rng):
    import fufft_amd as ff
    n, batch = 32768, 3
    a = crandn(rng, batch * n)
    specs = crandn(rng, (batch, n), scale=1.0 / n)
    perm = ff.large_digit_order(n, variant)
    fdr = np.ascontiguousarray(specs[:, perm]).reshape(-1)
    print(f"case large per-signal filter variant={variant}", flush=True)
    got = run_large(dev, a, fdr, n, filt_stride=n, variant=variant)
    assert bits_equal(got, O.conv(a, fdr, n, oracle_plan(n, variant), filt_stride=n))
    assert O.rel_l2(got, O.conv_spec_f64(a, specs.reshape(-1), n, spec_stride=n)) <= TOL_F32


def test_large_full_batch_sampled(dev, rng):
    """BASELINE config: N = 32768, batch 4096 (2^27 points): sampled signals
    bit-identical to the oracle, and the batch checked against fp64 on a sample."""
    import torch
    import fufft_amd as ff
    n, batch = 32768, 4096
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    x = (torch.rand(batch * n * 2, device=dev, generator=gen) * 2 - 1).view(torch.complex64)
    taps = cuniform(rng, n)
    filt = to_dev(ff.plan_filter_large(taps, n, kind=ff.FILTER_TAPS), dev)
    idx = [0, 1, 2047, 4095]
    a_s = x.view(batch, n)[idx].cpu().numpy().reshape(-1)
    print("case large full batch 2^27 points", flush=True)
    ff.conv_large(x, filt, n=n, batch=batch)
    torch.cuda.synchronize()
    got_s = x.view(batch, n)[idx].cpu().numpy().reshape(-1)
    assert bits_equal(got_s, O.conv(a_s, filt.cpu().numpy(), n, oracle_plan(n)))
    want = O.conv_spec_f64(a_s, np.fft.fft(taps.astype(np.complex128)) / n, n)
    assert O.rel_l2(got_s, want) <= TOL_F32


def test_large_rejects_bad_args(dev):
    import torch
    import fufft_amd as ff
    buf = torch.zeros(8192 * 2, dtype=torch.complex64, device=dev)
    with pytest.raises(ff.FufftError):
        ff.conv_large(buf, buf, n=4096, batch=1)            # below the four-step range
    with pytest.raises(ValueError):                         # the binding rejects the stride
        ff.conv_large(buf, buf, n=8192, batch=1, filt_stride=5)
    with pytest.raises(ff.FufftError):                      # and so does the library
        ff.check(ff.lib.fufft_conv_large_f32(buf.data_ptr(), buf.data_ptr(), 5, 8192, 1, 0, 2, None),
                 "fufft_conv_large_f32")
    with pytest.raises(ff.FufftError):                      # an unknown middle variant
        ff.check(ff.lib.fufft_conv_large_f32(buf.data_ptr(), buf.data_ptr(), 0, 8192, 1, 0, 9, None),
                 "fufft_conv_large_f32")
    ff.conv_large(buf, buf, n=8192, batch=0)                # empty batch is a no-op
