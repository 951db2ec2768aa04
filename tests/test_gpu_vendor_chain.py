"""The vendor-library chain as an on-GPU cross-check of the fused kernels.

The reference's benchmark runs the cuFFT chain (forward C2C -> pointwise
multiply -> inverse C2C) first and checks every fused kernel -- radix 8,
radix 16 and int16-BFP -- against that chain's output on the same data
(bench_fufft.cu:201-246).  On MI355X the chain is torch.fft, which calls
rocFFT.  For every BASELINE configs[1] size (N = 512..4096, Re/Im N(0,1),
one shared filter) the chain and the fused conv at both lane widths run on
the same device input, and:

  - each is within 2e-6 (rel L2) of an fp64 FFT convolution (numpy);
  - the fused output is within 4e-6 of the chain's (the two bounds added);
  - the int16-BFP conv (input quantised by the library codec, 64-point
    blocks) is within 1e-4 of the chain, as the reference checks it;
  - at BASELINE configs[3]'s N = 32768 and 65536 the four-step (both
    middles) and the single-launch conv meet the same fp32 bounds against
    the chain, as the reference checks run_large (bench_fufft.cu:453-464).
"""
import numpy as np
import pytest

from conftest import crandn

pytestmark = pytest.mark.gpu

TOL_F32 = 2e-6
TOL_BFP = 1e-4


def rel_l2(x, y):
    return float(np.linalg.norm(np.asarray(x) - np.asarray(y)) / np.linalg.norm(np.asarray(y)))


@pytest.mark.parametrize("n", [512, 1024, 2048, 4096])
def test_fused_agrees_with_rocfft_chain(dev, n, rng):
    import torch
    import fufft_amd as ff
    batch = (1 << 20) // n
    a = crandn(rng, (batch, n))
    taps = crandn(rng, n)
    x = torch.from_numpy(a).to(dev)
    spec = torch.fft.fft(torch.from_numpy(taps).to(dev))
    print(f"case vendor chain n={n} batch={batch}", flush=True)
    chain = torch.fft.ifft(torch.fft.fft(x, dim=1) * spec, dim=1)
    torch.cuda.synchronize()
    chain_h = chain.cpu().numpy()
    truth = np.fft.ifft(np.fft.fft(a.astype(np.complex128), axis=1)
                        * np.fft.fft(taps.astype(np.complex128))[None, :], axis=1)
    assert rel_l2(chain_h, truth) <= TOL_F32
    for variant in ("r8", "v16"):
        if not ff.supported(n, variant):
            continue
        filt = torch.from_numpy(ff.plan_filter(taps, n, variant=variant, kind=ff.FILTER_TAPS)).to(dev)
        out = torch.empty_like(x)
        ff.conv(x, filt, out, n=n, batch=batch, variant=variant)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        e_truth, e_chain = rel_l2(got, truth), rel_l2(got, chain_h)
        print(f"  {variant}: vs fp64 {e_truth:.2e}, vs rocFFT chain {e_chain:.2e}", flush=True)
        assert e_truth <= TOL_F32
        assert e_chain <= 2 * TOL_F32


@pytest.mark.parametrize("n", [512, 4096])
def test_bfp_agrees_with_rocfft_chain(dev, n, rng):
    import torch
    import fufft_amd as ff
    batch = (1 << 20) // n
    a = crandn(rng, (batch, n))
    taps = crandn(rng, n)
    q, e = ff.bfp_quantize(a)
    x = torch.from_numpy(a).to(dev)
    spec = torch.fft.fft(torch.from_numpy(taps).to(dev))
    print(f"case vendor chain bfp n={n} batch={batch}", flush=True)
    chain = torch.fft.ifft(torch.fft.fft(x, dim=1) * spec, dim=1).cpu().numpy()
    filt = torch.from_numpy(ff.plan_filter(taps, n, kind=ff.FILTER_TAPS)).to(dev)
    dq, de = torch.from_numpy(q).to(dev), torch.from_numpy(e).to(dev)
    qo, eo = torch.empty_like(dq), torch.empty_like(de)
    ff.conv_bfp16(dq, de, filt, qo, eo, n=n, batch=batch)
    torch.cuda.synchronize()
    got = ff.bfp_dequantize(qo.cpu().numpy(), eo.cpu().numpy()).reshape(batch, n)
    err = rel_l2(got, chain)
    print(f"  bfp: vs rocFFT chain {err:.2e}", flush=True)
    assert err <= TOL_BFP


@pytest.mark.parametrize("n", [32768, 65536])
def test_fourstep_agrees_with_rocfft_chain(dev, n, rng):
    """The reference checks its four-step run_large against the cuFFT chain on
    the same data (bench_fufft.cu:453-464).  Here: the four-step with both
    middles, and at N = 32768 the single-launch conv, each within 2e-6 of an
    fp64 FFT convolution and within 4e-6 of the rocFFT chain (BASELINE
    Re/Im U[-1,1), one shared filter)."""
    import torch
    import fufft_amd as ff
    batch = (1 << 20) // n
    a = (rng.uniform(-1, 1, (batch, n)) + 1j * rng.uniform(-1, 1, (batch, n))).astype(np.complex64)
    taps = (rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)).astype(np.complex64)
    x = torch.from_numpy(a).to(dev)
    spec = torch.fft.fft(torch.from_numpy(taps).to(dev))
    print(f"case vendor chain four-step n={n} batch={batch}", flush=True)
    chain_h = torch.fft.ifft(torch.fft.fft(x, dim=1) * spec, dim=1).cpu().numpy()
    truth = np.fft.ifft(np.fft.fft(a.astype(np.complex128), axis=1)
                        * np.fft.fft(taps.astype(np.complex128))[None, :], axis=1)
    assert rel_l2(chain_h, truth) <= TOL_F32
    outs = {}
    for variant in ("v16", "r8"):
        filt = torch.from_numpy(ff.plan_filter_large(taps, n, kind=ff.FILTER_TAPS, variant=variant)).to(dev)
        buf = x.clone()
        ff.conv_large(buf, filt, n=n, batch=batch, variant=variant)
        outs[f"four-step {variant} middle"] = buf
    if ff.supported(n, "v16"):
        filt = torch.from_numpy(ff.plan_filter(taps, n, variant="v16", layout="lane", kind=ff.FILTER_TAPS)).to(dev)
        out = torch.empty_like(x)
        ff.conv(x, filt, out, n=n, batch=batch, variant="v16", layout="lane")
        outs["single launch"] = out
    torch.cuda.synchronize()
    for name, o in outs.items():
        got = o.cpu().numpy()
        e_truth, e_chain = rel_l2(got, truth), rel_l2(got, chain_h)
        print(f"  {name}: vs fp64 {e_truth:.2e}, vs rocFFT chain {e_chain:.2e}", flush=True)
        assert e_truth <= TOL_F32
        assert e_chain <= 2 * TOL_F32
