"""GPU parity of the 2D paths (fufft_conv2d_f32, _r2, fwd2d / apply2d).

Bar: bit-identical to the oracle's 2D chain (rows DIF, columns DIF, mid,
columns DIT, rows DIT, verify_kernel.cpp:700-722) with the same per-dimension
plans in table-twiddle mode, and rel L2 <= 2e-6 against an fp64 FFT
convolution.  The split path equals the fused one bit for bit.  Filters run
in both column orders: the reference's ("dr", verify_kernel.cpp:738-748) and
the library's lane-major one ("lane"); the results are bit-identical.
"""
import numpy as np
import pytest

from conftest import bits_equal, cols_to_dr, crandn, cuniform, filt2d_dr
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL_F32 = 2e-6
SHAPES = [(256, 256), (512, 512), (256, 1024), (1024, 512), (2048, 256), (512, 2048)]


def to_dev(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def plans(h, w):
    import fufft_amd as ff
    vr, vc = ff.plan2d(h, w)
    return O.kernel_plan(h, vc), O.kernel_plan(w, vr)


def fp64_conv2d(a, taps, h, w, mid="mul"):
    a = a.reshape(-1, h, w).astype(np.complex128)
    s = np.fft.fft2(taps.reshape(h, w).astype(np.complex128))
    if mid == "conj":
        s = np.conj(s)
    if mid == "none":
        return (a * h * w).reshape(-1)
    return np.fft.ifft2(np.fft.fft2(a, axes=(1, 2)) * s[None], axes=(1, 2)).reshape(-1)


def run_conv2d(dev, a, filt, h, w, filt_stride=0, mid="mul", layout="lane"):
    import torch
    import fufft_amd as ff
    da, out = to_dev(a, dev), torch.empty(a.size, dtype=torch.complex64, device=dev)
    ff.conv2d(da, to_dev(filt, dev), out, h, w, batch=a.size // (h * w), filt_stride=filt_stride, mid=mid,
              layout=layout)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("layout", ["lane", "dr"])
@pytest.mark.parametrize("h,w", SHAPES)
@pytest.mark.parametrize("mid", ["mul", "conj", "none"])
def test_conv2d_matches_oracle(dev, h, w, mid, layout, rng):
    import fufft_amd as ff
    batch = 2
    a = cuniform(rng, batch * h * w)
    taps = cuniform(rng, h * w)
    filt = ff.plan_filter2d(taps, h, w, kind=ff.FILTER_TAPS, layout=layout)
    ph, pw = plans(h, w)
    print(f"case conv2d {h}x{w} mid={mid} layout={layout} plans {ph.radices} x {pw.radices}", flush=True)
    got = run_conv2d(dev, a, filt, h, w, mid=mid, layout=layout)
    assert bits_equal(got, O.conv2d(a, filt2d_dr(filt, h, w, layout), h, w, ph, pw, mid=mid))
    assert O.rel_l2(got, fp64_conv2d(a, taps, h, w, mid)) <= TOL_F32


@pytest.mark.parametrize("h,w", [(512, 512), (256, 1024), (2048, 256)])
def test_conv2d_reference_order_filter(dev, h, w, rng):
    """A filter built the way the reference's host code builds it, slot (r, c)
    = natural bin (rev_h(r), rev_w(c)) from each dimension's digit order
    (verify_kernel.cpp:738-748), fed with layout "dr": bit-identical to the
    oracle and to the same filter in the library's own column order."""
    import fufft_amd as ff
    batch = 2
    a = crandn(rng, batch * h * w)
    S = crandn(rng, (h, w), 1.0 / (h * w))            # natural-order spectrum, 1/(h w) folded
    ph, pw = plans(h, w)
    b_dr = np.ascontiguousarray(S[np.ix_(O.mixedrev(ph), O.mixedrev(pw))]).reshape(-1)
    print(f"case conv2d reference-order filter {h}x{w}", flush=True)
    got = run_conv2d(dev, a, b_dr, h, w, layout="dr")
    assert bits_equal(got, O.conv2d(a, b_dr, h, w, ph, pw))
    b_lane = ff.plan_filter2d(S, h, w, fold_inv_n=False, layout="lane")
    assert bits_equal(cols_to_dr(b_lane, h, w), b_dr)
    assert bits_equal(run_conv2d(dev, a, b_lane, h, w, layout="lane"), got)
    want = np.fft.ifft2(np.fft.fft2(a.reshape(batch, h, w).astype(np.complex128), axes=(1, 2))
                        * S.astype(np.complex128)[None] * (h * w), axes=(1, 2)).reshape(-1)
    assert O.rel_l2(got, want) <= TOL_F32


@pytest.mark.parametrize("layout", ["lane", "dr"])
def test_conv2d_per_image_filter_in_place(dev, layout, rng):
    import torch
    import fufft_amd as ff
    h, w, batch = 512, 512, 3
    a = crandn(rng, batch * h * w)
    filt = np.concatenate([ff.plan_filter2d(cuniform(rng, h * w), h, w, layout=layout) for _ in range(batch)])
    ph, pw = plans(h, w)
    buf = to_dev(a, dev)
    print(f"case conv2d per-image filters, in place, layout={layout}", flush=True)
    ff.conv2d(buf, to_dev(filt, dev), buf, h, w, batch=batch, filt_stride=h * w, layout=layout)
    torch.cuda.synchronize()
    assert bits_equal(buf.cpu().numpy(), O.conv2d(a, filt2d_dr(filt, h, w, layout), h, w, ph, pw,
                                                  filt_stride=h * w))


@pytest.mark.parametrize("layout", ["lane", "dr"])
@pytest.mark.parametrize("h,w", [(512, 512), (256, 1024)])
def test_conv2d_two_real_images(dev, h, w, layout, rng):
    """Two real images per complex transform with a real filter (BASELINE
    config 5: pixels and taps U[0,1))."""
    import torch
    import fufft_amd as ff
    batch = 2
    x = rng.uniform(0, 1, batch * h * w).astype(np.float32)
    y = rng.uniform(0, 1, batch * h * w).astype(np.float32)
    taps = rng.uniform(0, 1, h * w).astype(np.float32)
    filt = ff.plan_filter2d(taps.astype(np.complex64), h, w, kind=ff.FILTER_TAPS, layout=layout)
    dx, dy, df = to_dev(x, dev), to_dev(y, dev), to_dev(filt, dev)
    u, v = torch.empty_like(dx), torch.empty_like(dy)
    work = torch.empty(batch * h * w, dtype=torch.complex64, device=dev)
    print(f"case conv2d r2 {h}x{w} layout={layout}", flush=True)
    ff.conv2d_r2(dx, dy, df, u, v, work, h, w, batch, layout=layout)
    torch.cuda.synchronize()
    z = (x + 1j * y).astype(np.complex64)
    ph, pw = plans(h, w)
    want = O.conv2d(z, filt2d_dr(filt, h, w, layout), h, w, ph, pw)
    assert bits_equal(u.cpu().numpy(), np.ascontiguousarray(want.real))
    assert bits_equal(v.cpu().numpy(), np.ascontiguousarray(want.imag))
    s = np.fft.fft2(taps.reshape(h, w).astype(np.float64))
    ux = np.real(np.fft.ifft2(np.fft.fft2(x.reshape(batch, h, w).astype(np.float64), axes=(1, 2)) * s, axes=(1, 2)))
    assert O.rel_l2(u.cpu().numpy(), ux.reshape(-1)) <= TOL_F32


@pytest.mark.parametrize("layout", ["lane", "dr"])
@pytest.mark.parametrize("h,w", [(512, 512), (1024, 256)])
def test_split_2d_equals_fused(dev, h, w, layout, rng):
    """One signal transformed once, applied against several filters with a
    broadcast spectrum; every output equals the fused conv bit for bit."""
    import torch
    import fufft_amd as ff
    nf = 6
    a = cuniform(rng, h * w)
    filters = np.concatenate([ff.plan_filter2d(crandn(rng, h * w, 1.0 / (h * w)), h, w,
                                               fold_inv_n=False, layout=layout) for _ in range(nf)])
    ph, pw = plans(h, w)
    da = to_dev(a, dev)
    spec = torch.empty_like(da)
    print(f"case split 2d {h}x{w} layout={layout}", flush=True)
    ff.fwd2d(da, spec, h, w, batch=1)
    df = to_dev(filters, dev)
    out = torch.empty(nf * h * w, dtype=torch.complex64, device=dev)
    ff.apply2d(spec, df, out, h, w, batch=nf, spec_stride=0, filt_stride=h * w, layout=layout)
    torch.cuda.synchronize()
    got_spec = spec.cpu().numpy()
    assert bits_equal(cols_to_dr(got_spec, h, w), O.fwd2d(a, h, w, ph, pw))
    got = out.cpu().numpy()
    assert bits_equal(got, O.apply2d(cols_to_dr(got_spec, h, w), filt2d_dr(filters, h, w, layout), h, w, nf,
                                     ph, pw, spec_stride=0, filt_stride=h * w))
    fused = run_conv2d(dev, np.tile(a, nf), filters, h, w, filt_stride=h * w, layout=layout)
    assert bits_equal(got, fused)


def test_split_2d_baseline_config(dev, rng):
    """BASELINE config 5b: one 512x512 signal, 256 filters with Gaussian spectra;
    sampled outputs bit-identical to the oracle and within 2e-6 of fp64."""
    import torch
    import fufft_amd as ff
    h = w = 512
    nf = 256
    a = cuniform(rng, h * w)
    spec_nat = crandn(rng, (nf, h * w))
    filters = np.concatenate([ff.plan_filter2d(spec_nat[i], h, w, layout="lane") for i in range(nf)])
    ph, pw = plans(h, w)
    da = to_dev(a, dev)
    spec = torch.empty_like(da)
    out = torch.empty(nf * h * w, dtype=torch.complex64, device=dev)
    print("case split 2d 512x512 x 256 filters", flush=True)
    ff.fwd2d(da, spec, h, w, batch=1)
    ff.apply2d(spec, to_dev(filters, dev), out, h, w, batch=nf, filt_stride=h * w, layout="lane")
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(nf, h * w)
    sp = spec.cpu().numpy()
    fa = np.fft.fft2(a.reshape(h, w).astype(np.complex128))
    for i in (0, 77, 255):
        f_i = filters[i * h * w:(i + 1) * h * w]
        assert bits_equal(got[i], O.apply2d(cols_to_dr(sp, h, w), cols_to_dr(f_i, h, w), h, w, 1, ph, pw))
        want = np.fft.ifft2(fa * spec_nat[i].reshape(h, w).astype(np.complex128)).reshape(-1)
        assert O.rel_l2(got[i], want) <= TOL_F32


def test_2d_rejects_and_empty(dev):
    import torch
    import fufft_amd as ff
    buf = torch.zeros(2 * 512 * 512, dtype=torch.complex64, device=dev)
    with pytest.raises(ff.FufftError):
        ff.conv2d(buf, buf, buf, 128, 512, batch=1)        # column length below the kernels' range
    with pytest.raises(ff.FufftError):
        ff.conv2d(buf, buf, buf, 512, 100, batch=1)        # row length not a power of two
    with pytest.raises(ff.FufftError):
        ff.apply2d(buf, buf, buf, 512, 512, batch=2)       # shared spectrum overwritten by out
    ff.conv2d(buf, buf, buf, 512, 512, batch=0)
