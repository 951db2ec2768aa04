"""GPU parity of the fused small-image 2D conv (fufft_conv2d_f32 at H x W <=
8192 points, 8 <= H, W <= 512: the reference's fufft_conv2d<H, W, CPB>,
fufft.cuh:1209-1258, whose own shapes are powers of 8 up to 4096 points).

Bar: bit-identical to the oracle's 2D chain (rows DIF, columns DIF, mid,
columns DIT, rows DIT with radix-8 plans both ways; verify_kernel.cpp:700-722)
at every supported shape and mid operation, ragged batches, per-image filters
and in place; rel L2 <= 2e-6 against the fp64 2D convolution.  The golden
fixture written by the compiled reference (conv2d_64x64) is checked in
tests/test_gpu_reference_twiddles.py.
"""
import numpy as np
import pytest

from conftest import bits_equal, crandn, cuniform
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL_F32 = 2e-6
SHAPES = [(h, w) for h in (8, 16, 32, 64, 128, 256, 512) for w in (8, 16, 32, 64, 128, 256, 512)
          if h * w <= 8192]


def to_dev(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def fp64_conv2d(a, taps, h, w, mid="mul"):
    a = a.reshape(-1, h, w).astype(np.complex128)
    s = np.fft.fft2(taps.reshape(h, w).astype(np.complex128))
    if mid == "conj":
        s = np.conj(s)
    if mid == "none":
        return (a * h * w).reshape(-1)
    return np.fft.ifft2(np.fft.fft2(a, axes=(1, 2)) * s[None], axes=(1, 2)).reshape(-1)


@pytest.mark.parametrize("h,w", SHAPES)
@pytest.mark.parametrize("mid", ["mul", "conj", "none"])
def test_small2d_matches_oracle(dev, h, w, mid, rng):
    import torch
    import fufft_amd as ff
    assert ff.plan2d(h, w) == (8, 8)
    batch = 2 + 300 // (h * w // 8)                 # a ragged last workgroup at the small shapes
    a = cuniform(rng, batch * h * w)
    taps = cuniform(rng, h * w)
    filt = ff.plan_filter2d(taps, h, w, kind=ff.FILTER_TAPS, layout="dr")
    print(f"case small2d {h}x{w} mid={mid} batch={batch}", flush=True)
    da = to_dev(a, dev)
    out = torch.empty_like(da)
    ff.conv2d(da, None if mid == "none" else to_dev(filt, dev), out, h, w, batch=batch, mid=mid, layout="dr")
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ph, pw = O.kernel_plan(h, 8), O.kernel_plan(w, 8)
    assert bits_equal(got, O.conv2d(a, filt, h, w, ph, pw, mid=mid))
    assert O.rel_l2(got, fp64_conv2d(a, taps, h, w, mid)) <= TOL_F32


@pytest.mark.parametrize("h,w", [(8, 512), (64, 64), (512, 16), (16, 16)])
def test_small2d_per_image_filters_in_place(dev, h, w, rng):
    import torch
    import fufft_amd as ff
    batch = 5
    a = crandn(rng, batch * h * w)
    filt = np.concatenate([ff.plan_filter2d(cuniform(rng, h * w), h, w, layout="dr") for _ in range(batch)])
    print(f"case small2d per-image filters in place {h}x{w}", flush=True)
    buf = to_dev(a, dev)
    ff.conv2d(buf, to_dev(filt, dev), buf, h, w, batch=batch, filt_stride=h * w, layout="dr")
    torch.cuda.synchronize()
    ph, pw = O.kernel_plan(h, 8), O.kernel_plan(w, 8)
    assert bits_equal(buf.cpu().numpy(), O.conv2d(a, filt, h, w, ph, pw, filt_stride=h * w))


def test_small2d_lane_order_is_the_identity(dev, rng):
    """For small images the library's column order is the identity, so both
    filter layouts name the same filter."""
    import torch
    import fufft_amd as ff
    h, w = 32, 64
    assert np.array_equal(ff.column_order2d(h, w), np.arange(w))
    taps = cuniform(rng, h * w)
    f_dr = ff.plan_filter2d(taps, h, w, kind=ff.FILTER_TAPS, layout="dr")
    f_ln = ff.plan_filter2d(taps, h, w, kind=ff.FILTER_TAPS, layout="lane")
    assert bits_equal(f_dr, f_ln)
    a = cuniform(rng, 3 * h * w)
    da = to_dev(a, dev)
    o1, o2 = torch.empty_like(da), torch.empty_like(da)
    ff.conv2d(da, to_dev(f_dr, dev), o1, h, w, batch=3, layout="dr")
    ff.conv2d(da, to_dev(f_ln, dev), o2, h, w, batch=3, layout="lane")
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


def test_small2d_other_calls_unsupported(dev):
    """The reference has only the fused conv for small images; the split and
    two-for-one calls refuse them with FUFFT_ERR_UNSUPPORTED."""
    import torch
    import fufft_amd as ff
    h = w = 64
    buf = torch.zeros(2 * h * w, dtype=torch.complex64, device=dev)
    re = torch.zeros(2 * h * w, device=dev)
    for call in (lambda: ff.fwd2d(buf, buf, h, w, batch=1),
                 lambda: ff.apply2d(buf, buf, buf, h, w, batch=1, spec_stride=h * w),
                 lambda: ff.conv2d_r2(re, re, buf, re, re, buf, h, w, 1)):
        with pytest.raises(ff.FufftError) as ei:
            call()
        assert ei.value.status == ff.ERR_UNSUPPORTED
