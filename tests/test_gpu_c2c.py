"""GPU parity of the natural-order C2C (fufft_c2c_f32) and of filter planning
on the device (fufft_plan_filter_device_f32 / _large_ / 2d_).

Bar: C2C bit-identical to the oracle (table twiddles), rel L2 <= 2e-6 against
numpy's fp64 FFT; device planning of spectra bit-identical to the host
planner; device planning of taps bit-identical to the oracle's fp32 forward
transform times 1/n, within 1e-6 of the host's fp64 planning, and a conv with
the device-planned filter within 2e-6 of fp64.
"""
import numpy as np
import pytest

from conftest import bits_equal, cols_to_dr, crandn, cuniform, filt2d_dr, lane_major, bperm
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL_F32 = 2e-6
V = {"v16": 16, "r8": 8}
SIZES = [("v16", n) for n in (256, 512, 1024, 2048, 4096, 8192, 16384)] + \
        [("r8", n) for n in (512, 1024, 2048, 4096, 8192)]


def scaled(x, s):
    """x * s on the real and imaginary parts separately (no complex product)"""
    x = np.ascontiguousarray(x, dtype=np.complex64)
    return (x.view(np.float32) * np.float32(s)).view(np.complex64)


def to_dev(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def from_dev(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("variant,n", SIZES)
@pytest.mark.parametrize("direction", [-1, 1])
def test_c2c_matches_oracle_bitwise(dev, variant, n, direction, rng):
    import torch
    import fufft_amd as ff
    batch = max(3, 32768 // n)
    a = crandn(rng, (batch, n))
    print(f"case c2c variant={variant} n={n} dir={direction} batch={batch}", flush=True)
    da = to_dev(a, dev)
    dout = torch.empty_like(da)
    ff.c2c(da, dout, n=n, batch=batch, direction=direction, variant=variant)
    got = from_dev(dout).reshape(-1)
    plan = O.kernel_plan(n, V[variant])
    assert bits_equal(got, O.c2c(a, n, plan, direction))
    a64 = a[:4].astype(np.complex128)
    truth = np.fft.fft(a64, axis=1) if direction < 0 else np.fft.ifft(a64, axis=1) * n
    assert O.rel_l2(got[:4 * n], truth.reshape(-1)) <= TOL_F32


@pytest.mark.parametrize("variant,n", [("r8", 4096), ("v16", 1024), ("v16", 256)])
def test_c2c_in_place_and_round_trip(dev, variant, n, rng):
    import fufft_amd as ff
    batch = 37                              # ragged: not a multiple of the transforms per workgroup
    a = cuniform(rng, (batch, n))
    print(f"case c2c in-place variant={variant} n={n}", flush=True)
    d = to_dev(a, dev)
    ff.c2c(d, d, n=n, batch=batch, direction=ff.FORWARD, variant=variant)
    spec = from_dev(d).reshape(-1)
    plan = O.kernel_plan(n, V[variant])
    assert bits_equal(spec, O.c2c(a, n, plan, -1))
    ff.c2c(d, d, n=n, batch=batch, direction=ff.INVERSE, variant=variant)
    back = from_dev(d).reshape(-1)
    assert bits_equal(back, O.c2c(spec, n, plan, +1))
    assert O.rel_l2(back / n, a.reshape(-1)) <= TOL_F32


def test_c2c_full_size_properties(dev):
    """2^27 points: the forward C2C equals the split fwd kernel's digit-order
    spectrum permuted (every transform), and the inverse brings back n x."""
    import torch
    import fufft_amd as ff
    n, batch = 4096, (1 << 27) // 4096
    torch.manual_seed(11)
    da = torch.randn(batch * n, dtype=torch.complex64, device=dev)
    dnat = torch.empty_like(da)
    print("case c2c full-size n=4096 batch=32768", flush=True)
    ff.c2c(da, dnat, n=n, batch=batch, direction=ff.FORWARD, variant="auto")
    dspec = torch.empty_like(da)
    ff.fwd(da, dspec, n=n, batch=batch, variant="auto")
    perm = torch.from_numpy(ff.digit_order(n, "auto").astype(np.int64)).to(dev)
    same = torch.equal(dnat.view(batch, n)[:, perm].view(torch.int64), dspec.view(batch, n).view(torch.int64))
    assert same
    ff.c2c(dnat, dnat, n=n, batch=batch, direction=ff.INVERSE, variant="auto")
    err = torch.linalg.vector_norm(dnat / n - da) / torch.linalg.vector_norm(da)
    assert float(err) < 1e-6


def test_c2c_rejects_bad_args(dev):
    import torch
    import fufft_amd as ff
    d = torch.zeros(4096, dtype=torch.complex64, device=dev)
    with pytest.raises(ff.FufftError):
        ff.c2c(d, d, n=4096, batch=1, direction=0)
    with pytest.raises(ff.FufftError):
        ff.c2c(d, d, n=100, batch=1)
    ff.c2c(d, d, n=4096, batch=0)          # empty batch is a no-op


# ---- filter planning on the device ---------------------------------------------------------

@pytest.mark.parametrize("variant,n", [("v16", 256), ("v16", 4096), ("r8", 512), ("r8", 4096),
                                       ("r8", 8192), ("v16", 16384)])
@pytest.mark.parametrize("layout", ["dr", "lane", "bperm"])
def test_plan_device_1d(dev, variant, n, layout, rng):
    import torch
    import fufft_amd as ff
    count = 5
    taps = crandn(rng, (count, n))
    spec = np.fft.fft(taps.astype(np.complex128), axis=1).astype(np.complex64)
    print(f"case plan1d variant={variant} n={n} layout={layout}", flush=True)
    dt, ds = to_dev(taps, dev), to_dev(spec, dev)
    out_t, out_s = torch.empty_like(dt), torch.empty_like(ds)
    ff.plan_filter_device(dt, out_t, n, count, variant, layout, kind=ff.FILTER_TAPS)
    ff.plan_filter_device(ds, out_s, n, count, variant, layout, kind=ff.FILTER_SPECTRUM)
    got_t, got_s = from_dev(out_t), from_dev(out_s)
    host_s = np.stack([ff.plan_filter(spec[i], n, variant, layout, kind=ff.FILTER_SPECTRUM)
                       for i in range(count)])
    host_t = np.stack([ff.plan_filter(taps[i], n, variant, layout, kind=ff.FILTER_TAPS)
                       for i in range(count)])
    assert bits_equal(got_s, host_s)
    v = V[variant]
    want_t = scaled(O.fwd(taps, n, O.kernel_plan(n, v)), 1.0 / n).reshape(count, n)
    if layout == "lane":
        want_t = lane_major(want_t, n, v)
    elif layout == "bperm":
        want_t = bperm(want_t, n, v)
    assert bits_equal(got_t, want_t)
    assert O.rel_l2(got_t, host_t) <= 1e-6


def test_plan_device_taps_in_place_then_conv(dev, rng):
    import torch
    import fufft_amd as ff
    n, batch = 4096, 64
    taps = crandn(rng, n)
    a = crandn(rng, (batch, n))
    print("case plan1d in place + conv", flush=True)
    df = to_dev(taps, dev)
    ff.plan_filter_device(df, df, n, 1, "auto", "dr", kind=ff.FILTER_TAPS)
    da = to_dev(a, dev)
    dout = torch.empty_like(da)
    ff.conv(da, df, dout, n=n, batch=batch, variant="auto")
    got = from_dev(dout).reshape(-1)
    spec = np.fft.fft(taps.astype(np.complex128)) / n
    assert O.rel_l2(got[:8 * n], O.conv_spec_f64(a[:8], spec.astype(np.complex64), n)) <= TOL_F32


@pytest.mark.parametrize("n", [8192, 32768, 131072])
@pytest.mark.parametrize("variant", ["v16", "r8"])
def test_plan_device_large(dev, n, variant, rng):
    import torch
    import fufft_amd as ff
    count = 2
    taps = cuniform(rng, (count, n))
    spec = np.fft.fft(taps.astype(np.complex128), axis=1).astype(np.complex64)
    print(f"case plan large n={n} variant={variant}", flush=True)
    dt, ds = to_dev(taps, dev), to_dev(spec, dev)
    out_t, out_s = torch.empty_like(dt), torch.empty_like(ds)
    ff.plan_filter_large_device(dt, out_t, n, count, kind=ff.FILTER_TAPS, variant=variant)
    ff.plan_filter_large_device(ds, out_s, n, count, kind=ff.FILTER_SPECTRUM, variant=variant)
    got_t, got_s = from_dev(out_t), from_dev(out_s)
    host_s = np.stack([ff.plan_filter_large(spec[i], n, kind=ff.FILTER_SPECTRUM, variant=variant)
                       for i in range(count)])
    assert bits_equal(got_s, host_s)
    lout, mid = ff.large_plan(n)
    want_t = O.fwd(taps, n, O.large_plan(lout, mid, mid_v=ff.large_middle(variant)))
    assert bits_equal(got_t.reshape(-1), scaled(want_t, 1.0 / n))
    host_t = np.stack([ff.plan_filter_large(taps[i], n, kind=ff.FILTER_TAPS, variant=variant)
                       for i in range(count)])
    assert O.rel_l2(got_t, host_t) <= 1e-6


@pytest.mark.parametrize("layout", ["lane", "dr"])
@pytest.mark.parametrize("h,w", [(256, 256), (512, 512), (1024, 512)])
def test_plan_device_2d(dev, h, w, layout, rng):
    import torch
    import fufft_amd as ff
    count = 2
    taps = cuniform(rng, (count, h, w))
    spec = np.fft.fft2(taps.astype(np.complex128)).astype(np.complex64)
    print(f"case plan2d {h}x{w} layout={layout}", flush=True)
    dt, ds = to_dev(taps, dev), to_dev(spec, dev)
    out_t, out_s = torch.empty_like(dt), torch.empty_like(ds)
    ff.plan_filter2d_device(dt, out_t, h, w, count, kind=ff.FILTER_TAPS, layout=layout)
    ff.plan_filter2d_device(ds, out_s, h, w, count, kind=ff.FILTER_SPECTRUM, layout=layout)
    got_t, got_s = from_dev(out_t), from_dev(out_s)
    host_s = np.stack([ff.plan_filter2d(spec[i], h, w, kind=ff.FILTER_SPECTRUM, layout=layout)
                       for i in range(count)])
    assert bits_equal(got_s.reshape(count, -1), host_s)
    vr, vc = ff.plan2d(h, w)
    want_t = scaled(O.fwd2d(taps, h, w, O.kernel_plan(h, vc), O.kernel_plan(w, vr)), 1.0 / (h * w))
    assert bits_equal(filt2d_dr(got_t.reshape(-1), h, w, layout), want_t)
    host_t = np.stack([ff.plan_filter2d(taps[i], h, w, kind=ff.FILTER_TAPS, layout=layout)
                       for i in range(count)])
    assert O.rel_l2(got_t.reshape(count, -1), host_t) <= 1e-6


def test_plan_device_rejects_aliased_spectrum(dev):
    import torch
    import fufft_amd as ff
    d = torch.zeros(4096, dtype=torch.complex64, device=dev)
    with pytest.raises(ff.FufftError):
        ff.plan_filter_device(d, d, 4096, 1, kind=ff.FILTER_SPECTRUM)
