"""GPU kernels against the reference's own CPU transcription, bit for bit.

With the device table switched to the reference's base twiddles
(fufft_set_twiddles(FUFFT_TWIDDLES_REFERENCE): cosf / sinf of the fp32 angle
(2*pi/P)*j, as verify_kernel.cpp:31, 93-99 computes them), the fp32 kernels
perform exactly the operations of the reference's transcription
(verify_kernel.cpp: kernel_pipeline_v16, kernel_pipeline_ip, _fwd / _apply,
kernel_conv_r2, conv_foursteps_cfg, kernel_conv2d), so:

1. on the golden fixtures written from the compiled reference
   (tests/golden/make_golden.py) the GPU output equals the reference's output
   bit for bit, for every fixture whose plan a GPU kernel runs;
2. at every supported size, mid operation and path the GPU equals the oracle
   in libm-twiddle mode bit for bit -- the mode tests/test_oracle_pins.py pins
   bit for bit to the compiled reference -- and stays within 2e-6 of fp64.

The module switches the table back to the default source when it ends.
"""
import numpy as np
import pytest

from conftest import bits_equal, bperm, cols_to_dr, crandn, cuniform, lane_major
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL_F32 = 2e-6


def to_dev(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy().reshape(-1)


@pytest.fixture(scope="module")
def ref_tw(dev):
    import fufft_amd as ff
    ff.set_twiddles("reference")
    assert ff.get_twiddles() == "reference"
    try:
        yield dev
    finally:
        ff.set_twiddles("accurate")
        assert ff.get_twiddles() == "accurate"


def _golden():
    from tests.golden import golden
    return golden.load_all()


# fixtures whose plan a GPU kernel runs (the GPU's smallest sizes are N = 256
# radix 16 and N = 512 radix 8; its four-step middle is radix 16 or radix 8 in
# [512, 4096]; fourstep_n32768_mid2048_v16 is the reference bench's own
# run_large<32768, 1, 16, 2048, 8, 2>)
GPU_FIXTURES = ["v16_n512", "v16_n1024", "v16_n2048", "v16_n4096", "r8_n512", "r8_n1024",
                "r8_n2048", "r8_n4096", "split_n512", "r2_n512", "fourstep_n8192_mid512_r8",
                "fourstep_n32768_mid2048_v16", "conv2d_64x64"]


@pytest.mark.parametrize("name", GPU_FIXTURES)
def test_gpu_equals_reference_on_golden_fixture(ref_tw, name):
    import torch
    import fufft_amd as ff
    dev = ref_tw
    case = _golden()[name]
    kind = str(case["kind"])
    print(f"case golden {name} kind={kind}", flush=True)
    if kind in ("v16", "r8"):
        n = int(case["n"])
        a = case["a"]
        da = to_dev(a, dev)
        out = torch.empty_like(da)
        ff.conv(da, to_dev(case["bdr"], dev), out, n=n, batch=a.size // n, filt_stride=n, variant=kind)
        assert bits_equal(host(out), case["out"])
        # the same filters in the reference's bperm layout and in the library's
        # lane-major pairs give the compiled reference's outputs too
        v = 16 if kind == "v16" else 8
        for layout, moved in (("bperm", bperm(case["bdr"], n, v)), ("lane", lane_major(case["bdr"], n, v))):
            out2 = torch.empty_like(da)
            ff.conv(da, to_dev(moved, dev), out2, n=n, batch=a.size // n, filt_stride=n, variant=kind,
                    layout=layout)
            assert bits_equal(host(out2), case["out"]), layout
    elif kind == "split":
        n = int(case["n"])
        a = case["a"]
        batch = a.size // n
        da = to_dev(a, dev)
        spec, out = torch.empty_like(da), torch.empty_like(da)
        ff.fwd(da, spec, n=n, batch=batch, variant="r8")
        ff.apply(spec, to_dev(case["bdr"], dev), out, n=n, batch=batch, spec_stride=n, filt_stride=n,
                 variant="r8")
        assert bits_equal(host(spec), case["spec"])
        assert bits_equal(host(out), case["out"])
    elif kind == "r2":
        n = int(case["n"])
        x, y = case["x"], case["y"]
        dx, dy = to_dev(x, dev), to_dev(y, dev)
        du, dv = torch.empty_like(dx), torch.empty_like(dy)
        ff.conv_r2(dx, dy, to_dev(case["bdr"], dev), du, dv, n=n, batch=x.size // n, filt_stride=n,
                   variant="r8")
        assert bits_equal(host(du), case["u"])
        assert bits_equal(host(dv), case["v"])
    elif kind == "conv2d":
        # the reference's fused small-image 2D conv (fufft_conv2d<64, 64, CPB>)
        h, w = int(case["h"]), int(case["w"])
        a = case["a"]
        da = to_dev(a, dev)
        out = torch.empty_like(da)
        ff.conv2d(da, to_dev(case["bdr"], dev), out, h, w, batch=a.size // (h * w), filt_stride=h * w,
                  layout="dr")
        assert bits_equal(host(out), case["out"])
    elif kind == "fourstep":
        n = int(case["n"])
        lout, mid = ff.large_plan(n)
        assert (lout, mid) == (int(case["lout"]), int(case["mid"]))
        # the middle the fixture was made with: the reference's V=16 run_large
        # middle by default, radix 8 where the fixture says so
        variant = "r8" if "mid_v" in case and int(case["mid_v"]) == 8 else "v16"
        buf = to_dev(case["a"], dev)
        ff.conv_large(buf, to_dev(case["bdr"], dev), n=n, batch=case["a"].size // n, filt_stride=n,
                      variant=variant)
        assert bits_equal(host(buf), case["out"])
    else:
        raise AssertionError(kind)


SIZES = [("v16", n) for n in (256, 512, 1024, 2048, 4096, 8192, 16384, 32768)] + \
        [("r8", n) for n in (512, 1024, 2048, 4096, 8192)]
V = {"v16": 16, "r8": 8}


@pytest.mark.parametrize("variant,n", SIZES)
@pytest.mark.parametrize("mid", ["mul", "conj", "none"])
def test_conv_equals_libm_oracle(ref_tw, variant, n, mid, rng):
    import torch
    import fufft_amd as ff
    dev = ref_tw
    batch = max(2, 16384 // n)
    a = crandn(rng, (batch, n))
    spec = crandn(rng, n) / n
    plan = O.kernel_plan(n, V[variant])
    fdr = spec[O.mixedrev(plan)]
    print(f"case reftw conv variant={variant} n={n} mid={mid} batch={batch}", flush=True)
    da = to_dev(a, dev)
    out = torch.empty_like(da)
    ff.conv(da, to_dev(fdr, dev), out, n=n, batch=batch, mid=mid, variant=variant)
    got = host(out)
    assert bits_equal(got, O.conv(a, fdr, n, plan, mid=mid, tw=O.TW_LIBM))
    assert O.rel_l2(got, O.conv_spec_f64(a, spec, n, mid=mid)) <= TOL_F32


@pytest.mark.parametrize("n", [32768, 65536])
@pytest.mark.parametrize("variant", ["v16", "r8"])
def test_fourstep_equals_libm_oracle(ref_tw, n, variant, rng):
    import fufft_amd as ff
    dev = ref_tw
    lout, mid = ff.large_plan(n)
    plan = O.large_plan(lout, mid, ff.large_middle(variant))
    a = cuniform(rng, (2, n))
    spec = cuniform(rng, n) / n
    fdr = spec[O.mixedrev(plan)]
    print(f"case reftw fourstep n={n} variant={variant}", flush=True)
    buf = to_dev(a, dev)
    ff.conv_large(buf, to_dev(fdr, dev), n=n, batch=2, variant=variant)
    got = host(buf)
    assert bits_equal(got, O.conv(a, fdr, n, plan, tw=O.TW_LIBM))
    assert O.rel_l2(got, O.conv_spec_f64(a, spec, n)) <= TOL_F32


def rev8(x, digits):
    """base-8 digit reversal (the reference's rev8, verify_kernel.cpp:738-743)"""
    r = 0
    for _ in range(digits):
        r = r * 8 + (x & 7)
        x >>= 3
    return r


@pytest.mark.parametrize("layout", ["dr", "lane"])
@pytest.mark.parametrize("h,w", [(512, 512), (512, 4096)])
def test_conv2d_equals_libm_oracle(ref_tw, h, w, layout, rng):
    """The reference's 2D test setup (test_2d, verify_kernel.cpp:724-748):
    signal and filter U[-1, 1), the filter times 1/(h w), and the filter
    handed over in its order, slot (r, c) = natural bin (rev8(r), rev8(c)).
    Fed as is (layout "dr") or moved to the library's column order ("lane"),
    the GPU equals the LIBM-mode oracle (pinned bit for bit to the compiled
    kernel_conv2d) bit for bit."""
    import torch
    import fufft_amd as ff
    dev = ref_tw
    vr, vc = ff.plan2d(h, w)
    ph, pw = O.kernel_plan(h, vc), O.kernel_plan(w, vr)
    # at these shapes (powers of 8) the GPU's row and column plans are the
    # reference's radix-8 plans (kernel_conv2d runs radix 8 in both dimensions)
    assert (ph.radices, pw.radices) == (O.ref_plan(h, 8).radices, O.ref_plan(w, 8).radices)
    sh, sw = len(ph.radices), len(pw.radices)
    a = cuniform(rng, (2, h, w))
    b = cuniform(rng, (h, w)) * np.float32(1.0 / (h * w))
    b_dr = np.ascontiguousarray(b[np.ix_([rev8(r, sh) for r in range(h)],
                                         [rev8(c, sw) for c in range(w)])]).reshape(-1)
    if layout == "dr":
        filt = b_dr
    else:
        slot = ff.column_order2d(h, w)
        filt = np.ascontiguousarray(b_dr.reshape(h, w)[:, slot]).reshape(-1)
        assert bits_equal(cols_to_dr(filt, h, w), b_dr)
    print(f"case reftw conv2d {h}x{w} layout={layout}", flush=True)
    da = to_dev(a, dev)
    out = torch.empty_like(da)
    ff.conv2d(da, to_dev(filt, dev), out, h, w, batch=2, layout=layout)
    assert bits_equal(host(out), O.conv2d(a, b_dr, h, w, ph, pw, tw=O.TW_LIBM))


@pytest.mark.parametrize("layout", ["dr", "lane"])
@pytest.mark.parametrize("n", [512, 4096])
def test_bfp_equals_libm_oracle(ref_tw, n, layout, rng):
    """The BFP conv at FUFFT_AUTO with the digit-order filter, and at the bench's
    plan (lane-major filter, fufft_fastest_variant), equals the LIBM-mode oracle."""
    import torch
    import fufft_amd as ff
    dev = ref_tw
    batch = 16
    variant = "auto" if layout == "dr" else ff.fastest_variant(n, "lane")
    v = 8 if ff.resolve_variant(n, variant) == "r8" else 16
    x = (crandn(rng, (batch, n)) * 10.0 ** rng.uniform(-3, 3, (batch, 1))).astype(np.complex64)
    q, e = ff.bfp_quantize(x)
    taps = crandn(rng, n)
    filt = ff.plan_filter(taps, n, variant=variant, kind=ff.FILTER_TAPS)
    fdev = ff.plan_filter(taps, n, variant=variant, layout=layout, kind=ff.FILTER_TAPS)
    print(f"case reftw bfp n={n} layout={layout} v={v}", flush=True)
    dq, de = to_dev(q, dev), to_dev(e, dev)
    qo, eo = torch.empty_like(dq), torch.empty_like(de)
    ff.conv_bfp16(dq, de, to_dev(fdev, dev), qo, eo, n=n, batch=batch, variant=variant, layout=layout)
    oq, oe = O.bfp_conv(q, e, filt, n, O.kernel_plan(n, v), tw=O.TW_LIBM)
    assert np.array_equal(host(eo), oe)
    assert np.array_equal(host(qo), oq)


def test_set_twiddles_rejects_bad_source(dev):
    import fufft_amd as ff
    before = ff.get_twiddles()
    with pytest.raises(ff.FufftError):
        ff.check(ff.lib.fufft_set_twiddles(0, 5), "fufft_set_twiddles")
    assert ff.get_twiddles() == before


@pytest.mark.parametrize("name", ["bfp_scaled_n512", "bfp_scaled_n4096"])
def test_bfp_scaled_equals_reference_on_golden_fixture(ref_tw, name):
    """The reference's own BFP format at its plan (radix 16): words and scales
    equal the compiled reference's kernel_v16_bfp (verify_kernel.cpp:1107-1135)
    on the golden fixtures."""
    import torch
    import fufft_amd as ff
    dev = ref_tw
    case = _golden()[name]
    n = int(case["n"])
    batch = case["asc"].size
    print(f"case golden {name}", flush=True)
    dq, ds = to_dev(case["aq"], dev), to_dev(case["asc"], dev)
    qo, so = torch.empty_like(dq), torch.empty_like(ds)
    ff.conv_bfp16_scaled(dq, ds, to_dev(case["bq"], dev), to_dev(case["bsc"], dev), qo, so, n=n, batch=batch,
                         variant="v16")
    assert np.array_equal(host(qo), case["oq"])
    assert np.array_equal(host(so).view(np.uint32), case["osc"].view(np.uint32))
