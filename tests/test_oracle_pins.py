"""Pin the CPU oracle (oracle/oracle.c) before trusting it as the GPU checker.

1. Bit-identity with the reference's own CPU transcription of its kernels
   (verify_kernel.cpp, compiled where it lies into oracle/_ref) when the oracle
   takes its base twiddles from libm like the reference does (TW_LIBM).
2. The same against the committed golden fixtures (tests/golden), so the pin
   holds where the reference sources are absent.
3. Accuracy of the table-twiddle mode (what the GPU computes) against fp64.
4. Closed forms and invariants that a dropped term, wrong sign, wrong index or
   transposed operand would break: delta filter, delta signal, round trip,
   correlation by brute force, linearity, digit order by naive DFT.
5. The fp64 references themselves against numpy and a naive DFT.
"""
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from conftest import bits_equal, crandn, cuniform
from oracle import oracle as O

REF = O.load_ref()
needs_ref = pytest.mark.skipif(REF is None, reason="reference CPU sources not built here")


def lead_and_count(n, v):
    rads = O.factor(n, v)
    return (rads[0] if rads[0] != v else 1), rads.count(v)


# ---- 1. bit-identity with the reference transcription ---------------------------------

@needs_ref
@pytest.mark.parametrize("n", [16, 32, 64, 128, 256, 512, 1024, 2048, 4096])
@pytest.mark.parametrize("cpb", [1, 2])
def test_v16_libm_matches_reference_bitwise(n, cpb, rng):
    batch = 4
    a = cuniform(rng, (batch, n))
    b = cuniform(rng, (batch, n)) / n
    plan = O.ref_plan(n, 16)
    bdr = np.ascontiguousarray(b[:, O.mixedrev(plan)])
    lead, nrv = lead_and_count(n, 16)
    ref = np.empty_like(a)
    REF.ref_vk_pipeline_v16(n, lead, nrv, cpb, a.ctypes.data, bdr.ctypes.data, ref.ctypes.data, batch)
    ours = O.conv(a, bdr, n, plan, filt_stride=n, tw=O.TW_LIBM)
    assert bits_equal(ours, ref.reshape(-1))


@needs_ref
@pytest.mark.parametrize("n", [8, 64, 128, 256, 512, 1024, 2048, 4096])
def test_r8_libm_matches_reference_bitwise(n, rng):
    batch = 3
    a = cuniform(rng, (batch, n))
    b = cuniform(rng, (batch, n)) / n
    plan = O.ref_plan(n, 8)
    bdr = np.ascontiguousarray(b[:, O.mixedrev(plan)])
    lead, nr8 = lead_and_count(n, 8)
    ref = np.empty_like(a)
    REF.ref_vk_pipeline_ip(n, lead, nr8, 1, a.ctypes.data, bdr.ctypes.data, ref.ctypes.data, batch)
    ours = O.conv(a, bdr, n, plan, filt_stride=n, tw=O.TW_LIBM)
    assert bits_equal(ours, ref.reshape(-1))


@needs_ref
@pytest.mark.parametrize("n", [64, 512, 1024])
def test_split_libm_matches_reference_bitwise(n, rng):
    batch = 3
    a = cuniform(rng, (batch, n))
    b = cuniform(rng, (batch, n)) / n
    plan = O.ref_plan(n, 8)
    bdr = np.ascontiguousarray(b[:, O.mixedrev(plan)])
    lead, nr8 = lead_and_count(n, 8)
    spec = np.empty_like(a)
    out = np.empty_like(a)
    REF.ref_vk_pipeline_fwd(n, lead, nr8, 1, a.ctypes.data, spec.ctypes.data, batch)
    REF.ref_vk_pipeline_apply(n, lead, nr8, 1, spec.ctypes.data, bdr.ctypes.data, out.ctypes.data, batch)
    ospec = O.fwd(a, n, plan, tw=O.TW_LIBM)
    oout = O.apply(ospec, bdr, n, batch, plan, spec_stride=n, filt_stride=n, tw=O.TW_LIBM)
    assert bits_equal(ospec, spec.reshape(-1))
    assert bits_equal(oout, out.reshape(-1))


@needs_ref
@pytest.mark.parametrize("n,mid", [(32768, 2048), (65536, 4096), (131072, 8192), (524288, 2048)])
def test_fourstep_libm_matches_reference_bitwise(n, mid, rng):
    batch = 1
    a = cuniform(rng, (batch, n))
    b = cuniform(rng, (batch, n)) / n
    lout = 0
    m = n
    while m > mid:
        m //= 16
        lout += 1
    assert m == mid
    plan = O.large_plan(lout, mid, ref=True)
    bdr = np.ascontiguousarray(b[:, O.mixedrev(plan)])
    # the reference derives the chained order with its own chain_rev
    rads = (O.C.c_int * len(plan.radices))(*plan.radices)
    ref_perm = np.array([REF.ref_vk_chain_rev(i, rads, len(plan.radices)) for i in range(0, n, 97)])
    assert np.array_equal(ref_perm, O.mixedrev(plan)[::97])
    A = a.copy()
    REF.ref_vk_conv_foursteps_cfg(A.ctypes.data, bdr.ctypes.data, n, batch, 16, mid, 1)
    ours = O.conv(a, bdr, n, plan, filt_stride=n, tw=O.TW_LIBM)
    assert bits_equal(ours, A.reshape(-1))


@needs_ref
@pytest.mark.parametrize("h,w", [(64, 64), (8, 512), (512, 8)])
def test_conv2d_libm_matches_reference_bitwise(h, w, rng):
    batch = 2
    a = cuniform(rng, (batch, h, w))
    b = cuniform(rng, (batch, h, w)) / (h * w)
    ph, pw = O.ref_plan(h, 8), O.ref_plan(w, 8)
    bdr = np.ascontiguousarray(b[:, O.mixedrev(ph)][:, :, O.mixedrev(pw)])
    ref = np.empty_like(a)
    REF.ref_vk_conv2d(h, w, a.ctypes.data, bdr.ctypes.data, ref.ctypes.data, batch)
    ours = O.conv2d(a, bdr, h, w, ph, pw, filt_stride=h * w, tw=O.TW_LIBM)
    assert bits_equal(ours, ref.reshape(-1))


@needs_ref
@pytest.mark.parametrize("n", [256, 512])
def test_conv_r2_libm_matches_reference_bitwise(n, rng):
    batch = 4
    x = rng.uniform(-1, 1, (batch, n)).astype(np.float32)
    y = rng.uniform(-1, 1, (batch, n)).astype(np.float32)
    b = cuniform(rng, (batch, n)) / n
    plan = O.ref_plan(n, 8)
    bdr = np.ascontiguousarray(b[:, O.mixedrev(plan)])
    lead, nr8 = lead_and_count(n, 8)
    u = np.empty_like(x)
    v = np.empty_like(y)
    REF.ref_vk_conv_r2(n, lead, nr8, 1, x.ctypes.data, y.ctypes.data, bdr.ctypes.data,
                       u.ctypes.data, v.ctypes.data, batch)
    ou, ov = O.conv_r2(x, y, bdr, n, plan, filt_stride=n, tw=O.TW_LIBM)
    assert bits_equal(ou, u.reshape(-1)) and bits_equal(ov, v.reshape(-1))


@needs_ref
@pytest.mark.parametrize("entry", ["ref_vk_main", "ref_mixed_main", "ref_inplace_main"])
def test_reference_self_tests_pass_here(entry):
    """The reference's own CPU suites (verify_kernel, cpu_mixed, cpu_inplace),
    each in a child process: their reports go through C stdio, which would
    otherwise reach the terminal only when pytest exits."""
    code = ("import sys; sys.path.insert(0, sys.argv[1]); from oracle import oracle as O; "
            f"sys.exit(O.load_ref().{entry}())")
    root = str(Path(__file__).resolve().parent.parent)
    p = subprocess.run([sys.executable, "-c", code, root], capture_output=True, text=True, timeout=600)
    assert p.returncode == 0, p.stdout[-2000:] + p.stderr[-2000:]
    assert "FAIL" not in p.stdout.replace("ALL PASS", "")


@needs_ref
@pytest.mark.parametrize("n", [512, 4096])
def test_mixed_f64_restatement_matches_reference(n, rng):
    """The timed CPU baseline path (cpu_mixed.cpp fp64 DIF/mult/DIT)."""
    batch = 2
    a = (rng.uniform(-1, 1, (batch, n)) + 1j * rng.uniform(-1, 1, (batch, n)))
    s = (rng.uniform(-1, 1, (batch, n)) + 1j * rng.uniform(-1, 1, (batch, n))) / n
    ref = np.empty_like(a)
    REF.ref_mixed_conv_f64(n, 16, a.ctypes.data, s.ctypes.data, n, ref.ctypes.data, batch)
    ours = O.mixed_conv_f64(a, s, n, 16)
    assert np.max(np.abs(ours - ref.reshape(-1))) < 1e-12


# ---- 2. golden fixtures -------------------------------------------------------------------

def test_golden_fixtures():
    from tests.golden import golden
    cases = golden.load_all()
    assert cases, "no golden fixtures committed"
    for name, case in cases.items():
        got = golden.replay(case)
        for key, want in got.items():
            assert bits_equal(want, case[key]), f"{name}: {key}"


# ---- 3. table-twiddle accuracy vs fp64 ------------------------------------------------------

@pytest.mark.parametrize("n,v", [(256, 16), (512, 16), (1024, 16), (2048, 16), (4096, 16),
                                 (8192, 16), (16384, 16), (512, 8), (1024, 8), (2048, 8), (4096, 8)])
@pytest.mark.parametrize("mid", ["mul", "conj", "none"])
def test_table_mode_accuracy(n, v, mid, rng):
    batch = 4
    a = crandn(rng, (batch, n))
    spec = crandn(rng, n) / n
    plan = O.kernel_plan(n, v)
    fdr = spec[O.mixedrev(plan)]
    got = O.conv(a, fdr, n, plan, filt_stride=0, mid=mid)
    want = O.conv_spec_f64(a, spec, n, spec_stride=0, mid=mid)
    assert O.rel_l2(got, want) <= 2e-6


@pytest.mark.parametrize("lout,mid_n", [(1, 2048), (1, 4096), (2, 256)])
def test_table_mode_fourstep_accuracy(lout, mid_n, rng):
    n = 16 ** lout * mid_n
    a = cuniform(rng, (1, n))
    spec = cuniform(rng, n) / n
    plan = O.large_plan(lout, mid_n)
    got = O.conv(a, spec[O.mixedrev(plan)], n, plan)
    want = O.conv_spec_f64(a, spec, n)
    assert O.rel_l2(got, want) <= 2e-6


# ---- 4. closed forms --------------------------------------------------------------------------

@pytest.mark.parametrize("n,v", [(512, 16), (4096, 16), (512, 8)])
def test_delta_filter_returns_input(n, v, rng):
    a = crandn(rng, (3, n))
    plan = O.kernel_plan(n, v)
    flat = np.full(n, 1.0 / n, dtype=np.complex64)          # spectrum of delta, 1/N folded
    got = O.conv(a, flat, n, plan)
    assert O.rel_l2(got, a) < 1e-6


@pytest.mark.parametrize("n,v", [(1024, 16), (512, 8)])
def test_delta_signal_returns_taps(n, v, rng):
    h = crandn(rng, n)
    spec = (np.fft.fft(h.astype(np.complex128)) / n).astype(np.complex64)
    plan = O.kernel_plan(n, v)
    delta = np.zeros(n, dtype=np.complex64)
    delta[0] = 1
    got = O.conv(delta, spec[O.mixedrev(plan)], n, plan)
    assert O.rel_l2(got, h) < 1e-6


def test_round_trip_is_n_times_input(rng):
    n = 2048
    a = crandn(rng, (2, n))
    plan = O.kernel_plan(n, 16)
    got = O.conv(a, np.zeros(n, np.complex64), n, plan, mid="none")
    assert O.rel_l2(got, n * a.reshape(-1)) < 1e-6


def test_correlation_by_brute_force(rng):
    """conj-multiply with spec = DFT(h)/N gives y[k] = sum_i a[i+k] conj(h[i])."""
    n = 256
    a = crandn(rng, n).astype(np.complex128)
    h = crandn(rng, n).astype(np.complex128)
    spec = (np.fft.fft(h) / n).astype(np.complex64)
    plan = O.kernel_plan(n, 16)
    got = O.conv(a.astype(np.complex64), spec[O.mixedrev(plan)], n, plan, mid="conj")
    idx = (np.arange(n)[:, None] + np.arange(n)[None, :]) % n
    want = (a[idx] * np.conj(h)[None, :]).sum(axis=1)
    assert O.rel_l2(got, want) < 2e-6


def test_convolution_by_brute_force(rng):
    n = 512
    a = crandn(rng, n).astype(np.complex128)
    h = crandn(rng, n).astype(np.complex128)
    spec = (np.fft.fft(h) / n).astype(np.complex64)
    plan = O.kernel_plan(n, 8)
    got = O.conv(a.astype(np.complex64), spec[O.mixedrev(plan)], n, plan)
    idx = (np.arange(n)[:, None] - np.arange(n)[None, :]) % n
    want = (a[None, :] * h[idx]).sum(axis=1)
    assert O.rel_l2(got, want) < 2e-6


def test_linearity(rng):
    n = 1024
    plan = O.kernel_plan(n, 16)
    a, b = crandn(rng, n), crandn(rng, n)
    f = crandn(rng, n) / n
    lhs = O.conv(a + 2 * b, f, n, plan)
    rhs = O.conv(a, f, n, plan) + 2 * O.conv(b, f, n, plan)
    assert O.rel_l2(lhs, rhs) < 1e-6


@pytest.mark.parametrize("n,v", [(16, 16), (128, 16), (512, 16), (1024, 16), (512, 8), (4096, 8)])
def test_dif_output_order_is_mixedrev(n, v, rng):
    """Unscrambling the forward DIF with mixedrev gives the naive DFT."""
    x = crandn(rng, n)
    plan = O.kernel_plan(n, v)
    spec = O.fwd(x, n, plan)
    un = np.empty_like(spec)
    un[O.mixedrev(plan)] = spec
    k = np.arange(n)
    naive = (x.astype(np.complex128)[None, :] * np.exp(-2j * np.pi * np.outer(k, k) / n)).sum(axis=1)
    assert O.rel_l2(un, naive) < 2e-6


@pytest.mark.parametrize("n,v", [(4096, 16), (512, 8), (2048, 16)])
def test_mixedrev_is_a_permutation(n, v):
    plan = O.kernel_plan(n, v)
    p = O.mixedrev(plan)
    assert np.array_equal(np.sort(p), np.arange(n))
    if len(set(plan.radices)) == 1:                         # pure radix: an involution
        assert np.array_equal(p[p], np.arange(n))


def test_single_radix16_pass_is_dft16(rng):
    x = crandn(rng, 16)
    plan = O.kernel_plan(16, 16)
    assert plan.radices == [16]
    spec = O.fwd(x, 16, plan)
    un = np.empty_like(spec)
    un[O.mixedrev(plan)] = spec
    assert O.rel_l2(un, np.fft.fft(x.astype(np.complex128))) < 1e-6


# ---- 5. the fp64 references --------------------------------------------------------------------

@pytest.mark.parametrize("n", [8, 64, 1024, 4096])
def test_fft2_f64_matches_numpy(n, rng):
    x = (rng.standard_normal(n) + 1j * rng.standard_normal(n))
    assert np.max(np.abs(O.fft2_f64(x, -1) - np.fft.fft(x))) < 1e-10 * n
    assert np.max(np.abs(O.fft2_f64(x, +1) - n * np.fft.ifft(x))) < 1e-10 * n


def test_conv_spec_f64_is_cyclic_convolution(rng):
    n = 128
    a = crandn(rng, n)
    h = crandn(rng, n).astype(np.complex128)
    spec = (np.fft.fft(h) / n).astype(np.complex64)
    got = O.conv_spec_f64(a, spec, n)
    idx = (np.arange(n)[:, None] - np.arange(n)[None, :]) % n
    want = (a.astype(np.complex128)[None, :] * np.fft.ifft(spec.astype(np.complex128) * n)[idx]).sum(axis=1)
    assert np.max(np.abs(got - want)) < 1e-9


# ---- block floating point rule ------------------------------------------------------------------

def test_bfp_exponent_boundaries():
    f32 = np.float32
    assert O.bfp_exponent(0.0) == -128
    assert O.bfp_exponent(float(np.nextafter(f32(0), f32(1)))) == -128      # smallest subnormal
    assert O.bfp_exponent(float(np.finfo(np.float32).tiny)) == -128          # smallest normal
    for e in range(-100, 100):
        edge = f32(32767.0) * f32(2.0) ** e                                   # exactly 32767 * 2^e
        assert O.bfp_exponent(float(edge)) == e
        assert O.bfp_exponent(float(np.nextafter(edge, f32(np.inf)))) == e + 1
        assert O.bfp_exponent(float(np.nextafter(edge, f32(0)))) == e
        assert O.bfp_exponent(float(f32(2.0) ** (e + 14))) == e                 # 16384 * 2^e
        assert O.bfp_exponent(float(-edge)) == e                              # sign ignored


def test_bfp_exponent_is_minimal_and_sufficient(rng):
    vals = np.concatenate([np.exp(rng.uniform(-80, 80, 20000)).astype(np.float32),
                           rng.uniform(0, 1, 2000).astype(np.float32)])
    for a in vals:
        e = O.bfp_exponent(float(a))
        if a < np.finfo(np.float32).tiny or e == -128:
            continue
        assert float(a) <= 32767.0 * 2.0 ** e
        assert float(a) > 32767.0 * 2.0 ** (e - 1)


def test_bfp_quantize_round_trip_and_saturation(rng):
    x = crandn(rng, 64 * 50) * (10.0 ** rng.uniform(-3, 3, 64 * 50)).astype(np.float32)
    x[:64] = 0                                                  # a zero block
    q, e = O.bfp_quantize(x)
    assert e[0] == -128 and np.all(q[:128] == 0)
    assert np.abs(q.astype(np.int32)).max() <= 32767
    xr = O.bfp_dequantize(q, e)
    for b in range(1, 50):
        blk = x[64 * b:64 * (b + 1)]
        m = max(np.abs(blk.real).max(), np.abs(blk.imag).max())
        step = 2.0 ** e[b]
        d = xr[64 * b:64 * (b + 1)] - blk
        assert max(np.abs(d.real).max(), np.abs(d.imag).max()) <= 0.5 * step
        assert m <= 32767 * step
    # the block max lands within one binade below full scale
    assert np.abs(q.astype(np.int32)).reshape(-1, 128)[1:].max(axis=1).min() >= 16383


@pytest.mark.parametrize("block", [64, 128, 512, 4096])
def test_bfp_quantize_any_block_closed_form(block, rng):
    """Blocks of any length: q = rint(x * 2^-e) with e from the block's abs-max
    (the exponent rule is pinned above), restated in numpy."""
    nb = 6
    x = crandn(rng, block * nb) * np.repeat(10.0 ** rng.uniform(-3, 3, nb), block).astype(np.float32)
    x[:block] = 0                                               # a zero block
    q, e = O.bfp_quantize(x, block=block)
    assert e.size == nb
    for b in range(nb):
        blk = x[block * b:block * (b + 1)]
        m = np.float32(max(np.abs(blk.real).max(), np.abs(blk.imag).max()))
        eb = O.bfp_exponent(float(m))
        assert e[b] == eb
        want = np.empty(2 * block, dtype=np.int16)
        want[0::2] = np.rint(np.ldexp(blk.real.astype(np.float64), -eb))
        want[1::2] = np.rint(np.ldexp(blk.imag.astype(np.float64), -eb))
        assert np.array_equal(q[2 * block * b:2 * block * (b + 1)], want)
    assert np.array_equal(O.bfp_dequantize(q, e, block=block).view(np.uint32),
                          np.concatenate([np.ldexp(q[0::2].astype(np.float32), np.repeat(e, block))
                                          + 1j * np.ldexp(q[1::2].astype(np.float32), np.repeat(e, block))
                                          ]).astype(np.complex64).view(np.uint32))


@pytest.mark.parametrize("n,block", [(512, 512), (1024, 256), (4096, 64), (4096, 4096)])
def test_bfp_conv_is_dequantise_conv_quantise(n, block, rng):
    """The BFP conv is the fp32 conv of the dequantised input, quantised with
    the same block length: a composition of pinned pieces."""
    batch = 3
    x = crandn(rng, batch * n) * np.repeat(10.0 ** rng.uniform(-3, 3, batch), n).astype(np.float32)
    q, e = O.bfp_quantize(x, block=block)
    filt = crandn(rng, n, scale=1.0 / n)
    plan = O.kernel_plan(n, 8)
    oq, oe = O.bfp_conv(q, e, filt, n, plan, block=block)
    y = O.conv(O.bfp_dequantize(q, e, block=block), filt, n, plan)
    wq, we = O.bfp_quantize(y, block=block)
    assert np.array_equal(oe, we) and np.array_equal(oq, wq)


# ---- the reference's own BFP format (one fp32 scale per transform) ----------------------

def _scaled_inputs(rng, n, batch):
    """Gaussian signals times 10^u per signal, plus edge
    cases: an all-zero signal (mx = 1e-30) and one whose abs-max sits on the
    imaginary part of its last point."""
    x = (crandn(rng, (batch, n)) * (10.0 ** rng.uniform(-3, 3, (batch, 1)))).astype(np.complex64)
    x[0] = 0
    if batch > 2:
        x[1, -1] = x[1, -1].real + 1j * (4.0 * np.abs(x[1]).max())
    return x.reshape(-1)


@needs_ref
@pytest.mark.parametrize("n", [64, 512, 4096])
def test_bfp_scaled_quantize_matches_reference(n, rng):
    """bfp_quantize (verify_kernel.cpp:1092-1105), bit for bit: words and scales;
    the library's host codec agrees."""
    import fufft_amd as ff
    x = _scaled_inputs(rng, n, 4)
    q, s = O.bfp_scaled_quantize(x, n)
    hq, hs = ff.bfp_scaled_quantize(x, n)
    for t in range(4):
        rq = np.empty(2 * n, np.int16)
        xt = np.ascontiguousarray(x[t * n:(t + 1) * n])
        rs = np.float32(REF.ref_vk_bfp_quantize(xt.ctypes.data, n, rq.ctypes.data))
        assert np.array_equal(q[2 * n * t:2 * n * (t + 1)], rq)
        assert s[t].view(np.uint32) == rs.view(np.uint32)
    assert np.array_equal(q, hq) and np.array_equal(s.view(np.uint32), hs.view(np.uint32))
    assert bits_equal(O.bfp_scaled_dequantize(q, s, n), ff.bfp_scaled_dequantize(q, s, n))


@needs_ref
@pytest.mark.parametrize("n", [256, 512, 1024, 2048, 4096])
def test_bfp_scaled_libm_matches_reference_bitwise(n, rng):
    """kernel_v16_bfp (verify_kernel.cpp:1107-1135, the fufft_pipeline_v16_bfp
    dataflow) against the restatement in LIBM mode, words and scales."""
    batch = 3
    x = _scaled_inputs(rng, n, batch)
    q, s = O.bfp_scaled_quantize(x, n)
    plan = O.kernel_plan(n, 16)
    b = crandn(rng, n, scale=1.0 / n)
    fq, fs = O.bfp_scaled_quantize(b[O.mixedrev(plan)], n)
    lead, nrv = lead_and_count(n, 16)
    rq, rs = np.empty_like(q), np.empty(batch, np.float32)
    REF.ref_vk_v16_bfp(n, lead, nrv, q.ctypes.data, s.ctypes.data, fq.ctypes.data, float(fs[0]),
                       rq.ctypes.data, rs.ctypes.data, batch)
    oq, os_ = O.bfp_scaled_conv(q, s, fq, fs, n, plan, tw=O.TW_LIBM)
    assert np.array_equal(oq, rq)
    assert np.array_equal(os_.view(np.uint32), rs.view(np.uint32))


def test_bfp_scaled_quantize_closed_form(rng):
    """Without the reference: the largest component maps to +-32767, the
    round trip is within half a step, and an all-zero transform has scale
    1e-30 / 32767 and zero words."""
    n = 256
    x = _scaled_inputs(rng, n, 5)
    q, s = O.bfp_scaled_quantize(x, n)
    parts = x.view(np.float32).reshape(5, 2 * n)
    qq = q.reshape(5, 2 * n)
    for t in range(1, 5):
        i = np.argmax(np.abs(parts[t]))
        assert abs(int(qq[t, i])) == 32767 and np.sign(qq[t, i]) == np.sign(parts[t, i])
        err = np.abs(qq[t].astype(np.float64) * np.float64(s[t]) - parts[t])
        assert err.max() <= 0.5 * np.float64(s[t]) * (1 + 1e-6) + np.abs(parts[t]).max() * 1e-6
    assert not qq[0].any() and s[0] == np.float32(np.float32(1e-30) / np.float32(32767.0))


@pytest.mark.parametrize("n,v", [(512, 16), (4096, 8)])
def test_bfp_scaled_conv_is_dequantise_conv_quantise(n, v, rng):
    """The scaled BFP conv is the fp32 conv of the dequantised signal and
    filter, quantised per transform: a composition of pinned pieces, with
    per-transform filters too."""
    batch = 3
    x = _scaled_inputs(rng, n, batch)
    q, s = O.bfp_scaled_quantize(x, n)
    fq, fs = O.bfp_scaled_quantize(crandn(rng, batch * n, scale=1.0 / n), n)
    plan = O.kernel_plan(n, v)
    oq, os_ = O.bfp_scaled_conv(q, s, fq, fs, n, plan, filt_stride=n, mid="conj")
    y = O.conv(O.bfp_scaled_dequantize(q, s, n), O.bfp_scaled_dequantize(fq, fs, n), n, plan, filt_stride=n,
               mid="conj")
    wq, ws = O.bfp_scaled_quantize(y, n)
    assert np.array_equal(oq, wq) and np.array_equal(os_, ws)
