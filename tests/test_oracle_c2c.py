"""Pin the oracle's natural-order C2C (or_c2c_f32) before it checks the GPU.

The reference's fufft_c2c (fufft.cuh:879-904; CPU transcription kernel_c2c,
verify_kernel.cpp:1183-1203) is a forward radix-8 Stockham transform; this
build's C2C is the in-place DIF of the conv path plus one exact permutation
(and, inverse, the permutation plus the DIT).  Different operation orders, so
the pins are:

1. bit-identity of the forward C2C with the DIF output permuted by mixedrev,
   and of the inverse with the digit-order DIT -- the DIF / DIT passes are
   themselves pinned bit for bit to the reference transcription;
2. the reference's Stockham transform (compiled where it lies, and the
   golden fixture written from it) to within fp32 rounding;
3. closed forms: a delta gives exactly all ones, a pure tone gives N in one
   bin, numpy's fp64 FFT / IFFT within 2e-6, and inverse(forward(x)) = N x.
"""
import numpy as np
import pytest

from conftest import bits_equal, crandn, cuniform
from oracle import oracle as O

REF = O.load_ref()
needs_ref = pytest.mark.skipif(REF is None, reason="reference CPU sources not built here")

PLANS = [(n, 16) for n in (256, 512, 1024, 2048, 4096, 8192, 16384)] + \
        [(n, 8) for n in (512, 1024, 2048, 4096, 8192)]


@pytest.mark.parametrize("n,v", PLANS)
@pytest.mark.parametrize("tw", [O.TW_LIBM, O.TW_TABLE])
def test_forward_is_dif_then_permutation(n, v, tw, rng):
    a = crandn(rng, (3, n))
    plan = O.kernel_plan(n, v)
    perm = O.mixedrev(plan)
    spec = O.fwd(a, n, plan, tw=tw).reshape(3, n)
    nat = O.c2c(a, n, plan, -1, tw=tw).reshape(3, n)
    assert bits_equal(nat[:, perm], spec)


@pytest.mark.parametrize("n,v", PLANS)
def test_inverse_is_permutation_then_dit(n, v, rng):
    x = crandn(rng, (3, n))
    plan = O.kernel_plan(n, v)
    perm = O.mixedrev(plan)
    want = O.apply(np.ascontiguousarray(x[:, perm]), np.zeros(1, np.complex64), n, 3, plan,
                   spec_stride=n, mid="none")
    assert bits_equal(O.c2c(x, n, plan, +1), want)


@pytest.mark.parametrize("n,v", PLANS)
def test_against_numpy_fp64(n, v, rng):
    a = crandn(rng, (4, n))
    plan = O.kernel_plan(n, v)
    fwd = O.c2c(a, n, plan, -1).reshape(4, n)
    inv = O.c2c(a, n, plan, +1).reshape(4, n)
    a64 = a.astype(np.complex128)
    assert O.rel_l2(fwd, np.fft.fft(a64, axis=1)) <= 2e-6
    assert O.rel_l2(inv, np.fft.ifft(a64, axis=1) * n) <= 2e-6
    # inverse(forward(x)) = n x
    back = O.c2c(fwd, n, plan, +1).reshape(4, n)
    assert O.rel_l2(back / n, a64) <= 2e-6


@pytest.mark.parametrize("n,v", [(512, 8), (4096, 8), (1024, 16), (16384, 16)])
def test_delta_and_tone(n, v):
    plan = O.kernel_plan(n, v)
    d = np.zeros(n, np.complex64)
    d[0] = 1
    assert bits_equal(O.c2c(d, n, plan, -1), np.ones(n, np.complex64))
    assert bits_equal(O.c2c(d, n, plan, +1), np.ones(n, np.complex64))
    f = 37 % n
    tone = np.exp(2j * np.pi * f * np.arange(n) / n).astype(np.complex64)
    got = O.c2c(tone, n, plan, -1)
    want = np.zeros(n, np.complex128)
    want[f] = n
    assert O.rel_l2(got, want) <= 2e-6
    assert int(np.argmax(np.abs(got))) == f


@needs_ref
@pytest.mark.parametrize("n", [64, 512, 4096])
def test_reference_stockham_to_rounding(n, rng):
    batch = 4
    a = cuniform(rng, (batch, n))
    ref = np.empty_like(a)
    REF.ref_vk_c2c(n, 1, a.ctypes.data, ref.ctypes.data, batch)
    plan = O.ref_plan(n, 8)
    ours = O.c2c(a, n, plan, -1, tw=O.TW_LIBM)
    truth = np.fft.fft(a.astype(np.complex128), axis=1).reshape(-1)
    assert O.rel_l2(ref.reshape(-1), truth) <= 2e-6
    assert O.rel_l2(ours, truth) <= 2e-6
    assert O.rel_l2(ours, ref.reshape(-1)) <= 2e-6


def test_golden_stockham_fixture():
    from tests.golden import golden
    case = golden.load_all()["c2c_stockham_n512"]
    n = int(case["n"])
    ours = O.c2c(case["a"], n, O.ref_plan(n, 8), -1, tw=O.TW_LIBM)
    assert O.rel_l2(ours, case["out"]) <= 2e-6
    truth = np.fft.fft(case["a"].astype(np.complex128).reshape(-1, n), axis=1).reshape(-1)
    assert O.rel_l2(case["out"], truth) <= 2e-6
