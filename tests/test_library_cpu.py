"""CPU tests of the HIP library's host side (no GPU calls).

- every function include/fufft/fufft.h declares is exported by libfufft_amd.so;
- host planning (radices, digit orders, filter planning in 1D, four-step and
  2D) agrees with the oracle's plans;
- the twiddle table the library uploads equals the oracle's table entry for
  entry, bit for bit;
- the BFP host codec equals the oracle's;
- argument errors come back as status codes before any HIP call.
"""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from conftest import bperm, crandn, lane_major, lane_slot
from oracle import oracle as O

ROOT = Path(__file__).resolve().parent.parent


def header_functions():
    text = (ROOT / "include" / "fufft" / "fufft.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fufft_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    import fufft_amd as ff
    names = header_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(ff.lib, n)]
    assert not missing, missing


def test_abi_version_matches_header():
    import fufft_amd as ff
    text = (ROOT / "include" / "fufft" / "fufft.h").read_text()
    declared = int(re.search(r"#define FUFFT_ABI_VERSION\s+(\d+)", text).group(1))
    assert ff.lib.fufft_abi_version() == declared == ff.ABI_VERSION


@pytest.mark.parametrize("variant,v", [("v16", 16), ("r8", 8)])
@pytest.mark.parametrize("n", [256, 512, 1024, 2048, 4096, 8192, 16384])
def test_plan_and_digit_order_match_oracle(variant, v, n):
    import fufft_amd as ff
    plan = O.kernel_plan(n, v)
    assert ff.plan_radices(n, variant) == plan.radices
    assert ff.plan_chains(n, variant) == plan.chains
    assert np.array_equal(ff.digit_order(n, variant), O.mixedrev(plan))


def test_auto_variant_rule():
    import fufft_amd as ff
    for n in [256, 512, 1024, 2048, 4096, 8192, 16384]:
        want = "r8" if n in (512, 4096, 8192) else "v16"
        assert ff.resolve_variant(n, "auto") == want
        assert ff.plan_radices(n, "auto") == ff.plan_radices(n, want)
        # FUFFT_AUTO is the faster variant for the digit-order filter
        assert ff.fastest_variant(n, "dr") == want
        # with the lane-major filter radix 16 wins from n = 1024 on
        assert ff.fastest_variant(n, "lane") == ("r8" if n == 512 else "v16")
        assert ff.supported(n, ff.fastest_variant(n, "lane"))
    # N = 32768: the fused conv alone, radix 16 (wide.hip)
    assert ff.fastest_variant(32768, "lane") == ff.fastest_variant(32768, "dr") == "v16"
    assert ff.resolve_variant(32768, "auto") == "v16"
    assert ff.supported(32768, "v16") and ff.supported(32768, "auto") and not ff.supported(32768, "r8")
    for bad in (100, 128, 65536):
        with pytest.raises(ff.FufftError):
            ff.fastest_variant(bad, "lane")


def test_n32768_is_the_fused_conv_only():
    """At N = 32768 every 1D call but the fused conv refuses the size before
    touching a device (fake addresses, never used)."""
    import fufft_amd as ff
    L, A, n = ff.lib, 1 << 32, 32768
    B = A + (1 << 24)
    assert L.fufft_fwd_f32(A, B, n, 1, 0, None) == ff.ERR_UNSUPPORTED
    assert L.fufft_apply_f32(A, n, B, 0, B + (1 << 22), n, 1, 0, 0, 0, None) == ff.ERR_UNSUPPORTED
    assert L.fufft_c2c_f32(A, B, n, 1, -1, 0, None) == ff.ERR_UNSUPPORTED
    assert L.fufft_conv_r2_f32(A, A + (1 << 20), B, 0, B + (1 << 20), B + (1 << 21), n, 1, 0, 0, None) \
        == ff.ERR_UNSUPPORTED
    assert L.fufft_conv_bfp16(A, A + (1 << 20), B, 0, B + (1 << 20), B + (1 << 21), n, 1, 64, 0, 0, 0, None) \
        == ff.ERR_UNSUPPORTED
    assert L.fufft_conv_timed_f32(A, B, 0, B + (1 << 20), n, 1, 0, 0, 0, None, 0, None) == ff.ERR_UNSUPPORTED
    # taps need the forward transform (not built at this size); spectra are only permuted
    assert L.fufft_plan_filter_device_f32(A, B, n, 1, 0, 0, 1, 1, None) == ff.ERR_UNSUPPORTED
    assert L.fufft_plan_filter_device_f32(A, A + 8, n, 1, 0, 0, 0, 1, None) == ff.ERR_ALIGN
    # the radix-8 plan has no N = 32768 kernel, the fused conv included
    assert L.fufft_conv_f32(A, B, 0, B + (1 << 20), n, 1, 0, 1, 0, None) == ff.ERR_UNSUPPORTED


def run_large_chain_order(n, lout, mid):
    """The filter permutation run_large builds (bench_fufft.cu:410-428), restated
    from its loop: digit widths [4]*lout ++ [log2 lead] ++ [4]*nrv of the V=16
    middle, each index's digits read from the top, reassembled reversed."""
    lead_bits = int(np.log2(mid)) % 4
    wid = [4] * lout + ([lead_bits] if lead_bits else []) + [4] * (int(np.log2(mid)) // 4)
    mb = sum(wid)
    out = np.empty(n, dtype=np.int64)
    for i in range(n):
        pos, dg = mb, []
        for w in wid:
            pos -= w
            dg.append((i >> pos) & ((1 << w) - 1))
        r, op = 0, mb
        for k in range(len(wid) - 1, -1, -1):
            op -= wid[k]
            r |= dg[k] << op
        out[i] = r
    return out


@pytest.mark.parametrize("n", [8192, 32768, 65536, 131072])
@pytest.mark.parametrize("variant,v", [("v16", 16), ("r8", 8), ("auto", 16)])
def test_large_plan_matches_oracle(n, variant, v):
    import fufft_amd as ff
    lout, mid = ff.large_plan(n)
    assert 16 ** lout * mid == n and 512 <= mid <= 4096
    assert np.array_equal(ff.large_digit_order(n, variant), O.mixedrev(O.large_plan(lout, mid, v)))


@pytest.mark.parametrize("n,lout,mid", [(32768, 1, 2048), (65536, 1, 4096), (8192, 1, 512)])
def test_large_v16_chain_is_run_large_order(n, lout, mid):
    """The default four-step chain is the reference's: a filter permuted as
    run_large<32768, 1, 16, 2048, 8, 2> permutes it passes unchanged."""
    import fufft_amd as ff
    assert ff.large_plan(n) == (lout, mid)
    want = run_large_chain_order(n, lout, mid)
    assert np.array_equal(ff.large_digit_order(n), want)
    assert np.array_equal(ff.large_digit_order(n, "v16"), want)
    # the radix-8 middle is a different order (it is not the reference's GPU chain)
    assert not np.array_equal(ff.large_digit_order(n, "r8"), want)


def test_filter_planning_1d_layouts(rng):
    import fufft_amd as ff
    n, v = 2048, 8
    taps = crandn(rng, n)
    want = np.fft.fft(taps.astype(np.complex128)) / n
    dr = ff.plan_filter(taps, n, variant="r8", kind=ff.FILTER_TAPS)
    perm = O.mixedrev(O.kernel_plan(n, v))
    assert np.max(np.abs(dr - want[perm])) <= 2e-7 * np.max(np.abs(want))
    # the spectrum form skips the host DFT: slot i is the fp32 bin perm[i] / n
    spec = (want * n).astype(np.complex64)
    dr2 = ff.plan_filter(spec, n, variant="r8", kind=ff.FILTER_SPECTRUM)
    assert np.array_equal(dr2, (spec.astype(np.complex128) / n).astype(np.complex64)[perm])
    lane = ff.plan_filter(spec, n, variant="r8", layout="lane", kind=ff.FILTER_SPECTRUM)
    assert np.array_equal(lane, lane_major(dr2, n, v))
    # the reference's bperm (verify_kernel.cpp:1381-1387): bperm[L + k*T] = b_dr[V*L + k]
    bp = ff.plan_filter(spec, n, variant="r8", layout="bperm", kind=ff.FILTER_SPECTRUM)
    assert np.array_equal(bp, bperm(dr2, n, v))
    t = n // v
    assert np.array_equal(bp[3 + 5 * t], dr2[v * 3 + 5])
    # 2D filters take the reference's order or the library's, not bperm
    with pytest.raises(ff.FufftError) as ei:
        ff.plan_filter2d(crandn(rng, 256 * 256), 256, 256, layout="bperm")
    assert ei.value.status == ff.ERR_INVALID
    # the pairs: lane L's values 2m, 2m + 1 side by side at 2(L + m*T)
    t = n // v
    for L, m in ((0, 0), (3, 1), (t - 1, v // 2 - 1)):
        assert np.array_equal(lane[2 * (L + m * t): 2 * (L + m * t) + 2], dr2[L * v + 2 * m: L * v + 2 * m + 2])


def test_filter_planning_large_and_2d(rng):
    import fufft_amd as ff
    n = 32768
    taps = crandn(rng, n)
    want = np.fft.fft(taps.astype(np.complex128)) / n
    for variant in ("auto", "v16", "r8"):
        got = ff.plan_filter_large(taps, n, kind=ff.FILTER_TAPS, variant=variant)
        assert np.max(np.abs(got - want[ff.large_digit_order(n, variant)])) <= 2e-7 * np.max(np.abs(want))
    h, w = 256, 1024
    taps2 = crandn(rng, h * w)
    vr, vc = ff.plan2d(h, w)
    S = np.fft.fft2(taps2.reshape(h, w).astype(np.complex128)) / (h * w)
    rh, rw = O.mixedrev(O.kernel_plan(h, vc)), O.mixedrev(O.kernel_plan(w, vr))
    got2 = ff.plan_filter2d(taps2, h, w, kind=ff.FILTER_TAPS, layout="lane")
    # the reference's order: slot (r, c) = bin (rev_h(r), rev_w(c))
    got2_dr = ff.plan_filter2d(taps2, h, w, kind=ff.FILTER_TAPS, layout="dr")
    want2_dr = S[np.ix_(rh, rw)].reshape(-1)
    assert np.max(np.abs(got2_dr - want2_dr)) <= 2e-7 * np.max(np.abs(want2_dr))
    # columns in the library's order: the rows' lane-major pair layout
    slot = ff.column_order2d(h, w)
    assert np.array_equal(slot, [lane_slot(c, w, vr) for c in range(w)])
    assert sorted(slot) == list(range(w))
    want2 = S[np.ix_(rh, rw[slot])].reshape(-1)
    assert np.max(np.abs(got2 - want2)) <= 2e-7 * np.max(np.abs(want2))


def test_twiddle_table_matches_oracle_bitwise():
    import fufft_amd as ff
    log_max = 13
    tab = ff.twiddle_table_host(log_max).view(np.float32).reshape(-1, 2)
    c, s = C.c_float(), C.c_float()
    for p in range(1, log_max + 1):
        P = 1 << p
        js = range(P) if P <= 1024 else list(range(0, P, 7)) + [P - 1]
        for j in js:
            O.lib.or_twiddle(O.TW_TABLE, +1, P, j, C.byref(c), C.byref(s))
            assert tab[P + j, 0] == np.float32(c.value) and tab[P + j, 1] == np.float32(s.value), (P, j)


def test_reference_twiddle_table_matches_libm_mode_both_signs():
    """FUFFT_TWIDDLES_REFERENCE holds the fp32-angle cosf/sinf of the
    reference's transcription (the oracle's LIBM mode, which is pinned bit for
    bit to the compiled reference).  The kernels negate the stored sine for
    the forward passes, so that negation must equal the forward's own
    cosf/sinf(-angle) bit for bit too."""
    import fufft_amd as ff
    log_max = 20
    tab = ff.twiddle_table_host(log_max, "reference").view(np.float32).reshape(-1, 2)
    acc = ff.twiddle_table_host(log_max, "accurate").view(np.float32).reshape(-1, 2)
    c, s = C.c_float(), C.c_float()
    differs = 0
    for p in range(1, log_max + 1):
        P = 1 << p
        js = range(P) if P <= 4096 else list(range(0, P, 97)) + [P - 1]
        for j in js:
            O.lib.or_twiddle(O.TW_LIBM, +1, P, j, C.byref(c), C.byref(s))
            assert tab[P + j].view(np.uint32).tolist() == \
                np.array([c.value, s.value], np.float32).view(np.uint32).tolist(), (P, j)
            O.lib.or_twiddle(O.TW_LIBM, -1, P, j, C.byref(c), C.byref(s))
            neg = np.array([tab[P + j, 0], -tab[P + j, 1]], np.float32)
            assert neg.view(np.uint32).tolist() == \
                np.array([c.value, s.value], np.float32).view(np.uint32).tolist(), (P, j, "fwd")
            differs += int(tab[P + j, 0] != acc[P + j, 0] or tab[P + j, 1] != acc[P + j, 1])
    assert differs > 1000          # the two sources really differ
    with pytest.raises(ff.FufftError):
        ff.check(ff.lib.fufft_twiddle_table_host_source(4, 7, tab.ctypes.data), "bad source")


def test_bfp_codec_matches_oracle(rng):
    import fufft_amd as ff
    vals = [0.0, 1e-45, 1.17e-38, 1.0, 32767.0, 32767.5, 32768.0, 65534.0, 65535.0, 3.4e38]
    for m in vals + list(np.abs(rng.standard_normal(200) * 10.0 ** rng.uniform(-30, 30, 200))):
        x = float(np.float32(m))
        assert ff.bfp_exponent(x) == O.bfp_exponent(x), x
    x = (crandn(rng, 64 * 40) * 10.0 ** rng.uniform(-3, 3)).astype(np.complex64)
    x[:64] = 0
    for block in (64, 128, 640, 64 * 40):
        q, e = ff.bfp_quantize(x, block=block)
        oq, oe = O.bfp_quantize(x, block=block)
        assert e.size == x.size // block
        assert np.array_equal(q, oq) and np.array_equal(e, oe)
        assert np.array_equal(ff.bfp_dequantize(q, e, block=block), O.bfp_dequantize(oq, oe, block=block))


def test_status_codes_without_gpu_calls():
    """Size, pointer and alignment checks precede every HIP call."""
    import fufft_amd as ff
    L = ff.lib
    fake = 1 << 20                              # never dereferenced: the checks fail first
    assert L.fufft_conv_f32(fake, fake, 0, fake, 1000, 1, 0, 2, 0, None) == ff.ERR_UNSUPPORTED
    assert L.fufft_conv_f32(fake, fake, 0, fake, 4096, 1, 7, 2, 0, None) == ff.ERR_INVALID
    assert L.fufft_conv_f32(None, fake, 0, fake, 4096, 1, 0, 2, 0, None) == ff.ERR_INVALID
    assert L.fufft_conv_f32(fake + 8, fake, 0, fake, 4096, 1, 0, 2, 0, None) == ff.ERR_ALIGN
    assert L.fufft_conv_f32(fake, fake, 17, fake, 4096, 1, 0, 2, 0, None) == ff.ERR_INVALID
    assert L.fufft_conv_f32(fake, fake, 0, fake, 4096, -1, 0, 2, 0, None) == ff.ERR_INVALID
    assert L.fufft_conv_f32(fake, fake, 0, fake, 4096, 1, 0, 9, 0, None) == ff.ERR_INVALID
    assert L.fufft_conv_bfp16(fake, fake, fake, 0, fake, fake, 256, 1, 64, 0, 1, 0, None) == ff.ERR_UNSUPPORTED
    for block in (32, 96, 8192):                # below 64, not a power of two, longer than n
        assert L.fufft_conv_bfp16(fake, fake, fake, 0, fake, fake, 4096, 1, block, 0, 1, 0, None) == ff.ERR_INVALID
    assert L.fufft_conv_large_f32(fake, fake, 0, 4096, 1, 0, 2, None) == ff.ERR_UNSUPPORTED
    assert L.fufft_conv_large_f32(fake, fake, 3, 32768, 1, 0, 2, None) == ff.ERR_INVALID
    assert L.fufft_conv_large_f32(fake, fake, 0, 32768, 1, 0, 7, None) == ff.ERR_INVALID   # variant
    assert L.fufft_large_digit_order(32768, 7, (C.c_int32 * 32768)()) == ff.ERR_INVALID
    assert L.fufft_plan_filter_large_f32(32768, 7, 1, 1, fake, fake) == ff.ERR_INVALID
    assert L.fufft_conv2d_f32(fake, fake, 0, fake, 128, 512, 1, 0, 0, None) == ff.ERR_UNSUPPORTED
    assert L.fufft_conv2d_f32(fake, fake, 0, fake, 512, 100, 1, 0, 0, None) == ff.ERR_UNSUPPORTED
    assert L.fufft_conv2d_f32(fake, fake, 5, fake, 512, 512, 1, 0, 0, None) == ff.ERR_INVALID
    assert L.fufft_conv2d_f32(fake, fake, 0, fake, 512, 512, 1, 0, 7, None) == ff.ERR_INVALID
    assert L.fufft_conv2d_r2_f32(fake, fake, fake, 0, fake, fake, fake, 512, 512, 1, 7, None) == ff.ERR_INVALID
    assert L.fufft_apply2d_f32(fake, 0, fake, 0, fake, 512, 512, 2, 0, 0, None) == ff.ERR_INVALID
    assert L.fufft_apply2d_f32(fake, 0, fake, 0, fake + 16, 512, 512, 2, 0, 7, None) == ff.ERR_INVALID
    # 1D apply: a spectrum shared by the batch must not be the output
    assert L.fufft_apply_f32(fake, 0, fake, 0, fake, 4096, 2, 0, 2, 0, None) == ff.ERR_INVALID
    assert L.fufft_plan_filter2d_f32(512, 512, 7, 0, 1, fake, fake) == ff.ERR_INVALID
    # the workspace-free 2D call refuses an image larger than its static scratch before any GPU call
    assert L.fufft_conv2d_r2_noalloc_f32(fake, fake, fake, 0, fake, fake, 2048, 8192, 1, 1, None) == ff.ERR_SCRATCH
    assert L.fufft_conv2d_r2_noalloc_f32(fake, fake, fake, 0, fake, fake, 512, 512, 1, 7, None) == ff.ERR_INVALID
    assert L.fufft_bfp_quantize(None, 64, 64, None, None) == ff.ERR_INVALID
    assert L.fufft_bfp_quantize(fake, 65, 64, fake, fake) == ff.ERR_INVALID
    assert L.fufft_bfp_quantize(fake, 64, 0, fake, fake) == ff.ERR_INVALID
    assert L.fufft_c2c_f32(fake, fake, 4096, 1, 0, 2, None) == ff.ERR_INVALID
    assert L.fufft_c2c_f32(fake, fake, 4097, 1, -1, 2, None) == ff.ERR_UNSUPPORTED
    assert L.fufft_c2c_f32(fake + 8, fake, 4096, 1, -1, 2, None) == ff.ERR_ALIGN
    assert L.fufft_plan_filter_device_f32(fake, fake, 4096, 1, 2, 0, 0, 1, None) == ff.ERR_INVALID
    assert L.fufft_plan_filter_device_f32(fake, fake + 16, 4096, 1, 2, 0, 5, 1, None) == ff.ERR_INVALID
    assert L.fufft_plan_filter_large_device_f32(fake, fake, 4096, 1, 2, 1, 1, None) == ff.ERR_UNSUPPORTED
    assert L.fufft_plan_filter_large_device_f32(fake, fake + 16, 32768, 1, 7, 1, 1, None) == ff.ERR_INVALID
    assert L.fufft_plan_filter2d_device_f32(fake, fake, 512, 100, 1, 0, 1, 1, None) == ff.ERR_UNSUPPORTED
    assert L.fufft_plan_filter2d_device_f32(fake, fake + 16, 512, 512, 1, 7, 1, 1, None) == ff.ERR_INVALID
    # the reference-format BFP conv and codec
    S = L.fufft_conv_bfp16_scaled
    assert S(fake, fake, fake, fake, 0, fake, fake, 128, 1, 0, 0, 0, None) == ff.ERR_UNSUPPORTED   # radix 16 from 256
    assert S(fake, fake, fake, fake, 0, fake, fake, 256, 1, 0, 1, 0, None) == ff.ERR_UNSUPPORTED   # radix 8 from 512
    assert S(fake, fake, None, fake, 0, fake, fake, 4096, 1, 0, 0, 0, None) == ff.ERR_INVALID     # mul reads a filter
    assert S(fake, None, fake, fake, 0, fake, fake, 4096, 1, 0, 0, 0, None) == ff.ERR_INVALID     # no input scales
    assert S(fake, fake, fake, fake, 5, fake, fake, 4096, 1, 0, 0, 0, None) == ff.ERR_INVALID     # filter stride
    assert S(fake, fake, fake + 4, fake, 0, fake, fake, 4096, 1, 0, 0, 0, None) == ff.ERR_ALIGN
    assert S(fake + 2, fake, fake, fake, 0, fake, fake, 4096, 1, 0, 0, 0, None) == ff.ERR_ALIGN
    assert S(fake, fake, None, None, 0, fake, fake, 4096, 1, 7, 0, 0, None) == ff.ERR_INVALID     # unknown mid
    assert S(fake, fake, fake, fake, 0, fake, fake, 4096, 1, 0, 0, 3, None) == ff.ERR_INVALID  # unknown layout
    assert L.fufft_bfp_scaled_quantize(None, 64, 1, fake, fake) == ff.ERR_INVALID
    assert L.fufft_bfp_scaled_quantize(fake, 0, 1, fake, fake) == ff.ERR_INVALID
    # the stream copy's shape is checked before any launch
    SS = L.fufft_stream_shape_f32
    assert SS(fake, fake + 1024, 4096, 128, 16, 8, 1, 0, 0, 0, None) == ff.ERR_INVALID     # lanes
    assert SS(fake, fake + 1024, 4096, 256, 16, 6, 1, 0, 0, 0, None) == ff.ERR_INVALID     # loads per lane
    assert SS(fake, fake + 1024, 4096, 1024, 16, 32, 1, 0, 0, 0, None) == ff.ERR_INVALID   # 512 KiB tile
    assert SS(fake, fake + 1024, 4096, 256, 16, 64, 1, 0, 0, 0, None) == ff.ERR_INVALID
    assert SS(fake, fake + 1024, 4096, 256, 4, 8, 1, 0, 0, 0, None) == ff.ERR_INVALID      # load width
    assert SS(fake, fake + 1024, 4096, 256, 16, 8, 0, 0, 0, 0, None) == ff.ERR_INVALID     # tiles per group
    assert SS(fake, fake + 1024, 4096, 256, 16, 8, 1, -1, 0, 0, None) == ff.ERR_INVALID    # groups
    assert SS(fake, fake + 1024, 4096, 256, 16, 8, 1, 0, 4, 0, None) == ff.ERR_INVALID     # load policy
    assert SS(fake, fake + 1024, 4096, 256, 16, 8, 1, 0, 0, 4, None) == ff.ERR_INVALID     # store policy
    assert SS(fake, fake + 1024, 4100, 256, 16, 8, 1, 0, 0, 0, None) == ff.ERR_INVALID     # not 16-byte granular
    assert SS(fake, fake, 4096, 256, 16, 8, 1, 0, 0, 0, None) == ff.ERR_INVALID            # in == out
    assert SS(fake + 8, fake + 1024, 4096, 256, 16, 8, 1, 0, 0, 0, None) == ff.ERR_ALIGN
    assert L.fufft_status_string(ff.ERR_ALIGN).decode().startswith("misaligned pointer")
    assert "scratch" in L.fufft_status_string(ff.ERR_SCRATCH).decode()


def test_mid_policy_registry():
    """The mid ids the library registers (MidMultiply, MidConjMultiply,
    MidNothing: fufft.cuh:616-650) and which read a filter; an id no policy
    has is refused by every call that takes one, before any device work, and
    by the binding whether given as a name or an id."""
    import fufft_amd as ff
    L = ff.lib
    assert [L.fufft_mid_reads_filter(m) for m in (0, 1, 2)] == [1, 1, 0]
    for bad in (-1, 3, 99):
        assert L.fufft_mid_reads_filter(bad) == ff.ERR_INVALID
    assert [ff.mid_reads_filter(m) for m in ("mul", "conj", "none")] == [True, True, False]
    assert ff.mid_reads_filter(ff.MID["conj"]) is True
    with pytest.raises(ff.FufftError):
        ff.mid_reads_filter(3)
    with pytest.raises(ValueError, match="mid must be"):
        ff.mid_reads_filter("product")
    fake = 1 << 20
    # a filter pointer may be NULL exactly where the policy reads none
    assert L.fufft_conv_f32(fake, None, 0, fake, 4096, 1, 0, 2, 0, None) == ff.ERR_INVALID
    assert L.fufft_conv_f32(fake, None, 0, fake, 4096, 1, 1, 2, 0, None) == ff.ERR_INVALID
    for mid in (3, -1):
        assert L.fufft_conv_f32(fake, fake, 0, fake, 4096, 1, mid, 2, 0, None) == ff.ERR_INVALID
        assert L.fufft_apply_f32(fake, 4096, fake, 0, fake + 16, 4096, 1, mid, 2, 0, None) == ff.ERR_INVALID
        assert L.fufft_conv_bfp16(fake, fake, fake, 0, fake, fake, 4096, 1, 64, mid, 1, 0, None) == ff.ERR_INVALID
        assert L.fufft_conv_large_f32(fake, fake, 0, 32768, 1, mid, 2, None) == ff.ERR_INVALID
        assert L.fufft_conv2d_f32(fake, fake, 0, fake, 512, 512, 1, mid, 0, None) == ff.ERR_INVALID
        assert L.fufft_apply2d_f32(fake, 0, fake, 0, fake + 16, 512, 512, 1, mid, 0, None) == ff.ERR_INVALID


def test_cpp_mirror_header_builds_and_runs(tmp_path):
    """include/fufft/fufft.hpp compiles with g++ and links against the library."""
    import shutil
    import subprocess
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    lib_dir = ROOT / "fufft_amd"
    exe = tmp_path / "hpp_check"
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", f"-I{ROOT / 'include'}",
                    str(ROOT / "tests" / "cpp" / "hpp_check.cpp"), f"-L{lib_dir}", "-lfufft_amd",
                    f"-Wl,-rpath,{lib_dir}", "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, (out.returncode, out.stderr)
    assert out.stdout.startswith("ok")


# fufft::ref (the reference's launch surface by name): a template whose
# parameters do not spell a plan the library runs must not compile.  Each case
# is a call that compiles with the first template arguments and fails with the
# second, with the static_assert's text.
REF_TEMPLATE_CASES = [
    ("fufft_pipeline_v16<4096, 1, 3, 1>", "fufft_pipeline_v16<4096, 2, 3, 1>",
     "(nullptr, nullptr, fufft::MidMultiply{}, 1)", "N must be LEAD * 16^NRV"),
    ("fufft_pipeline_v16f<2048, 8, 2, 1>", "fufft_pipeline_v16f<2048, 16, 1, 1>",
     "(nullptr, nullptr, nullptr, 1)", "N must be LEAD * 16^NRV"),
    ("fufft_pipeline_ip<1024, 2, 3, 4, fufft::MidNothing>", "fufft_pipeline_ip<4096, 8, 3, 4, fufft::MidNothing>",
     "(nullptr, nullptr, fufft::MidNothing{}, 1)", "N must be LEAD * 8^NR8"),
    ("fufft_pipeline_v16_bfp<4096, 1, 3, 16>", "fufft_pipeline_v16_bfp<4096, 1, 3, 32>",
     "(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 1)", "1 <= CPB <= 16"),
    ("fufft_c2c<4096, 4, 1>", "fufft_c2c<4096, 3, 1>", "(nullptr, nullptr, 1)", "N must be 8^LOG8N"),
    ("run_large<32768, 1, 16, 2048, 8, 2>", "run_large<32768, 1, 8, 4096, 1, 4>", "(nullptr, nullptr, 1)",
     "the outer levels are radix 16"),
    ("run_large<65536, 1, 16, 4096, 1, 3>", "run_large<65536, 1, 16, 4096, 2, 3>", "(nullptr, nullptr, 1)",
     "N must be 16^LOUT * MID"),
]


@pytest.mark.parametrize("good,bad,args,message", REF_TEMPLATE_CASES)
def test_cpp_reference_templates_checked_at_compile_time(tmp_path, good, bad, args, message):
    import shutil
    import subprocess
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")

    def compile_call(call):
        src = tmp_path / "ref_case.cpp"
        src.write_text('#include "fufft/fufft.hpp"\nint f() { return fufft::ref::' + call + args + '; }\n')
        return subprocess.run(["g++", "-std=c++17", "-fsyntax-only", f"-I{ROOT / 'include'}", str(src)],
                              capture_output=True, text=True)

    ok = compile_call(good)
    assert ok.returncode == 0, ok.stderr
    refused = compile_call(bad)
    assert refused.returncode != 0
    assert message in refused.stderr, refused.stderr[-2000:]


def test_cpp_plan_objects_build_and_reject_bad_arguments(tmp_path):
    """include/fufft/plan.hpp (plan objects that own their device filter)
    compiles with g++ against the HIP headers, and each plan object throws
    fufft::Error with the C ABI status before any allocation or device call
    (tests/cpp/plan_check.cpp)."""
    import shutil
    import subprocess
    rocm = Path("/opt/rocm")
    if shutil.which("g++") is None or not (rocm / "include" / "hip" / "hip_runtime_api.h").exists():
        pytest.skip("g++ or the HIP headers are not available")
    lib_dir = ROOT / "fufft_amd"
    exe = tmp_path / "plan_check"
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
                    f"-I{ROOT / 'include'}", f"-I{rocm / 'include'}",
                    str(ROOT / "tests" / "cpp" / "plan_check.cpp"), f"-L{lib_dir}", "-lfufft_amd",
                    f"-L{rocm / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{lib_dir}", f"-Wl,-rpath,{rocm / 'lib'}",
                    "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, (out.returncode, out.stdout, out.stderr)
    assert out.stdout.startswith("ok")
