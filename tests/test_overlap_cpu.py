"""Buffer overlap rules of the C ABI, checked without a GPU: the device
buffers of one call either coincide where the call works in place, or share
no byte; a partial overlap (an output reaching into an input another
workgroup or sub-batch still reads, an output over the filter, two outputs
over each other) returns FUFFT_ERR_INVALID before anything touches a device.
No reference counterpart: the reference's kernels take `__restrict__`
pointers (fufft.cuh:1499-1534) and leave aliasing to the caller.  Every case
names the pointer that overlaps: moved far away (by `AWAY`), the same call
passes every argument check and stops at the missing device, which shows
the overlap alone was refused.  The pointers are fake addresses; no call
here reaches a kernel, and the moved-away calls run only where no GPU is
visible."""
import pytest

import fufft_amd as ff

A = 1 << 32                 # fake, 16-byte aligned device addresses, never dereferenced
MUL, NONE = 0, 2
V16, AUTO = 0, 2
DR, LANE = 0, 1
SPECTRUM, TAPS = 0, 1
FWD = -1

AWAY = 1 << 40              # moves the overlapping pointer clear of every other buffer
N = 4096
D = N * 8                   # bytes of one complex transform


def cases():
    L = ff.lib
    hw = 512 * 512
    return {
        # 1D fused conv: out reaching into the next transform of in, out over the filter
        "conv out into in": lambda o: L.fufft_conv_f32(A, A + 4 * D, 0, A + D + o, N, 2, MUL, V16, DR, None),
        "conv out over filter": lambda o: L.fufft_conv_f32(A, A + 2 * D + 16 + o, 0, A + 2 * D, N, 2, MUL, V16, DR, None),
        "conv out over per-signal filter": lambda o: L.fufft_conv_f32(A, A + 8 * D, N, A + 9 * D + o, N, 2, MUL, V16, LANE,
                                                                    None),
        "timed record over out": lambda o: L.fufft_conv_timed_f32(A, A + 8 * D, 0, A + 2 * D, N, 2, MUL, V16, DR,
                                                                A + 2 * D + 64 + o, 4, None),
        "fwd spectrum into in": lambda o: L.fufft_fwd_f32(A, A + 16 + o, N, 1, V16, None),
        "apply shared spectrum under out": lambda o: L.fufft_apply_f32(A + D + o, 0, A + 8 * D, 0, A, N, 2, MUL, V16, DR,
                                                                    None),
        "apply shared spectrum is out": lambda o: L.fufft_apply_f32(A + o, 0, A + 8 * D, 0, A, N, 2, MUL, V16, DR, None),
        "apply out over filter": lambda o: L.fufft_apply_f32(A, N, A + 8 * D, 0, A + 8 * D - 16 + o, N, 1, MUL, V16, DR,
                                                          None),
        "r2 u is v": lambda o: L.fufft_conv_r2_f32(A, A + D, A + 8 * D, 0, A + 2 * D, A + 2 * D + o, N, 1, V16, DR, None),
        "r2 u into x": lambda o: L.fufft_conv_r2_f32(A, A + D, A + 8 * D, 0, A + 16 + o, A + 2 * D, N, 1, V16, DR, None),
        "r2 v over filter": lambda o: L.fufft_conv_r2_f32(A, A + D, A + 8 * D, 0, A + 2 * D, A + 8 * D + o, N, 1, V16, DR,
                                                       None),
        "c2c out into in": lambda o: L.fufft_c2c_f32(A, A + 16 + o, N, 1, FWD, V16, None),
        "device planner out into taps": lambda o: L.fufft_plan_filter_device_f32(A, A + 16 + o, N, 1, V16, DR, TAPS, 1,
                                                                             None),
        # BFP: words and exponents of the two sides
        "bfp words into words": lambda o: L.fufft_conv_bfp16(A, A + 8 * D, A + 9 * D, 0, A + 4 + o, A + 10 * D, N, 2, 64,
                                                         MUL, V16, DR, None),
        "bfp exponents over words": lambda o: L.fufft_conv_bfp16(A, A + 8 * D, A + 9 * D, 0, A + 2 * D, A + 2 * D + 8 + o,
                                                             N, 2, 64, MUL, V16, DR, None),
        "bfp exponents into exponents": lambda o: L.fufft_conv_bfp16(A, A + 8 * D, A + 9 * D, 0, A + 2 * D,
                                                                 A + 8 * D + 4 + o, N, 2, 64, MUL, V16, DR, None),
        "bfp words over filter": lambda o: L.fufft_conv_bfp16(A, A + 8 * D, A + 9 * D, 0, A + 9 * D + o, A + 10 * D, N, 1,
                                                          64, MUL, V16, DR, None),
        "scaled bfp scales into scales": lambda o: L.fufft_conv_bfp16_scaled(A, A + 8 * D, A + 9 * D, A + 10 * D, 0,
                                                                         A + 2 * D, A + 8 * D + 4 + o, N, 2, MUL, V16,
                                                                         DR, None),
        "scaled bfp words over filter scale": lambda o: L.fufft_conv_bfp16_scaled(A, A + 8 * D, A + 9 * D,
                                                                              A + 10 * D, 0, A + 10 * D + o,
                                                                              A + 11 * D, N, 1, MUL, V16, DR, None),
        "stream out into in": lambda o: L.fufft_stream_f32(A, A + 16 + o, 4096, 1, None),
        "stream shape out into in": lambda o: L.fufft_stream_shape_f32(A, A + 16 + o, 4096, 256, 16, 8, 1, 0, 0, 0, None),
        # four-step and 2D (several launches: whole arrays coincide or are apart)
        "four-step filter inside the data": lambda o: L.fufft_conv_large_f32(A, A + 32768 * 8 + o, 0, 32768, 2, MUL, V16,
                                                                          None),
        "four-step planner out into taps": lambda o: L.fufft_plan_filter_large_device_f32(A, A + 16 + o, 32768, 1, V16,
                                                                                       TAPS, 1, None),
        "2d planner out into taps": lambda o: L.fufft_plan_filter2d_device_f32(A, A + 16 + o, 512, 512, 1, DR, TAPS, 1,
                                                                           None),
        "2d out into in": lambda o: L.fufft_conv2d_f32(A, A + 8 * hw * 8, 0, A + hw * 8 + o, 512, 512, 2, MUL, DR, None),
        "2d out over filter": lambda o: L.fufft_conv2d_f32(A, A + 8 * hw * 8, 0, A + 8 * hw * 8 - 16 + o, 512, 512, 1,
                                                         MUL, DR, None),
        "2d r2 workspace over x": lambda o: L.fufft_conv2d_r2_f32(A, A + 8 * hw * 8, A + 16 * hw * 8, 0,
                                                               A + 17 * hw * 8, A + 18 * hw * 8, A + hw * 2 + o,
                                                               512, 512, 1, DR, None),
        "2d r2 u is v": lambda o: L.fufft_conv2d_r2_f32(A, A + 8 * hw * 8, A + 16 * hw * 8, 0, A + 17 * hw * 8,
                                                     A + 17 * hw * 8 + o, A + 20 * hw * 8, 512, 512, 1, DR, None),
        "2d r2 no-alloc u into y": lambda o: L.fufft_conv2d_r2_noalloc_f32(A, A + 8 * hw * 8, A + 16 * hw * 8, 0,
                                                                        A + 8 * hw * 8 + 64 + o, A + 18 * hw * 8,
                                                                        512, 512, 1, DR, None),
        "2d fwd spectrum into in": lambda o: L.fufft_fwd2d_f32(A, A + 16 + o, 512, 512, 1, None),
        "2d apply shared spectrum under out": lambda o: L.fufft_apply2d_f32(A + hw * 8 + o, 0, A + 8 * hw * 8, 0, A,
                                                                          512, 512, 2, MUL, DR, None),
        "2d apply out over filter": lambda o: L.fufft_apply2d_f32(A, hw, A + 8 * hw * 8, 0, A + 8 * hw * 8 - 16 + o,
                                                                512, 512, 1, MUL, DR, None),
    }


@pytest.mark.parametrize("name", sorted(cases()))
def test_partial_overlap_is_rejected(name):
    assert cases()[name](0) == ff.ERR_INVALID, name


def _no_gpu_visible() -> bool:
    import torch
    return torch.cuda.device_count() == 0     # counts devices without initialising one


@pytest.mark.parametrize("name", sorted(cases()))
def test_the_same_call_apart_passes_the_checks(name):
    if not _no_gpu_visible():
        pytest.skip("the call would launch on fake addresses where a GPU is visible")
    # every argument check passed; the first device call finds no GPU
    assert cases()[name](AWAY) == ff.ERR_HIP, name


def test_every_device_entry_point_is_covered():
    """Each entry point that takes device buffers has at least one case."""
    text = " ".join(cases()[k].__code__.co_names.__repr__() for k in cases())
    for fn in ("fufft_conv_f32", "fufft_conv_timed_f32", "fufft_fwd_f32", "fufft_apply_f32", "fufft_conv_r2_f32",
               "fufft_c2c_f32", "fufft_plan_filter_device_f32", "fufft_conv_bfp16", "fufft_conv_bfp16_scaled",
               "fufft_stream_f32", "fufft_stream_shape_f32", "fufft_conv_large_f32",
               "fufft_plan_filter_large_device_f32", "fufft_plan_filter2d_device_f32", "fufft_conv2d_f32",
               "fufft_conv2d_r2_f32", "fufft_conv2d_r2_noalloc_f32", "fufft_fwd2d_f32", "fufft_apply2d_f32"):
        assert fn in text, fn
