"""CPU tests of the Python binding's argument checks (no GPU needed).

Every launch wrapper checks its tensors -- type, dtype, contiguity, size
against what n, batch and the strides imply, then device -- before the call
reaches the library.  The library is replaced by a stub that fails the test
if any entry point is called, so each rejection below is shown to happen in
Python, before any GPU call.  Also checked: every variant default is "auto",
so a filter planned with the defaults matches a launch with the defaults.
"""
import inspect

import numpy as np
import pytest

torch = pytest.importorskip("torch")


class _NoCalls:
    """Stands in for the library: any call is a test failure."""

    def __getattr__(self, name):
        def fail(*args, **kwargs):
            raise AssertionError(f"{name} was called: the binding did not reject its arguments")
        return fail


@pytest.fixture
def ff(monkeypatch):
    import fufft_amd
    monkeypatch.setattr(fufft_amd, "lib", _NoCalls())
    return fufft_amd


def c64(n):
    return torch.zeros(n, dtype=torch.complex64)


def test_host_arrays_are_refused(ff):
    n, b = 4096, 2
    with pytest.raises(TypeError, match="torch tensor"):
        ff.conv(np.zeros(n * b, np.complex64), c64(n), c64(n * b), n=n, batch=b)
    with pytest.raises(TypeError, match="torch tensor"):
        ff.conv2d_r2(12345, torch.zeros(512 * 512), c64(512 * 512),
                     torch.zeros(512 * 512), torch.zeros(512 * 512), c64(512 * 512), 512, 512, 1)


def test_every_argument_is_checked_before_any_device_check(ff):
    """Shapes of all arguments are checked before any device: on a machine
    without a GPU a bad later argument still names itself."""
    n, b = 4096, 2
    with pytest.raises(TypeError, match="filt"):
        ff.conv(c64(n * b), None, c64(n * b), n=n, batch=b)           # a filter is read for "mul"
    with pytest.raises(TypeError, match="work"):
        ff.conv2d_r2(torch.zeros(512 * 512), torch.zeros(512 * 512), c64(512 * 512),
                     torch.zeros(512 * 512), torch.zeros(512 * 512), 12345, 512, 512, 1)
    with pytest.raises(ValueError, match="not in GPU memory"):         # no filter read for "none"
        ff.conv(c64(n * b), None, c64(n * b), n=n, batch=b, mid="none")


def test_wrong_dtype(ff):
    n, b = 4096, 2
    with pytest.raises(ValueError, match="dtype"):
        ff.conv(torch.zeros(n * b, dtype=torch.complex128), c64(n), c64(n * b), n=n, batch=b)
    with pytest.raises(ValueError, match="dtype"):
        ff.conv_r2(c64(n), torch.zeros(n), c64(n), torch.zeros(n), torch.zeros(n), n=n, batch=1)
    with pytest.raises(ValueError, match="dtype"):
        ff.conv_bfp16(torch.zeros(2 * n, dtype=torch.int16), torch.zeros(n // 64, dtype=torch.int32),
                      c64(n), torch.zeros(2 * n, dtype=torch.int16), torch.zeros(n // 64, dtype=torch.int8),
                      n=n, batch=1)


def test_not_contiguous(ff):
    n, b = 4096, 2
    x = torch.zeros(2 * n * b, dtype=torch.complex64)[::2]
    with pytest.raises(ValueError, match="contiguous"):
        ff.conv(x, c64(n), c64(n * b), n=n, batch=b)


@pytest.mark.parametrize("case", ["in", "out", "filt_shared", "filt_per_signal"])
def test_short_buffers(ff, case):
    n, b = 4096, 4
    sizes = {"in": n * b, "out": n * b, "filt_shared": n, "filt_per_signal": n * b}
    short = dict(sizes)
    short[case] -= 1
    stride = n if case == "filt_per_signal" else 0
    filt = c64(short["filt_per_signal"] if case == "filt_per_signal" else short["filt_shared"])
    with pytest.raises(ValueError, match="holds"):
        ff.conv(c64(short["in"]), filt, c64(short["out"]), n=n, batch=b, filt_stride=stride)


def test_short_buffers_other_paths(ff):
    n, b = 4096, 3
    with pytest.raises(ValueError, match="holds"):            # apply: one spectrum per item
        ff.apply(c64(n), c64(n), c64(n * b), n=n, batch=b, spec_stride=n)
    with pytest.raises(ValueError, match="holds"):            # BFP exponents: n / block per signal
        ff.conv_bfp16(torch.zeros(2 * n * b, dtype=torch.int16), torch.zeros(n * b // 64 - 1, dtype=torch.int8),
                      c64(n), torch.zeros(2 * n * b, dtype=torch.int16),
                      torch.zeros(n * b // 64, dtype=torch.int8), n=n, batch=b)
    with pytest.raises(ValueError, match="holds"):            # four-step buffer
        ff.conv_large(c64(32768 * b - 1), c64(32768), n=32768, batch=b)
    h = w = 512
    with pytest.raises(ValueError, match="holds"):            # 2D two-for-one work array
        ff.conv2d_r2(torch.zeros(h * w * b), torch.zeros(h * w * b), c64(h * w), torch.zeros(h * w * b),
                     torch.zeros(h * w * b), c64(h * w * b - 1), h, w, b)
    with pytest.raises(ValueError, match="holds"):            # C2C output
        ff.c2c(c64(n * b), c64(n * b - 8), n=n, batch=b)
    with pytest.raises(ValueError, match="holds"):            # phase-timer records
        ff.conv_timed(c64(n), c64(n), c64(n), torch.zeros(11, dtype=torch.int32), n=n, batch=1,
                      timing_groups=1)


def test_bad_stride(ff):
    n = 4096
    with pytest.raises(ValueError, match="stride"):
        ff.conv(c64(n), c64(n), c64(n), n=n, batch=1, filt_stride=17)


def test_host_tensor_of_the_right_shape_is_refused(ff):
    """Everything right except the device: still rejected before the call."""
    n, b = 4096, 2
    with pytest.raises(ValueError, match="not in GPU memory"):
        ff.conv(c64(n * b), c64(n), c64(n * b), n=n, batch=b)
    with pytest.raises(ValueError, match="not in GPU memory"):
        ff.conv2d(c64(512 * 512), c64(512 * 512), c64(512 * 512), 512, 512, 1)


def test_variant_defaults_are_auto():
    import fufft_amd
    for name in ("supported", "plan_radices", "plan_chains", "digit_order", "plan_filter", "conv",
                 "conv_timed", "fwd", "apply", "conv_r2", "conv_bfp16", "c2c", "plan_filter_device",
                 "transforms_per_workgroup"):
        p = inspect.signature(getattr(fufft_amd, name)).parameters
        assert p["variant"].default == "auto", name
    # 2D planners and launches share one default column order
    for name in ("plan_filter2d", "plan_filter2d_device", "conv2d", "conv2d_r2", "apply2d"):
        assert inspect.signature(getattr(fufft_amd, name)).parameters["layout"].default == "dr", name


def test_host_bfp_codecs_check_their_arrays(ff):
    """The host dequantisers refuse words that are not int16, exponents that
    are not int8, and too few exponents or scales, before the library reads
    past a host array."""
    n = 64
    q = np.zeros(2 * n * 2, dtype=np.int16)
    with pytest.raises(TypeError, match="int16"):
        ff.bfp_dequantize(q.astype(np.int32), np.zeros(2, dtype=np.int8), block=64)
    with pytest.raises(TypeError, match="int8"):
        ff.bfp_dequantize(q, np.zeros(2, dtype=np.int32), block=64)
    with pytest.raises(ValueError, match="exponents"):
        ff.bfp_dequantize(q, np.zeros(1, dtype=np.int8), block=64)
    with pytest.raises(ValueError, match="whole blocks"):
        ff.bfp_dequantize(q[:-2], np.zeros(2, dtype=np.int8), block=64)
    with pytest.raises(TypeError, match="int16"):
        ff.bfp_scaled_dequantize(q.astype(np.int32), np.ones(2, dtype=np.float32), n)
    with pytest.raises(ValueError, match="scales"):
        ff.bfp_scaled_dequantize(q, np.ones(1, dtype=np.float32), n)
    with pytest.raises(ValueError, match="whole transforms"):
        ff.bfp_scaled_dequantize(q[:-2], np.ones(2, dtype=np.float32), n)
