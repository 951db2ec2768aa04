"""GPU tests of the in-kernel phase timer (fufft_conv_timed_f32).

The timed launch must compute exactly what fufft_conv_f32 computes (the marks
only add waits and barriers), and every record must be well formed: five
phases in order, non-decreasing marks, an XCD id the part has.
"""
import numpy as np
import pytest

from conftest import bits_equal, crandn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("variant,n,batch", [("r8", 4096, 256), ("v16", 1024, 300), ("v16", 256, 1000),
                                             ("r8", 512, 77)])
@pytest.mark.parametrize("mid", ["mul", "conj"])
def test_timed_conv_bit_identical_and_records(dev, variant, n, batch, mid, rng):
    import torch
    import fufft_amd as ff
    print(f"case timed variant={variant} n={n} batch={batch} mid={mid}", flush=True)
    a = torch.from_numpy(crandn(rng, (batch, n))).to(dev)
    spec = crandn(rng, n) / n
    filt = torch.from_numpy(spec[ff.digit_order(n, variant)]).to(dev)
    want, got = torch.empty_like(a), torch.empty_like(a)
    ff.conv(a, filt, want, n=n, batch=batch, mid=mid, variant=variant)
    tpw = ff.transforms_per_workgroup(n, variant)
    groups = -(-batch // tpw)
    timing = torch.zeros(groups * ff.TIMER_STRIDE, dtype=torch.int32, device=dev)
    ff.conv_timed(a, filt, got, timing, n=n, batch=batch, timing_groups=groups, mid=mid, variant=variant)
    torch.cuda.synchronize()
    assert bits_equal(got.cpu().numpy(), want.cpu().numpy())
    rec = ff.decode_timing(timing.cpu().numpy().view(np.uint32))
    marks = rec["marks"]
    assert marks.shape == (groups, 5)
    assert np.all(np.diff(marks, axis=1) >= 0)
    assert np.all(marks[:, -1] > 0)
    assert np.all(rec["xcd"] < 8)


def test_timed_conv_fewer_records_than_workgroups(dev, rng):
    import torch
    import fufft_amd as ff
    n, batch = 4096, 64
    print("case timed partial records", flush=True)
    a = torch.from_numpy(crandn(rng, (batch, n))).to(dev)
    filt = torch.from_numpy(crandn(rng, n) / n).to(dev)
    out = torch.empty_like(a)
    timing = torch.full((16 * ff.TIMER_STRIDE,), -1, dtype=torch.int32, device=dev)
    ff.conv_timed(a, filt, out, timing, n=n, batch=batch, timing_groups=8, variant="auto")
    w = timing.cpu().numpy().view(np.uint32).reshape(16, ff.TIMER_STRIDE)
    assert np.all(w[:8, 2] == 5)
    assert np.all(w[8:] == 0xFFFFFFFF)                 # records past timing_groups untouched
    with pytest.raises(TypeError):                     # records asked for, no buffer given
        ff.conv_timed(a, filt, out, None, n=n, batch=batch, timing_groups=4)
