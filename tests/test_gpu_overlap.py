"""GPU check of the buffer rules of the C ABI: arrays cut from one allocation
that touch but share no byte give results bit-identical to separate
allocations, in place works where a call allows it, and a partial overlap
raises FufftError (FUFFT_ERR_INVALID) before any launch, leaving every
buffer as it was.  No reference counterpart: the reference's kernels take
`__restrict__` pointers (fufft.cuh:1499-1534)."""
import numpy as np
import pytest

from conftest import bits_equal, crandn, cuniform

pytestmark = pytest.mark.gpu


def _dt(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def test_conv_adjacent_in_place_and_partial(dev):
    import torch
    import fufft_amd as ff
    n, batch = 4096, 6
    rng = np.random.default_rng(5)
    a = crandn(rng, batch * n)
    filt = ff.plan_filter(cuniform(rng, n), n, variant="v16", layout="lane", kind=ff.FILTER_TAPS)
    print(f"case overlap conv n={n} batch={batch}", flush=True)
    ref = torch.empty(batch * n, dtype=torch.complex64, device=dev)
    ff.conv(_dt(a, dev), _dt(filt, dev), ref, n, batch, variant="v16", layout="lane")
    # one allocation: in | out | filter, each touching the next
    pool = torch.empty(2 * batch * n + n, dtype=torch.complex64, device=dev)
    x, y, f = pool[:batch * n], pool[batch * n:2 * batch * n], pool[2 * batch * n:]
    x.copy_(_dt(a, dev))
    f.copy_(_dt(filt, dev))
    ff.conv(x, f, y, n, batch, variant="v16", layout="lane")
    torch.cuda.synchronize()
    assert bits_equal(y.cpu().numpy(), ref.cpu().numpy())
    # out one transform into in, and out over the filter: refused, nothing written
    before = pool.clone()
    with pytest.raises(ff.FufftError):
        ff.conv(pool[:batch * n], f, pool[n:(batch + 1) * n], n, batch, variant="v16", layout="lane")
    with pytest.raises(ff.FufftError):
        ff.conv(x, f, pool[n + batch * n:n + 2 * batch * n], n, batch, variant="v16", layout="lane")
    torch.cuda.synchronize()
    assert torch.equal(pool.view(torch.int32), before.view(torch.int32))
    # in place
    ff.conv(x, f, x, n, batch, variant="v16", layout="lane")
    torch.cuda.synchronize()
    assert bits_equal(x.cpu().numpy(), ref.cpu().numpy())


def test_apply_shared_spectrum_next_to_out(dev):
    import torch
    import fufft_amd as ff
    n, batch = 1024, 5
    rng = np.random.default_rng(6)
    a = cuniform(rng, n)
    filt = np.concatenate([ff.plan_filter(crandn(rng, n, 1.0 / n), n, fold_inv_n=False) for _ in range(batch)])
    spec = torch.empty(n, dtype=torch.complex64, device=dev)
    ff.fwd(_dt(a, dev), spec, n, 1)
    print(f"case overlap apply n={n} batch={batch}", flush=True)
    ref = torch.empty(batch * n, dtype=torch.complex64, device=dev)
    ff.apply(spec, _dt(filt, dev), ref, n, batch, spec_stride=0, filt_stride=n)
    # spectrum | outputs in one allocation
    pool = torch.empty((batch + 1) * n, dtype=torch.complex64, device=dev)
    pool[:n].copy_(spec)
    ff.apply(pool[:n], _dt(filt, dev), pool[n:], n, batch, spec_stride=0, filt_stride=n)
    torch.cuda.synchronize()
    assert bits_equal(pool[n:].cpu().numpy(), ref.cpu().numpy())
    # outputs starting half a transform before the shared spectrum: refused
    with pytest.raises(ff.FufftError):
        ff.apply(pool[n:2 * n], _dt(filt, dev), pool[n // 2:n // 2 + batch * n], n, batch, spec_stride=0,
                 filt_stride=n)


def test_bfp_exponents_next_to_each_other(dev):
    import torch
    import fufft_amd as ff
    n, batch = 512, 8
    rng = np.random.default_rng(7)
    q, e = ff.bfp_quantize(crandn(rng, batch * n))
    filt = ff.plan_filter(cuniform(rng, n), n, kind=ff.FILTER_TAPS)
    eb = e.size
    print(f"case overlap bfp n={n} batch={batch} exponents={eb}", flush=True)
    qo = torch.empty(q.size, dtype=torch.int16, device=dev)
    eo = torch.empty(eb, dtype=torch.int8, device=dev)
    ff.conv_bfp16(_dt(q, dev), _dt(e, dev), _dt(filt, dev), qo, eo, n=n, batch=batch)
    # in exponents | out exponents in one allocation, the words likewise
    ep = torch.empty(2 * eb, dtype=torch.int8, device=dev)
    qp = torch.empty(2 * q.size, dtype=torch.int16, device=dev)
    ep[:eb].copy_(_dt(e, dev))
    qp[:q.size].copy_(_dt(q, dev))
    ff.conv_bfp16(qp[:q.size], ep[:eb], _dt(filt, dev), qp[q.size:], ep[eb:], n=n, batch=batch)
    torch.cuda.synchronize()
    assert bits_equal(qp[q.size:].cpu().numpy(), qo.cpu().numpy())
    assert np.array_equal(ep[eb:].cpu().numpy(), eo.cpu().numpy())
    # output exponents four blocks into the input exponents: refused
    with pytest.raises(ff.FufftError):
        ff.conv_bfp16(qp[:q.size], ep[:eb], _dt(filt, dev), qp[q.size:], ep[4:4 + eb], n=n, batch=batch)


def test_conv2d_r2_workspace_next_to_outputs(dev):
    import torch
    import fufft_amd as ff
    h = w = 512
    batch = 2
    rb = h * w * batch
    rng = np.random.default_rng(8)
    xs = rng.uniform(0, 1, (2, rb)).astype(np.float32)
    filt = ff.plan_filter2d(rng.uniform(0, 1, h * w).astype(np.complex64), h, w, kind=ff.FILTER_TAPS)
    print(f"case overlap conv2d_r2 {h}x{w} batch={batch}", flush=True)
    u0, v0 = (torch.empty(rb, dtype=torch.float32, device=dev) for _ in range(2))
    work0 = torch.empty(rb, dtype=torch.complex64, device=dev)
    ff.conv2d_r2(_dt(xs[0], dev), _dt(xs[1], dev), _dt(filt, dev), u0, v0, work0, h, w, batch)
    # x | y | u | v | workspace in one float allocation (the workspace 2 * rb floats)
    pool = torch.empty(6 * rb, dtype=torch.float32, device=dev)
    pool[:rb].copy_(_dt(xs[0], dev))
    pool[rb:2 * rb].copy_(_dt(xs[1], dev))
    x, y, u, v = (pool[i * rb:(i + 1) * rb] for i in range(4))
    work = pool[4 * rb:]
    ff.conv2d_r2(x, y, _dt(filt, dev), u, v, work, h, w, batch)
    torch.cuda.synchronize()
    assert bits_equal(u.cpu().numpy(), u0.cpu().numpy())
    assert bits_equal(v.cpu().numpy(), v0.cpu().numpy())
    # the workspace reaching back into v: refused
    with pytest.raises(ff.FufftError):
        ff.conv2d_r2(x, y, _dt(filt, dev), u, v, pool[4 * rb - 64:6 * rb - 64], h, w, batch)
    # in place: u over x, v over y
    ff.conv2d_r2(x, y, _dt(filt, dev), x, y, work, h, w, batch)
    torch.cuda.synchronize()
    assert bits_equal(x.cpu().numpy(), u0.cpu().numpy())
    assert bits_equal(y.cpu().numpy(), v0.cpu().numpy())
