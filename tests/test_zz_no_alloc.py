"""fufft_conv2d_r2_noalloc_f32: the two-for-one 2D conv without a workspace.

Called through the C ABI (ctypes, device pointers of torch tensors), its
output is compared bit for bit with fufft_conv2d_r2_f32 (the same conv with a
caller workspace) on two calls in a row, the second smaller than the first,
so the second reuses the static scratch the first left behind.  The first
call spans two sub-batches of the scratch (40 images of 512 x 512 against
FUFFT_SCRATCH_BYTES / 2 MiB = 32 per sub-batch).  Also: an image larger than
the scratch is refused with FUFFT_ERR_SCRATCH, and a repeated call leaves the
device's free memory unchanged.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _filter(ff, rng, h, w, layout):
    taps = rng.uniform(0, 1, h * w).astype(np.float32).astype(np.complex64)
    return ff.plan_filter2d(taps, h, w, kind=ff.FILTER_TAPS, layout=layout)


def _case(torch, ff, dev, rng, h, w, batch, layout):
    x = torch.from_numpy(rng.uniform(0, 1, batch * h * w).astype(np.float32)).to(dev)
    y = torch.from_numpy(rng.uniform(0, 1, batch * h * w).astype(np.float32)).to(dev)
    f = torch.from_numpy(_filter(ff, rng, h, w, layout)).to(dev)
    return x, y, f


def _noalloc(ff, x, y, f, u, v, h, w, batch, layout):
    """the new entry point, called through the C ABI"""
    return ff.lib.fufft_conv2d_r2_noalloc_f32(x.data_ptr(), y.data_ptr(), f.data_ptr(), 0, u.data_ptr(),
                                              v.data_ptr(), h, w, batch, ff.LAYOUT[layout], None)


def _with_work(ff, x, y, f, u, v, work, h, w, batch, layout):
    return ff.lib.fufft_conv2d_r2_f32(x.data_ptr(), y.data_ptr(), f.data_ptr(), 0, u.data_ptr(), v.data_ptr(),
                                      work.data_ptr(), h, w, batch, ff.LAYOUT[layout], None)


def _bits(t):
    return t.cpu().numpy().view(np.uint32)


def test_noalloc_equals_workspace_call_twice(dev):
    import torch
    import fufft_amd as ff
    rng = np.random.default_rng(2024)
    for h, w, batch, layout in ((512, 512, 40, "lane"), (256, 512, 3, "dr")):
        print(f"case no-alloc r2 {h}x{w} batch={batch} layout={layout}", flush=True)
        if batch == 40:                                 # more images than one scratch sub-batch holds
            assert batch * h * w * 8 > ff.SCRATCH_BYTES
        x, y, f = _case(torch, ff, dev, rng, h, w, batch, layout)
        u0, v0 = torch.empty_like(x), torch.empty_like(y)
        u1, v1 = torch.full_like(x, float("nan")), torch.full_like(y, float("nan"))
        work = torch.empty(batch * h * w, dtype=torch.complex64, device=dev)
        assert _with_work(ff, x, y, f, u0, v0, work, h, w, batch, layout) == ff.OK
        assert _noalloc(ff, x, y, f, u1, v1, h, w, batch, layout) == ff.OK
        torch.cuda.synchronize()
        assert np.array_equal(_bits(u1), _bits(u0))
        assert np.array_equal(_bits(v1), _bits(v0))
        del work


def test_noalloc_refuses_images_beyond_the_scratch(dev):
    import torch
    import fufft_amd as ff
    h, w = 2048, 8192                                   # 128 MiB of packed points > 64 MiB
    assert h * w * 8 > ff.SCRATCH_BYTES
    t = torch.zeros(16, dtype=torch.float32, device=dev)
    c = torch.zeros(16, dtype=torch.complex64, device=dev)
    st = ff.lib.fufft_conv2d_r2_noalloc_f32(t.data_ptr(), t.data_ptr(), c.data_ptr(), 0, t.data_ptr(),
                                            t.data_ptr(), h, w, 1, ff.LAYOUT["lane"], None)
    assert st == ff.ERR_SCRATCH
    assert "scratch" in ff.lib.fufft_status_string(st).decode()


def test_noalloc_leaves_free_memory_unchanged(dev):
    import torch
    import fufft_amd as ff
    rng = np.random.default_rng(7)
    h, w, batch = 512, 512, 36
    x, y, f = _case(torch, ff, dev, rng, h, w, batch, "lane")
    u, v = torch.empty_like(x), torch.empty_like(y)
    assert _noalloc(ff, x, y, f, u, v, h, w, batch, "lane") == ff.OK   # kernels loaded, nothing pending
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    assert _noalloc(ff, x, y, f, u, v, h, w, batch, "lane") == ff.OK
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0
