"""Arrays beyond 4 GiB: the kernels address one transform (or image) with
32-bit byte offsets from a 64-bit base, and the entry points split a launch
whose per-transform filter array exceeds 4 GiB into chunks of transforms.
Every case here has its signal and its per-signal (per-image) filter array
above 4 GiB, so those base computations and the chunking run; sampled
transforms from both sides of every chunk boundary are bit-identical to the
CPU oracle.  Data are generated on the device; only samples travel.
"""
import numpy as np
import pytest

from conftest import bits_equal, cols_to_dr
from oracle import oracle as O

pytestmark = pytest.mark.gpu

GIB4 = 1 << 32


def sample_rows(batch, chunk):
    """indices around the start, the chunk boundaries and the end"""
    idx = {0, 1, batch - 2, batch - 1}
    for b in range(chunk, batch, chunk):
        idx |= {b - 1, b}
    return sorted(i for i in idx if 0 <= i < batch)


def chunk_len(n):
    """transforms per chunk of the entry points (capi.hip: 4 GiB of filter, multiple of 256)"""
    return ((GIB4 - 1) // (n * 8)) & ~255


def test_conv_f32_per_signal_filters_beyond_4gib(dev):
    import torch
    import fufft_amd as ff
    n = 4096
    batch = GIB4 // (n * 8) + 3                     # 4 GiB + 96 KiB per array
    gen = torch.Generator(device=dev)
    gen.manual_seed(41)
    x = torch.randn(batch * n, dtype=torch.complex64, device=dev, generator=gen)
    f = (torch.randn(batch * n, dtype=torch.complex64, device=dev, generator=gen) / n)
    out = torch.empty_like(x)
    assert x.numel() * 8 > GIB4 and f.numel() * 8 > GIB4
    idx = sample_rows(batch, chunk_len(n))
    print(f"case f32 conv beyond 4 GiB n={n} batch={batch} samples={idx}", flush=True)
    ff.conv(x, f, out, n=n, batch=batch, filt_stride=n, variant="auto")
    torch.cuda.synchronize()
    ti = torch.tensor(idx, device=dev)
    a_s = x.view(batch, n)[ti].cpu().numpy()
    f_s = f.view(batch, n)[ti].cpu().numpy()
    got = out.view(batch, n)[ti].cpu().numpy()
    v = 8 if ff.resolve_variant(n, "auto") == "r8" else 16
    want = O.conv(a_s, f_s, n, O.kernel_plan(n, v), filt_stride=n).reshape(len(idx), n)
    assert bits_equal(got, want)
    del x, f, out


def test_conv_bfp16_per_signal_filters_beyond_4gib(dev):
    import torch
    import fufft_amd as ff
    n = 4096
    batch = GIB4 // (n * 8) + 3                     # filter array 4 GiB + 96 KiB
    gen = torch.Generator(device=dev)
    gen.manual_seed(43)
    q = torch.randint(-32767, 32768, (2 * batch * n,), dtype=torch.int16, device=dev, generator=gen)
    e = torch.randint(-30, 10, (batch * n // 64,), dtype=torch.int8, device=dev, generator=gen)
    f = (torch.randn(batch * n, dtype=torch.complex64, device=dev, generator=gen) / n)
    qo, eo = torch.empty_like(q), torch.empty_like(e)
    idx = sample_rows(batch, chunk_len(n))
    print(f"case bfp conv beyond 4 GiB of filters n={n} batch={batch} samples={idx}", flush=True)
    ff.conv_bfp16(q, e, f, qo, eo, n=n, batch=batch, filt_stride=n)
    torch.cuda.synchronize()
    ti = torch.tensor(idx, device=dev)
    q_s = q.view(batch, 2 * n)[ti].cpu().numpy()
    e_s = e.view(batch, n // 64)[ti].cpu().numpy()
    f_s = f.view(batch, n)[ti].cpu().numpy()
    v = 8 if ff.resolve_variant(n, "auto") == "r8" else 16
    oq, oe = O.bfp_conv(q_s, e_s, f_s, n, O.kernel_plan(n, v), filt_stride=n)
    assert np.array_equal(eo.view(batch, n // 64)[ti].cpu().numpy(), oe.reshape(len(idx), -1))
    assert np.array_equal(qo.view(batch, 2 * n)[ti].cpu().numpy(), oq.reshape(len(idx), -1))
    del q, e, f, qo, eo


def test_conv_large_per_signal_filters_beyond_4gib(dev):
    import torch
    import fufft_amd as ff
    n = 32768
    batch = GIB4 // (n * 8) + 1                     # 4 GiB + 256 KiB per array
    gen = torch.Generator(device=dev)
    gen.manual_seed(47)
    x = torch.randn(batch * n, dtype=torch.complex64, device=dev, generator=gen)
    f = (torch.randn(batch * n, dtype=torch.complex64, device=dev, generator=gen) / n)
    idx = [0, 1, batch // 2, batch - 2, batch - 1]
    ti = torch.tensor(idx, device=dev)
    a_s = x.view(batch, n)[ti].cpu().numpy()
    f_s = f.view(batch, n)[ti].cpu().numpy()
    print(f"case four-step beyond 4 GiB n={n} batch={batch} samples={idx}", flush=True)
    ff.conv_large(x, f, n=n, batch=batch, filt_stride=n)
    torch.cuda.synchronize()
    lout, mid = ff.large_plan(n)
    want = O.conv(a_s, f_s, n, O.large_plan(lout, mid, ff.large_middle("auto")), filt_stride=n).reshape(len(idx), n)
    assert bits_equal(x.view(batch, n)[ti].cpu().numpy(), want)
    del x, f


def test_conv2d_per_image_filters_beyond_4gib(dev):
    import torch
    import fufft_amd as ff
    h = w = 512
    np_img = h * w
    batch = GIB4 // (np_img * 8) + 1                # 4 GiB + 2 MiB per array
    gen = torch.Generator(device=dev)
    gen.manual_seed(53)
    x = torch.randn(batch * np_img, dtype=torch.complex64, device=dev, generator=gen)
    f = (torch.randn(batch * np_img, dtype=torch.complex64, device=dev, generator=gen) / np_img)
    out = torch.empty_like(x)
    idx = [0, batch // 2, batch - 1]
    print(f"case conv2d beyond 4 GiB {h}x{w} batch={batch} samples={idx}", flush=True)
    ff.conv2d(x, f, out, h, w, batch=batch, filt_stride=np_img, layout="lane")
    torch.cuda.synchronize()
    ti = torch.tensor(idx, device=dev)
    a_s = x.view(batch, np_img)[ti].cpu().numpy()
    f_s = f.view(batch, np_img)[ti].cpu().numpy()
    got = out.view(batch, np_img)[ti].cpu().numpy()
    vr, vc = ff.plan2d(h, w)                        # values per lane: row plan, column plan
    ph, pw = O.kernel_plan(h, vc), O.kernel_plan(w, vr)
    want = O.conv2d(a_s, cols_to_dr(f_s, h, w), h, w, ph, pw, filt_stride=np_img)
    assert bits_equal(got.reshape(-1), want.reshape(-1))
    del x, f, out
