"""The C ABI on explicit streams and inside HIP graphs.

- Two conv calls issued on two different streams at once compute exactly what
  they compute one after the other (the calls are stateless).
- fufft_conv_f32, the four-step chain and the 2D conv captured in a graph
  (torch.cuda.CUDAGraph drives hipStreamBeginCapture) replay bit-identically
  to the eager call, replay after replay, with eager work in between.  None
  of these paths issues a memset or allocates, so they capture as plain
  kernel nodes.
"""
import numpy as np
import pytest

from conftest import crandn

pytestmark = pytest.mark.gpu


def test_two_streams_concurrently(dev, rng):
    import torch
    import fufft_amd as ff
    n, batch = 4096, 2048
    print("case two streams", flush=True)
    a = torch.from_numpy(crandn(rng, (batch, n))).to(dev)
    b = torch.from_numpy(crandn(rng, (batch, n))).to(dev)
    fa = torch.from_numpy(ff.plan_filter(crandn(rng, n), n, "auto", kind=ff.FILTER_TAPS)).to(dev)
    fb = torch.from_numpy(ff.plan_filter(crandn(rng, n), n, "auto", kind=ff.FILTER_TAPS)).to(dev)
    ra, rb = torch.empty_like(a), torch.empty_like(b)
    ff.conv(a, fa, ra, n=n, batch=batch, variant="auto")
    ff.conv(b, fb, rb, n=n, batch=batch, mid="conj", variant="auto")
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    oa, ob = torch.empty_like(a), torch.empty_like(b)
    for _ in range(3):
        ff.conv(a, fa, oa, n=n, batch=batch, variant="auto", stream=s1)
        ff.conv(b, fb, ob, n=n, batch=batch, mid="conj", variant="auto", stream=s2)
    torch.cuda.synchronize()
    assert torch.equal(oa.view(torch.int64), ra.view(torch.int64))
    assert torch.equal(ob.view(torch.int64), rb.view(torch.int64))


def _graph_matches_eager(run, out, reps=3):
    """capture run() (writing out), replay reps times with eager work between
    replays, every replay equal to the eager result"""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run(s)                                     # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    want = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        run(s)
    for i in range(reps):
        out.zero_()
        scratch = torch.randn(1 << 20, device=out.device)      # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), want.view(torch.int32)), f"replay {i}"
        del scratch


def test_graph_capture_conv(dev, rng):
    import torch
    import fufft_amd as ff
    n, batch = 4096, 512
    print("case graph conv", flush=True)
    a = torch.from_numpy(crandn(rng, (batch, n))).to(dev)
    f = torch.from_numpy(ff.plan_filter(crandn(rng, n), n, "auto", kind=ff.FILTER_TAPS)).to(dev)
    out = torch.empty_like(a)
    _graph_matches_eager(lambda s: ff.conv(a, f, out, n=n, batch=batch, variant="auto", stream=s), out)


def test_graph_capture_fourstep_and_2d(dev, rng):
    import torch
    import fufft_amd as ff
    print("case graph four-step", flush=True)
    n, batch = 32768, 8
    x0 = torch.from_numpy(crandn(rng, (batch, n))).to(dev)
    buf = torch.empty_like(x0)
    f = torch.from_numpy(ff.plan_filter_large(crandn(rng, n), n, kind=ff.FILTER_TAPS)).to(dev)

    def large(s):
        buf.copy_(x0)                              # in place: restart from the same input each time
        ff.conv_large(buf, f, n=n, batch=batch, stream=s)
    _graph_matches_eager(large, buf)
    print("case graph 2D", flush=True)
    h = w = 512
    img = torch.from_numpy(crandn(rng, (2, h, w))).to(dev)
    f2 = torch.from_numpy(ff.plan_filter2d(crandn(rng, (h, w)), h, w, kind=ff.FILTER_TAPS)).to(dev)
    out2 = torch.empty_like(img)
    _graph_matches_eager(lambda s: ff.conv2d(img, f2, out2, h, w, batch=2, stream=s), out2)
