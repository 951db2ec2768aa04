"""The C ABI on explicit streams and inside HIP graphs.

- Two conv calls issued on two different streams at once compute exactly what
  they compute one after the other (the calls are stateless).
- Four host threads on four streams call four entry points concurrently, with
  the same results.
- fufft_conv_f32 (N = 4096 and the single-launch N = 32768), the four-step
  chain, the 2D conv and both BFP formats captured in a graph
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
    """capture run() (writing out, a tensor or a tuple of them), replay reps
    times with eager work between replays, every replay equal to the eager
    result"""
    import torch
    outs = out if isinstance(out, tuple) else (out,)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run(s)                                     # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    want = [o.clone() for o in outs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        run(s)
    for i in range(reps):
        for o in outs:
            o.zero_()
        scratch = torch.randn(1 << 20, device=outs[0].device)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, w in zip(outs, want):
            if o.is_floating_point() or o.is_complex():          # bit for bit, not value for value
                o, w = o.view(torch.int32), w.view(torch.int32)
            assert torch.equal(o, w), f"replay {i}"
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


def test_graph_capture_conv_n32768(dev, rng):
    """the single-launch conv at N = 32768 (136 KiB of dynamic LDS) captured and replayed"""
    import torch
    import fufft_amd as ff
    n, batch = 32768, 8
    print("case graph conv n=32768", flush=True)
    a = torch.from_numpy(crandn(rng, (batch, n))).to(dev)
    f = torch.from_numpy(ff.plan_filter(crandn(rng, n), n, "v16", layout="lane", kind=ff.FILTER_TAPS)).to(dev)
    out = torch.empty_like(a)
    _graph_matches_eager(lambda s: ff.conv(a, f, out, n=n, batch=batch, variant="v16", layout="lane", stream=s),
                         out)


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


def test_graph_capture_bfp(dev, rng):
    """both int16-BFP formats captured and replayed: 64-point blocks, whole-
    signal blocks (the LDS rendezvous of the block maxima) and the reference's
    fp32-scale format with its int16 filter"""
    import torch
    import fufft_amd as ff
    n, batch = 4096, 64
    x = crandn(rng, (batch, n))
    taps = crandn(rng, n)
    f = torch.from_numpy(ff.plan_filter(taps, n, "v16", layout="lane", kind=ff.FILTER_TAPS)).to(dev)
    for block in (64, n):
        print(f"case graph bfp block={block}", flush=True)
        q, e = ff.bfp_quantize(x, block=block)
        dq, de = torch.from_numpy(q).to(dev), torch.from_numpy(e).to(dev)
        qo, eo = torch.empty_like(dq), torch.empty_like(de)
        _graph_matches_eager(lambda s: ff.conv_bfp16(dq, de, f, qo, eo, n=n, batch=batch, variant="v16",
                                                     layout="lane", stream=s, block=block), (qo, eo))
    print("case graph bfp scaled", flush=True)
    q, sc = ff.bfp_scaled_quantize(x, n)
    fq, fs = ff.bfp_scaled_quantize(ff.plan_filter(taps, n, variant="v16", kind=ff.FILTER_TAPS), n)
    dq, ds = torch.from_numpy(q).to(dev), torch.from_numpy(sc).to(dev)
    dfq, dfs = torch.from_numpy(fq).to(dev), torch.from_numpy(fs).to(dev)
    qo, so = torch.empty_like(dq), torch.empty_like(ds)
    _graph_matches_eager(lambda s: ff.conv_bfp16_scaled(dq, ds, dfq, dfs, qo, so, n=n, batch=batch,
                                                        variant="v16", stream=s), (qo, so))


def test_host_threads_call_concurrently(dev, rng):
    """Four host threads, each on its own stream, call different entry points
    at the same time (ctypes releases the GIL, so the library is entered
    concurrently, including first-use paths such as the dynamic-LDS
    attribute); every result equals the one computed alone beforehand."""
    import threading
    import torch
    import fufft_amd as ff
    n1, b1 = 8192, 512                                  # fp32 conv, radix 16
    x1 = torch.from_numpy(crandn(rng, (b1, n1))).to(dev)
    f1 = torch.from_numpy(ff.plan_filter(crandn(rng, n1), n1, "auto", kind=ff.FILTER_TAPS)).to(dev)
    nq, bq = 2048, 512                                  # BFP, 256-point blocks
    q, e = ff.bfp_quantize(crandn(rng, bq * nq), block=256)
    dq, de = torch.from_numpy(q).to(dev), torch.from_numpy(e).to(dev)
    fq = torch.from_numpy(ff.plan_filter(crandn(rng, nq), nq, "auto", kind=ff.FILTER_TAPS)).to(dev)
    nl, bl = 65536, 8                                   # four-step
    xl = torch.from_numpy(crandn(rng, bl * nl)).to(dev)
    fl = torch.from_numpy(ff.plan_filter_large(crandn(rng, nl), nl, kind=ff.FILTER_TAPS)).to(dev)
    h = w = 256                                         # 2D
    x2 = torch.from_numpy(crandn(rng, 6 * h * w)).to(dev)
    f2 = torch.from_numpy(ff.plan_filter2d(crandn(rng, h * w), h, w, kind=ff.FILTER_TAPS)).to(dev)

    def job_conv(out, s):
        ff.conv(x1, f1, out, n=n1, batch=b1, variant="auto", stream=s)

    def job_bfp(out, s):
        ff.conv_bfp16(dq, de, fq, out[0], out[1], n=nq, batch=bq, block=256, stream=s)

    def job_large(out, s):
        out.copy_(xl)                                   # conv_large works in place
        ff.conv_large(out, fl, n=nl, batch=bl, stream=s)

    def job_2d(out, s):
        ff.conv2d(x2, f2, out, h, w, batch=6, stream=s)

    jobs = [(job_conv, lambda: torch.empty_like(x1)),
            (job_bfp, lambda: (torch.empty_like(dq), torch.empty_like(de))),
            (job_large, lambda: torch.empty_like(xl)),
            (job_2d, lambda: torch.empty_like(x2))]
    ref = []
    for job, make in jobs:
        out = make()
        job(out, None)
        ref.append(out)
    torch.cuda.synchronize()
    print("case four host threads", flush=True)
    errors, outs = [], [make() for _, make in jobs]

    def worker(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                if jobs[i][0] is job_large:
                    jobs[i][0](outs[i], s)              # the copy rides on s as well
                else:
                    for _ in range(4):
                        jobs[i][0](outs[i], s)
            s.synchronize()
        except Exception as ex:                         # reported by the main thread
            errors.append(repr(ex))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(jobs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads)
    assert not errors, errors
    torch.cuda.synchronize()
    for i, (r, o) in enumerate(zip(ref, outs)):
        if isinstance(r, tuple):
            assert torch.equal(r[0], o[0]) and torch.equal(r[1], o[1]), i
        else:
            assert torch.equal(r.view(torch.int64), o.view(torch.int64)), i
