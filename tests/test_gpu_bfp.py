"""GPU parity of the int16 block-floating-point fused conv (fufft_conv_bfp16).

Bar: int16 words and int8 exponents bit-identical to the oracle's BFP conv
(same plan, same exponent rule, same block length), and rel L2 <= 1e-4 against the fp64
convolution of the UNquantised input (input quantisation included), on the
BASELINE config-3 style input: per-signal N(0,1) scaled by 10^u, u ~ U[-3, 3].
"""
import numpy as np
import pytest

from conftest import crandn, lane_major
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL_BFP = 1e-4


def to_dev(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def config3_signals(rng, batch, n):
    scale = 10.0 ** rng.uniform(-3, 3, (batch, 1))
    return (crandn(rng, (batch, n)) * scale).astype(np.complex64)


def run_bfp(dev, q, e, filt, n, batch, filt_stride=0, mid="mul", variant="auto", inplace=False,
            block=64):
    import torch
    import fufft_amd as ff
    dq, de, df = to_dev(q, dev), to_dev(e, dev), to_dev(filt, dev)
    qo = dq if inplace else torch.empty_like(dq)
    eo = de if inplace else torch.empty_like(de)
    ff.conv_bfp16(dq, de, df, qo, eo, n=n, batch=batch, filt_stride=filt_stride, mid=mid,
                  variant=variant, block=block)
    torch.cuda.synchronize()
    return qo.cpu().numpy(), eo.cpu().numpy()


@pytest.mark.parametrize("n,variant", [(512, "auto"), (1024, "auto"), (2048, "auto"), (4096, "auto"),
                                       (8192, "auto"), (1024, "v16"), (4096, "v16")])
@pytest.mark.parametrize("mid", ["mul", "conj"])
def test_bfp_conv_matches_oracle_and_fp64(dev, n, variant, mid, rng):
    import fufft_amd as ff
    batch = max(8, 32768 // n)
    x = config3_signals(rng, batch, n)
    q, e = ff.bfp_quantize(x)
    taps = crandn(rng, n)
    v = 8 if ff.resolve_variant(n, variant) == "r8" else 16
    filt = ff.plan_filter(taps, n, variant=variant, kind=ff.FILTER_TAPS)
    print(f"case bfp n={n} variant={variant} mid={mid} batch={batch}", flush=True)
    qo, eo = run_bfp(dev, q, e, filt, n, batch, mid=mid, variant=variant)
    oq, oe = O.bfp_conv(q, e, filt, n, O.kernel_plan(n, v), mid=mid)
    assert np.array_equal(eo, oe)
    assert np.array_equal(qo, oq)
    # accuracy against fp64 on the unquantised input, input quantisation included
    spec = np.fft.fft(taps.astype(np.complex128)) / n
    if mid == "conj":
        spec = np.conj(spec)
    want = np.fft.ifft(np.fft.fft(x.astype(np.complex128), axis=1) * spec[None, :] * n, axis=1)
    got = O.bfp_dequantize(qo, eo).reshape(batch, n)
    rel = np.sqrt(np.sum(np.abs(got - want) ** 2) / np.sum(np.abs(want) ** 2))
    per_signal = np.sqrt(np.sum(np.abs(got - want) ** 2, axis=1) / np.sum(np.abs(want) ** 2, axis=1))
    print(f"   rel L2 {rel:.3e}, worst signal {per_signal.max():.3e}", flush=True)
    assert rel <= TOL_BFP


# blocks longer than 64 points: one LDS atomic max per (wavefront, register)
# pair; T = 64 plans (one wavefront per transform, 4 per workgroup) sync by a
# wavefront fence, wider ones by the workgroup barrier.  block = n is one
# exponent per signal, the reference's per-transform scale.
BLOCKS = [(512, "auto", 128), (512, "auto", 512), (1024, "v16", 1024), (1024, "auto", 256),
          (2048, "auto", 256), (4096, "auto", 128), (4096, "auto", 1024), (4096, "auto", 4096),
          (4096, "v16", 2048), (8192, "auto", 8192), (16384, "v16", 16384)]


@pytest.mark.parametrize("n,variant,block", BLOCKS)
def test_bfp_block_lengths(dev, n, variant, block, rng):
    import fufft_amd as ff
    batch = max(5, 20480 // n) | 1                # odd: a partly filled last workgroup at T = 64
    x = config3_signals(rng, batch, n)
    x[1] = 0                                      # a zero signal: every block e = -128
    x[2, : min(block, n // 2)] = 0                # a zero block (or part of one)
    q, e = ff.bfp_quantize(x, block=block)
    oq0, oe0 = O.bfp_quantize(x, block=block)
    assert np.array_equal(q, oq0) and np.array_equal(e, oe0)
    assert e.size == batch * n // block
    taps = crandn(rng, n)
    v = 8 if ff.resolve_variant(n, variant) == "r8" else 16
    filt = ff.plan_filter(taps, n, variant=variant, kind=ff.FILTER_TAPS)
    print(f"case bfp block={block} n={n} variant={variant} batch={batch}", flush=True)
    qo, eo = run_bfp(dev, q, e, filt, n, batch, variant=variant, block=block, inplace=(block == n))
    oq, oe = O.bfp_conv(q, e, filt, n, O.kernel_plan(n, v), block=block)
    assert np.array_equal(eo, oe)
    assert np.array_equal(qo, oq)
    assert np.all(eo.reshape(batch, -1)[1] == -128) and np.all(qo.reshape(batch, -1)[1] == 0)
    spec = np.fft.fft(taps.astype(np.complex128))
    want = np.fft.ifft(np.fft.fft(x.astype(np.complex128), axis=1) * spec[None, :], axis=1)
    got = O.bfp_dequantize(qo, eo, block=block).reshape(batch, n)
    rel = np.sqrt(np.sum(np.abs(got - want) ** 2) / np.sum(np.abs(want) ** 2))
    print(f"   rel L2 {rel:.3e}", flush=True)
    assert rel <= TOL_BFP


def test_bfp_block_rejects_bad_lengths(dev):
    import fufft_amd as ff
    import torch
    n = 4096
    d = torch.zeros(2 * n, dtype=torch.int16, device=dev)
    de = torch.zeros(n // 32, dtype=torch.int8, device=dev)     # room for 32-point blocks: the library decides
    f = torch.zeros(n, dtype=torch.complex64, device=dev)
    for block in (32, 96, 2 * n):
        with pytest.raises(ff.FufftError):
            ff.conv_bfp16(d, de, f, d, de, n=n, batch=1, block=block)


def test_bfp_zero_blocks_and_in_place(dev, rng):
    import fufft_amd as ff
    n, batch = 4096, 16
    x = config3_signals(rng, batch, n)
    x[3] = 0                                   # a zero signal: every block e = -128
    x[5, :64] = 0                              # one zero input block
    q, e = ff.bfp_quantize(x)
    assert np.all(e.reshape(batch, -1)[3] == -128)
    filt = ff.plan_filter(crandn(rng, n), n, variant="auto", kind=ff.FILTER_TAPS)
    print("case bfp zero blocks in place", flush=True)
    qo, eo = run_bfp(dev, q, e, filt, n, batch, inplace=True)
    oq, oe = O.bfp_conv(q, e, filt, n, O.kernel_plan(n, 8 if ff.resolve_variant(n, "auto") == "r8" else 16))
    assert np.array_equal(eo, oe) and np.array_equal(qo, oq)
    assert np.all(eo.reshape(batch, -1)[3] == -128) and np.all(qo.reshape(batch, -1)[3] == 0)


def test_bfp_per_signal_filter_and_none(dev, rng):
    import fufft_amd as ff
    n, batch = 1024, 64
    x = config3_signals(rng, batch, n)
    q, e = ff.bfp_quantize(x)
    spec = (crandn(rng, (batch, n)) / n).astype(np.complex64)
    plan = O.kernel_plan(n, 8 if ff.resolve_variant(n, "auto") == "r8" else 16)
    fdr = np.ascontiguousarray(spec[:, O.mixedrev(plan)]).reshape(-1)
    print("case bfp per-signal filter", flush=True)
    qo, eo = run_bfp(dev, q, e, fdr, n, batch, filt_stride=n)
    oq, oe = O.bfp_conv(q, e, fdr, n, plan, filt_stride=n)
    assert np.array_equal(eo, oe) and np.array_equal(qo, oq)
    # the round trip (no mid operation) returns N * input through the codec
    qo, eo = run_bfp(dev, q, e, fdr, n, batch, mid="none")
    got = O.bfp_dequantize(qo, eo)
    assert O.rel_l2(got, n * O.bfp_dequantize(q, e)) < 1e-4


@pytest.mark.parametrize("n,variant,block", [(512, "auto", 64), (1024, "auto", 64), (2048, "auto", 64),
                                             (4096, "auto", 64), (8192, "auto", 64), (1024, "v16", 64),
                                             (4096, "v16", 64), (16384, "v16", 64), (512, "auto", 512),
                                             (4096, "auto", 4096), (16384, "v16", 1024)])
def test_bfp_full_batch_every_size(dev, n, variant, block):
    """2^27 points (full occupancy): 16 transforms spread over the batch,
    words and exponents bit-identical to the oracle."""
    import torch
    import fufft_amd as ff
    batch = (1 << 27) // n
    nb = n // block
    gen = torch.Generator(device=dev)
    gen.manual_seed(n + block)
    dq = torch.randint(-32767, 32768, (2 * batch * n,), dtype=torch.int16, device=dev, generator=gen)
    de = torch.randint(-30, 10, (batch * nb,), dtype=torch.int8, device=dev, generator=gen)
    rng = np.random.default_rng(n)
    filt = ff.plan_filter(crandn(rng, n), n, variant=variant, kind=ff.FILTER_TAPS)
    qo, eo = torch.empty_like(dq), torch.empty_like(de)
    print(f"case bfp full-batch n={n} variant={variant} block={block} batch={batch}", flush=True)
    ff.conv_bfp16(dq, de, to_dev(filt, dev), qo, eo, n=n, batch=batch, variant=variant, block=block)
    idx = torch.from_numpy(np.linspace(0, batch - 1, 16).astype(np.int64)).to(dev)
    q_s = dq.view(batch, 2 * n)[idx].cpu().numpy()
    e_s = de.view(batch, nb)[idx].cpu().numpy()
    v = 8 if ff.resolve_variant(n, variant) == "r8" else 16
    oq, oe = O.bfp_conv(q_s, e_s, filt, n, O.kernel_plan(n, v), block=block)
    torch.cuda.synchronize()
    assert np.array_equal(eo.view(batch, nb)[idx].cpu().numpy(), oe.reshape(16, -1))
    assert np.array_equal(qo.view(batch, 2 * n)[idx].cpu().numpy(), oq.reshape(16, -1))
    del dq, de, qo, eo


@pytest.mark.parametrize("n", [512, 1024, 2048, 4096, 8192, 16384])
def test_bfp_full_batch_lane_layout_fastest_variant(dev, n):
    """The bench's BFP plan: the filter planned lane-major at the variant
    fufft_fastest_variant picks for it, 2^27 points, 64-point blocks; 16
    transforms spread over the batch bit-identical to the oracle (which reads
    the same filter in digit order)."""
    import torch
    import fufft_amd as ff
    variant = ff.fastest_variant(n, "lane")
    v = 8 if variant == "r8" else 16
    batch = (1 << 27) // n
    nb = n // 64
    gen = torch.Generator(device=dev)
    gen.manual_seed(3 * n + 1)
    dq = torch.randint(-32767, 32768, (2 * batch * n,), dtype=torch.int16, device=dev, generator=gen)
    de = torch.randint(-30, 10, (batch * nb,), dtype=torch.int8, device=dev, generator=gen)
    rng = np.random.default_rng(3 * n)
    taps = crandn(rng, n)
    fdr = ff.plan_filter(taps, n, variant=variant, kind=ff.FILTER_TAPS)
    flane = ff.plan_filter(taps, n, variant=variant, layout="lane", kind=ff.FILTER_TAPS)
    assert np.array_equal(flane, lane_major(fdr, n, v))
    qo, eo = torch.empty_like(dq), torch.empty_like(de)
    print(f"case bfp full-batch lane n={n} variant={variant} batch={batch}", flush=True)
    ff.conv_bfp16(dq, de, to_dev(flane, dev), qo, eo, n=n, batch=batch, variant=variant, layout="lane")
    idx = torch.from_numpy(np.linspace(0, batch - 1, 16).astype(np.int64)).to(dev)
    q_s = dq.view(batch, 2 * n)[idx].cpu().numpy()
    e_s = de.view(batch, nb)[idx].cpu().numpy()
    oq, oe = O.bfp_conv(q_s, e_s, fdr, n, O.kernel_plan(n, v), block=64)
    torch.cuda.synchronize()
    assert np.array_equal(eo.view(batch, nb)[idx].cpu().numpy(), oe.reshape(16, -1))
    assert np.array_equal(qo.view(batch, 2 * n)[idx].cpu().numpy(), oq.reshape(16, -1))
    del dq, de, qo, eo


@pytest.mark.parametrize("n,variant,layout", [(512, "auto", "dr"), (4096, "auto", "dr"),
                                              (512, "fastest", "lane"), (4096, "fastest", "lane")])
def test_bfp_config3_full_size(dev, n, variant, layout):
    """BASELINE config 3 as written: 2^27 points of per-signal Gaussian x 10^u
    (u ~ U[-3, 3]) signals, quantised by the library's host codec (64-point
    blocks), one shared fp32 filter, at N = 512 and 4096 with the default
    plan and with the bench's (lane-major filter at the fastest variant).
    16 signals spread over the batch: words and exponents bit-identical to
    the oracle, and rel L2 <= 1e-4 against the fp64 convolution of the
    unquantised signals (input quantisation included)."""
    import torch
    import fufft_amd as ff
    batch = (1 << 27) // n
    gen = torch.Generator(device=dev)
    gen.manual_seed(31 * n + len(layout))
    scale = torch.pow(10.0, torch.rand(batch, 1, device=dev, generator=gen) * 6 - 3)
    x = (torch.randn(batch, n, dtype=torch.complex64, device=dev, generator=gen) * scale).cpu().numpy()
    del scale
    q, e = ff.bfp_quantize(x)
    rng = np.random.default_rng(n)
    taps = crandn(rng, n)
    var = ff.fastest_variant(n, layout) if variant == "fastest" else variant
    v = 8 if ff.resolve_variant(n, var) == "r8" else 16
    filt = ff.plan_filter(taps, n, variant=var, layout=layout, kind=ff.FILTER_TAPS)
    fdr = ff.plan_filter(taps, n, variant=var, layout="dr", kind=ff.FILTER_TAPS)
    dq, de = to_dev(q, dev), to_dev(e, dev)
    qo, eo = torch.empty_like(dq), torch.empty_like(de)
    print(f"case bfp config 3 full size n={n} variant={var} layout={layout} batch={batch}", flush=True)
    ff.conv_bfp16(dq, de, to_dev(filt, dev), qo, eo, n=n, batch=batch, variant=var, layout=layout)
    idx = np.linspace(0, batch - 1, 16).astype(np.int64)
    tidx = torch.from_numpy(idx).to(dev)
    nb = n // 64
    q_s = q.reshape(batch, 2 * n)[idx]
    e_s = e.reshape(batch, nb)[idx]
    oq, oe = O.bfp_conv(q_s, e_s, fdr, n, O.kernel_plan(n, v))
    torch.cuda.synchronize()
    got_q = qo.view(batch, 2 * n)[tidx].cpu().numpy()
    got_e = eo.view(batch, nb)[tidx].cpu().numpy()
    assert np.array_equal(got_e, oe.reshape(16, -1))
    assert np.array_equal(got_q, oq.reshape(16, -1))
    spec = np.fft.fft(taps.astype(np.complex128)) / n
    want = np.fft.ifft(np.fft.fft(x[idx].astype(np.complex128), axis=1) * spec[None, :] * n, axis=1)
    got = O.bfp_dequantize(got_q, got_e).reshape(16, n)
    rel = np.sqrt(np.sum(np.abs(got - want) ** 2) / np.sum(np.abs(want) ** 2))
    print(f"   rel L2 {rel:.3e}", flush=True)
    assert rel <= TOL_BFP
    del dq, de, qo, eo
