"""GPU check of the stream-ceiling copy (fufft_stream_f32 and its shapes,
fufft_stream_shape_f32): every shape bench.py sweeps copies exactly, also
with a last partial tile, and writes nothing past the copied bytes.  No
reference counterpart (measurement only)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LOADS = (1, 2, 4, 8, 16, 32)
GRID = ((1, 0), (2, 0), (4, 0), (3, 0), (1, 7), (1, 1024))
POLICY = ((0, 0), (2, 2), (2, 0), (0, 2), (1, 1), (3, 3))


# every shape of the copy: a workgroup tile of at most 256 KiB (1024 lanes of
# 512 bytes in flight would spill registers and is refused)
SHAPES = [(lanes, width, loads) for lanes in (64, 256, 1024) for width in (8, 16) for loads in LOADS
          if lanes * width * loads <= 256 * 1024]


@pytest.mark.parametrize("lanes,width,loads", SHAPES)
def test_stream_shapes_copy_exactly(dev, loads, width, lanes):
    import torch
    import fufft_amd as ff
    # 1 MiB + 3 KiB + 16 B: several tiles of every size and a partial last one
    nbytes = (1 << 20) + 3 * 1024 + 16
    gen = torch.Generator(device=dev)
    gen.manual_seed(loads)
    x = torch.randn(nbytes // 8, dtype=torch.complex64, device=dev, generator=gen)
    # the output buffer is longer than the copy: the tail must stay untouched
    y = torch.empty(nbytes // 8 + 4096, dtype=torch.complex64, device=dev)
    for per, groups in GRID:
        for pld, pst in POLICY:
            print(f"case stream lanes={lanes} width={width} loads={loads} per={per} groups={groups} "
                  f"policy={pld}/{pst}", flush=True)
            y.fill_(7.0)
            ff.stream_copy_shape(x, y, nbytes, loads, per, groups, pld, pst, width=width, lanes=lanes)
            torch.cuda.synchronize()
            assert torch.equal(y[: x.numel()].view(torch.int32), x.view(torch.int32))
            assert bool((y[x.numel():] == 7.0).all())


def test_stream_fixed_shapes(dev):
    import torch
    import fufft_amd as ff
    x = torch.arange(2 * 100000, dtype=torch.float32, device=dev).view(torch.complex64)
    for nt in (False, True):
        y = torch.zeros_like(x)
        print(f"case stream fixed nt={nt}", flush=True)
        ff.stream_copy(x, y, x.numel() * 8, nt)
        torch.cuda.synchronize()
        assert torch.equal(x, y)
