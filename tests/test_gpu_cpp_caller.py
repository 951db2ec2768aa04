"""A C++ caller on the GPU, with no Python on the compute path.

tests/cpp/abi_gpu_check.cpp (built by fufft_amd/build.py, linked against
libfufft_amd.so and the HIP runtime) allocates with hipMalloc, plans the filter
with include/fufft/fufft.hpp, and checks the template surface against an fp64
direct cyclic convolution (rel L2 <= 2e-6) and, bit for bit, against the raw C
entry point, the split forward/apply path and an in-place call; the int16 BFP
conv in the reference's own format bit for bit against dequantise -> fp32 conv
-> quantise; a 64 x 64 image (one fused launch) against an fp64 direct 2D
cyclic convolution; and the plan objects of include/fufft/plan.hpp (Conv1d
lane-major / digit order / planned on the device / BFP, ConvLarge with the
reference's V=16 middle, Conv2d, a Conv1d at N = 32768) bit for bit against
the C calls with filters planned by hand, a per-signal plan refusing a
mismatched batch.
"""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "cpp" / "_build" / "abi_gpu_check"


def test_cpp_caller_through_the_c_abi(dev):
    assert EXE.exists(), f"{EXE} is missing: run python fufft_amd/build.py"
    print("case C++ caller n=4096 batch=16", flush=True)
    out = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=120)
    print(out.stdout.strip(), out.stderr.strip(), flush=True)
    assert out.returncode == 0, (out.returncode, out.stderr)
    assert out.stdout.startswith("ok C++ caller")
