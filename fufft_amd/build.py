"""Build the gfx950 library (fufft_amd/libfufft_amd.so) and the CPU oracle.

Everything is compiled in-tree so the shared objects travel with the source
tree to the GPU box.  hipcc cross-compiles for gfx950 without a GPU.

    python fufft_amd/build.py            # library + oracle (+ reference shim)
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libfufft_amd.so"
ORACLE = ROOT / "oracle"
REFERENCE = Path(os.environ.get("FUFFT_REFERENCE", "/root/reference"))

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -ffp-contract=off: the operation order is part of the parity contract.
# -packed-fp32-ops removed: packed fp32 VALU forms are not used on this pool.
HIPFLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _run(cmd: list[str]) -> None:
    p = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the packed-fp32 feature; that warning is noise
    err = "\n".join(l for l in p.stderr.splitlines() if "not a recognized feature" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build_library(jobs: int = 8) -> Path:
    OBJ.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    headers = list(CSRC.glob("*.hpp")) + [ROOT / "include" / "fufft" / "fufft.h"]
    newest_header = max(h.stat().st_mtime for h in headers)

    def compile_one(src: Path) -> Path:
        obj = OBJ / (src.stem + ".o")
        if obj.exists() and obj.stat().st_mtime > max(src.stat().st_mtime, newest_header):
            return obj
        _run([HIPCC, *HIPFLAGS, "-c", str(src), "-o", str(obj)])
        return obj

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, sources))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


def build_cpp_checks() -> Path:
    """The C++ caller test (tests/cpp/abi_gpu_check.cpp): host code only,
    linked against this library and the HIP runtime; run on a GPU by
    tests/test_gpu_cpp_caller.py."""
    src = ROOT / "tests" / "cpp" / "abi_gpu_check.cpp"
    out_dir = ROOT / "tests" / "cpp" / "_build"
    out_dir.mkdir(exist_ok=True)
    exe = out_dir / "abi_gpu_check"
    rocm = Path(HIPCC).resolve().parent.parent
    _run(["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
          f"-I{ROOT / 'include'}", f"-I{rocm / 'include'}", str(src),
          f"-L{PKG}", "-lfufft_amd", f"-L{rocm / 'lib'}", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN/../../../fufft_amd", f"-Wl,-rpath,{rocm / 'lib'}", "-o", str(exe)])
    return exe


def build_oracle() -> None:
    _run(["make", "-s", "-C", str(ORACLE)])
    if (REFERENCE / "verify_kernel.cpp").exists() and shutil.which("g++"):
        _run(["make", "-s", "-C", str(ORACLE), "ref", f"REF={REFERENCE}"])


def build(jobs: int = 8) -> None:
    build_oracle()
    build_library(jobs)
    if shutil.which("g++"):
        build_cpp_checks()


if __name__ == "__main__":
    build()
    print(LIB)
