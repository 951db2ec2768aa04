"""Static checks of this build's own gfx950 code (fufft_amd/isa_report.py).

- No kernel of the library spills registers or uses scratch.
- The analytic operation model (fp32 arithmetic, LDS traffic and
  vector-memory instructions per pass plan) matches the compiled kernels:
  the kernels are straight-line code, so static counts are what each
  wavefront executes (plus the untaken side of the filter-layout branch).
- The same counts match what rocprofv3 measured per wavefront for the
  headline kernel (profiles/conv_f32_n4096.md): model, ISA and hardware
  counters agree.
- Occupancy: radix-8 lanes give 8 wavefronts per SIMD where radix-16 lanes
  are held to 4 by LDS -- the reason FUFFT_AUTO picks radix 8.
"""
import re
from pathlib import Path

import pytest

from fufft_amd import isa_report as R

ROOT = Path(__file__).resolve().parent.parent
pytestmark = pytest.mark.skipif(not R.tools_available() or not list(R.OBJ.glob("*.o")),
                                reason="needs this build's objects and the ROCm LLVM tools")


@pytest.fixture(scope="module")
def rows():
    return R.load()


@pytest.fixture(scope="module")
def conv(rows):
    return R.conv_rows(rows)


def pick(conv, kind, n, v, layout=None, mid="mul"):
    layout = layout or R.default_layout(n, v)
    got = [r for r in conv if r["family"] == "conv1d" and r["kind"] == kind and r["n"] == n and r["v"] == v
           and r["layout"] == layout and r["mid"] == mid]
    assert len(got) == 1, (kind, n, v)
    return got[0]


SIZES = [(n, 16) for n in (256, 512, 1024, 2048, 4096, 8192, 16384)] + [(n, 8) for n in (512, 1024, 2048, 4096, 8192)]


def test_no_kernel_spills_or_uses_scratch(rows):
    """Every kernel of the default LDS layouts is spill-free.  The opt-in XOR
    layout (FUFFT_LDS_LAYOUT=xor) keeps one address register per tap; at
    N = 16384 (1024 threads, so at most 128 VGPRs) it spills, which is one
    more reason the additive layouts are the default."""
    assert len(rows) > 100
    bad, xor16k = [], []
    for r in rows:
        m = r["meta"]
        if m.get("private_segment_fixed_size", 0) or m.get("vgpr_spill_count", 0) or m.get("sgpr_spill_count", 0):
            d = r["decoded"]
            (xor16k if d and d["layout"] == "xor" and d["n"] == 16384 else bad).append(r["name"])
    assert not bad, bad[:3]
    assert len(xor16k) <= 8


@pytest.mark.parametrize("n,v", SIZES)
@pytest.mark.parametrize("kind,mid", [("conv", "mul"), ("conv", "conj"), ("c2c_fwd", "none"),
                                      ("c2c_inv", "none"), ("plan_taps", "none"), ("fwd", "none")])
def test_model_matches_compiled_kernel(conv, n, v, kind, mid):
    r = pick(conv, kind, n, v, mid=mid)
    m = r["model"]
    # the compiler may fold a few products into constants, never add arithmetic
    assert 0.985 * m["fp32_arith_per_lane"] <= r["fp32_arith"] <= m["fp32_arith_per_lane"], r
    assert r["lds_access_8B"] == m["lds_access_8B_per_lane"], r
    assert r["vmem_load"] == m["vmem_loads_per_wave"] + m["untaken_branch"]["loads"], r
    assert r["vmem_store"] == m["vmem_stores_per_wave"] + m["untaken_branch"]["stores"], r


def test_occupancy_radix8_vs_radix16(conv):
    for n in (512, 1024, 2048, 4096, 8192):
        assert pick(conv, "conv", n, 8)["waves_per_simd"] == 8, n
    # radix 16 at N = 4096: 4 wavefronts per SIMD by LDS (one transform of 34 KiB
    # per 4-wavefront workgroup), which the kept radix-16 chain's VGPRs (at most
    # 128 for 4 wavefronts) do not lower
    r16 = pick(conv, "conv", 4096, 16)
    assert r16["waves_per_simd"] == 4 and r16["limited_by"] in ("LDS", "VGPRs") and r16["vgpr"] <= 128


def test_counters_agree_with_model_and_isa(conv):
    """profiles/conv_f32_n4096.md: SQ_INSTS_VALU, SQ_INSTS_LDS and SQ_INSTS_VMEM
    per wavefront of the headline kernel, conv1d_kernel<4096, 16, xchg, conv, mul>
    (radix-16 lanes, lane-major pair filter)."""
    text = (ROOT / "profiles" / "conv_f32_n4096.md").read_text()

    def per_wave(counter):
        m = re.search(rf"\|\s*{counter}\s*\|\s*\d+\s*\|\s*([0-9.]+)\s*\|", text)
        assert m, counter
        return float(m.group(1))

    r = pick(conv, "conv", 4096, 16)
    m = r["model"]
    # the kernel also holds the digit-order filter's hand-over through LDS
    # (mid_op_dr_staged: 8 ds_write2_b64 + 8 ds_read2_b64 and their address
    # arithmetic), a branch the profile's lane-major filter does not take
    staged_lds = 16
    assert 0 <= r["valu"] - per_wave("SQ_INSTS_VALU") <= 48
    assert per_wave("SQ_INSTS_LDS") == r["lds"] - staged_lds
    assert per_wave("SQ_INSTS_VMEM") == m["vmem_loads_per_wave"] + m["vmem_stores_per_wave"]


def test_wide_kernel_matches_model(rows):
    """The N = 16384 / 32768 conv (wide.hip) against its op model: LDS accesses
    and vector-memory instructions exactly; fp32 arithmetic within 0.5% (at
    N = 32768 the compiled code has 16 fewer operations than the model's 3936
    with a filter, 3808 without, in every variant; not traced to a pass)."""
    wide = [r for r in R.conv_rows(rows) if r["family"] == "wide"]
    # per size: 2 mids x 3 filter layouts + mid none
    assert sorted(r["n"] for r in wide) == [16384] * 7 + [32768] * 7
    for r in wide:
        m = r["model"]
        assert r["lds_access_8B"] == m["lds_access_8B_per_lane"]
        assert (r["vmem_load"], r["vmem_store"]) == (m["vmem_loads_per_wave"], m["vmem_stores_per_wave"])
        assert 0 <= m["fp32_arith_per_lane"] - r["fp32_arith"] <= 0.005 * m["fp32_arith_per_lane"]
        assert r["vgpr"] <= 128 and r["scratch"] == 0 and r["waves_per_simd"] == 4
