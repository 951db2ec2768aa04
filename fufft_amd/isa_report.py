"""Static instruction report of this library's own gfx950 kernels, beside an
analytic operation model and an occupancy explainer.

The counterpart of the reference's count_instructions.py / occupancy.py /
ncu_compare.py (instruction classes per kernel from the compiled code, a
per-point operation model, and which resource limits resident warps).  Here:

- the gfx950 code object of each translation unit is taken out of this
  build's own objects (fufft_amd/_build/*.o: objcopy of .hip_fatbin, then
  clang-offload-bundler) and disassembled with llvm-objdump; kernel metadata
  (VGPRs, SGPRs, scratch, spills) comes from the code object's note;
- the kernels are straight-line code (every pass loop is unrolled), so the
  static count of a class equals the count each wavefront executes, apart
  from the untaken side of the filter-layout branch;
- model_conv() counts the fp32 arithmetic the pipeline needs per lane
  (butterflies: 4 / 16 / 56 / 168 operations for radix 2 / 4 / 8 / 16; stage
  twiddles: 2R - 3 complex products of 2 MUL + 2 FMA per twiddled group,
  i.e. R - 1 applied and R - 2 generated, less the R - 2 a fused kernel
  carries from its forward to its inverse where it keeps that chain; the mid product: 4 per
  value), the
  LDS traffic (V writes and V reads per lane per exchange) and the
  vector-memory instructions per wavefront;
- occupancy() gives wavefronts per SIMD and the limiting resource from VGPRs
  (512 per lane, granule 8), LDS (160 KiB per CU) and the 8-wave cap.

    python -m fufft_amd.isa_report [--kind conv] [--markdown]
"""
from __future__ import annotations

import argparse
import json
import re
import shutil
import subprocess
import tempfile
from pathlib import Path

PKG = Path(__file__).resolve().parent
OBJ = PKG / "_build"
LLVM = Path("/opt/rocm/llvm/bin")
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"

KINDS = {0: "conv", 1: "conv_r2", 2: "fwd", 3: "apply", 4: "fwd_r2", 5: "apply_r2",
         6: "c2c_fwd", 7: "c2c_inv", 8: "plan_taps", 9: "conv_timed", 10: "conv_mid",
         11: "conv_psf", 12: "conv_psf_dr"}
MIDS = {0: "mul", 1: "conj", 2: "none"}
LAYOUTS = {0: "xor", 1: "pad", 2: "xchg"}
FILTERS = {0: "dr", 1: "lane", 2: "bperm"}

FP32_ARITH = re.compile(r"^v_(add|sub|subrev|mul|fma|fmac|fmaak|fmamk)_f32")
# bytes moved per lane by each LDS data instruction
LDS_BYTES = {"ds_read_b32": 4, "ds_write_b32": 4, "ds_read2_b32": 8, "ds_write2_b32": 8,
             "ds_read2st64_b32": 8, "ds_write2st64_b32": 8, "ds_read_b64": 8, "ds_write_b64": 8,
             "ds_read2_b64": 16, "ds_write2_b64": 16, "ds_read2st64_b64": 16, "ds_write2st64_b64": 16,
             "ds_read_b128": 16, "ds_write_b128": 16}


# ---- code objects --------------------------------------------------------------------------

def tools_available() -> bool:
    return all((LLVM / t).exists() for t in ("llvm-objdump", "llvm-readelf", "clang-offload-bundler")) \
        and shutil.which("objcopy") is not None


def code_object(obj: Path, workdir: Path) -> Path:
    """The gfx950 code object bundled into one of this build's object files."""
    fat = workdir / (obj.stem + ".fatbin")
    co = workdir / (obj.stem + ".co")
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", str(obj), str(fat)], check=True)
    subprocess.run([str(LLVM / "clang-offload-bundler"), "--type=o", f"--targets={TARGET}",
                    f"--input={fat}", f"--output={co}", "--unbundle"], check=True)
    return co


def kernel_metadata(co: Path) -> dict:
    notes = subprocess.run([str(LLVM / "llvm-readelf"), "--notes", str(co)], check=True,
                           capture_output=True, text=True).stdout
    out, cur = {}, {}
    keys = ("name", "vgpr_count", "agpr_count", "sgpr_count", "private_segment_fixed_size",
            "group_segment_fixed_size", "vgpr_spill_count", "sgpr_spill_count", "max_flat_workgroup_size")
    for line in notes.splitlines():
        m = re.match(r"\s+(- )?\.(\w+):\s+(\S+)\s*$", line)
        if not m:
            continue
        if m.group(1) and cur:               # a new list item starts a new kernel
            if "name" in cur:
                out[cur["name"]] = cur
            cur = {}
        if m.group(2) in keys:
            cur[m.group(2)] = m.group(3) if m.group(2) == "name" else int(m.group(3))
    if "name" in cur:
        out[cur["name"]] = cur
    return out


def kernel_instructions(co: Path) -> dict:
    text = subprocess.run([str(LLVM / "llvm-objdump"), "-d", str(co)], check=True,
                          capture_output=True, text=True).stdout
    out, name = {}, None
    for line in text.splitlines():
        m = re.match(r"^[0-9a-f]+ <(\S+)>:", line)
        if m:
            name = m.group(1)
            out[name] = []
            continue
        if name and line.startswith((" ", "\t")):
            t = line.split()
            if t and re.match(r"^[a-z_0-9]+$", t[0]):
                out[name].append(t[0])
    return out


def classify(ops: list) -> dict:
    c = {"valu": 0, "fp32_arith": 0, "salu": 0, "smem": 0, "vmem_load": 0, "vmem_store": 0,
         "lds": 0, "lds_bytes": 0, "branch": 0, "waitcnt_barrier": 0}
    for op in ops:
        if op.startswith("v_"):
            c["valu"] += 1
            if FP32_ARITH.match(op):
                c["fp32_arith"] += 1
        elif op.startswith("ds_"):
            c["lds"] += 1
            c["lds_bytes"] += LDS_BYTES.get(op, 0)
        elif op.startswith(("buffer_load", "global_load")):
            c["vmem_load"] += 1
        elif op.startswith(("buffer_store", "global_store")):
            c["vmem_store"] += 1
        elif op.startswith(("s_load", "s_buffer_load", "s_memtime", "s_memrealtime")):
            c["smem"] += 1
        elif op.startswith(("s_cbranch", "s_branch", "s_setpc", "s_endpgm")):
            c["branch"] += 1
        elif op.startswith(("s_waitcnt", "s_barrier")):
            c["waitcnt_barrier"] += 1
        elif op.startswith("s_"):
            c["salu"] += 1
    c["lds_access_8B"] = c["lds_bytes"] / 8
    return c


def decode_name(name: str) -> dict | None:
    m = re.search(r"conv1d_kernelILi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)E", name)
    if m:
        n, v, lay, kind, mid = map(int, m.groups())
        return {"family": "conv1d", "n": n, "v": v, "layout": LAYOUTS[lay], "kind": KINDS[kind],
                "mid": MIDS[mid]}
    m = re.search(r"bfp_kernelILi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELb([01])E", name)
    if m:
        n, v, lay, mid, big = map(int, m.groups())
        # big: blocks of more than 64 points (LDS rendezvous of the block maxima)
        return {"family": "bfp", "n": n, "v": v, "layout": LAYOUTS[lay],
                "kind": "conv_blocks" if big else "conv", "mid": MIDS[mid]}
    # the N = 16384 / 32768 conv (wide.hip): 32 values per lane, float exchanges
    m = re.search(r"conv_wide_kernelILi(\d+)ELi(\d+)ELi(\d+)E", name)
    if m:
        n, mid, flt = map(int, m.groups())
        return {"family": "wide", "n": n, "v": 32, "layout": "split", "kind": "conv", "mid": MIDS[mid],
                "filter": FILTERS[flt]}
    return None


def load(objs=None) -> list:
    """Every kernel of the given objects (default: all of fufft_amd/_build)."""
    objs = sorted(OBJ.glob("*.o")) if objs is None else objs
    rows = []
    with tempfile.TemporaryDirectory() as d:
        for obj in objs:
            co = code_object(obj, Path(d))
            meta = kernel_metadata(co)
            ins = kernel_instructions(co)
            for name, ops in ins.items():
                if name not in meta:
                    continue
                rows.append({"tu": obj.stem, "name": name, "meta": meta[name], "counts": classify(ops),
                             "decoded": decode_name(name)})
    return rows


# ---- model -------------------------------------------------------------------------------

DFT_OPS = {2: 4, 4: 16, 8: 56, 16: 168}


def plan(n: int, v: int) -> list:
    """(radix, stride) per DIF pass: leftover radix first, then radix v."""
    m, lv = n.bit_length() - 1, v.bit_length() - 1
    rads = ([1 << (m % lv)] if m % lv else []) + [v] * (m // lv)
    out, M = [], n
    for r in rads:
        M //= r
        out.append((r, M))
    return out


def model_conv(n: int, v: int, kind: str = "conv", mid: str = "mul") -> dict:
    """Per-lane fp32 arithmetic and LDS accesses, per-wavefront vector-memory
    instructions, of one kernel (digit-order filter)."""
    if kind == "conv_mid":               # the four-step middle: the conv with another cache policy
        kind = "conv"
    ps = plan(n, v)
    one_dir =sum((v // r) * (DFT_OPS[r] + (4 * (2 * r - 3) if M > 1 else 0)) for r, M in ps)
    exchanges = len(ps) - 1
    twiddle_slots = sum(v // r for r, M in ps if M > 1)
    two = kind in ("conv", "conv_r2", "conv_timed", "conv_psf", "conv_psf_dr")
    arith = one_dir * (2 if two else 1)
    # the forward's last twiddled pass hands its chain to the inverse when that
    # pass has one group per lane and the registers allow it (KeptChain): pure
    # powers of the radix, and radix 16 up to N = 2048 behind a lead pass;
    # R - 2 fewer complex products per lane, 6 at radix 8 and 14 at radix 16
    # (the per-signal kernels that read their filter early, conv_psf at radix 16 N = 1024 .. 4096 and
    # conv_psf_dr, hold it in those registers instead; conv_psf at radix 8 N = 512 reads it late and
    # keeps the chain)
    early = kind == "conv_psf_dr" or (kind == "conv_psf" and v == 16 and n in (1024, 2048, 4096))
    if two and not early and len(ps) >= 2 and ps[-2][0] == v and ps[-2][1] > 1 and \
            (all(r == v for r, _ in ps) or (v == 16 and n // v <= 128)):
        arith -= 4 * (v - 2)
    if kind in ("conv", "conv_r2", "conv_timed", "conv_psf", "conv_psf_dr", "apply", "apply_r2") and mid != "none":
        arith += 4 * v
    if kind == "plan_taps":
        arith += 2 * v                   # the 1/N scale
    lds = 2 * v * exchanges * (2 if two else 1)
    if kind in ("c2c_fwd", "c2c_inv"):
        lds += 2 * v                     # the digit <-> natural exchange
    if kind in ("conv", "conv_r2", "conv_timed", "conv_psf_dr", "apply", "apply_r2") and mid != "none" and \
            v == 16 and n >= 2048:
        lds += 2 * v                     # the digit-order filter handed over through LDS (dr_runs_stage)
    loads = {"conv": v, "conv_timed": v, "conv_psf": v, "conv_psf_dr": v, "conv_r2": 2 * v, "fwd": v, "fwd_r2": 2 * v, "apply": v // 2,
             "apply_r2": v // 2, "c2c_fwd": v, "c2c_inv": v, "plan_taps": v}[kind]
    loads += twiddle_slots
    if kind in ("conv", "conv_r2", "conv_timed", "conv_psf", "conv_psf_dr", "apply", "apply_r2") and mid != "none":
        loads += v // 2
    stores = {"conv_r2": 2 * v, "apply_r2": 2 * v, "fwd": v // 2, "fwd_r2": v // 2,
              "plan_taps": v // 2}.get(kind, v)
    # code for the other side of a runtime layout branch sits in the kernel but does not run:
    # the lane-major pair filter read (V/2 16-byte loads), the lane-major spectrum read of the
    # inverse-only kernels (V/2) and the bperm store of the taps planner (V 8-byte stores).  The
    # digit-order and pair spectrum stores take one code path (the offsets are selected); a
    # bperm filter read has kernels of its own (conv1d_bperm_kernel, bfp_bperm_kernel).
    untaken_loads = v // 2 if (kind in ("conv", "conv_r2", "conv_timed", "apply", "apply_r2") and mid != "none") else 0
    if kind in ("apply", "apply_r2"):
        untaken_loads += v // 2
    untaken = {"loads": untaken_loads, "stores": v if kind == "plan_taps" else 0}
    return {"fp32_arith_per_lane": arith, "lds_access_8B_per_lane": lds, "vmem_loads_per_wave": loads,
            "vmem_stores_per_wave": stores, "untaken_branch": untaken, "passes": ps}


def model_wide(mid: str = "mul", filt: str = "lane", n: int = 32768, v: int = 32) -> dict:
    """The N = 16384 / 32768 conv (wide.hip): the radix-16 plan with V/R groups
    per lane in every pass (8 / 4 in the radix-4 / radix-8 lead, 2 in the
    radix-16 passes), no kept chain; each exchange writes and reads both float
    components of the lane's V values (V 8-byte equivalents each way); the
    filter as V/2 16-byte loads (V 8-byte ones in bperm).  A lead pass of more
    than 4 groups per lane reads its base twiddles again for the inverse."""
    ps = plan(n, 16)
    one_dir = sum((v // r) * (DFT_OPS[r] + (4 * (2 * r - 3) if M > 1 else 0)) for r, M in ps)
    arith = 2 * one_dir + (4 * v if mid != "none" else 0)
    lds = 2 * v * (len(ps) - 1) * 2
    # a pass with M <= T gives both of a lane's groups the same base twiddle
    # index ((L + g T) mod M = L mod M), and the compiler merges those loads
    t = n // v
    loads = v + sum((v // r) if M > t else 1 for r, M in ps if M > 1)
    if v // ps[0][0] > 4:
        loads += v // ps[0][0]
    if mid != "none":
        loads += v if filt == "bperm" else v // 2
    return {"fp32_arith_per_lane": arith, "lds_access_8B_per_lane": lds, "vmem_loads_per_wave": loads,
            "vmem_stores_per_wave": v, "untaken_branch": {"loads": 0, "stores": 0}, "passes": ps}


# ---- occupancy ---------------------------------------------------------------------------

def occupancy(vgpr: int, agpr: int, lds_bytes: int, waves_per_wg: int) -> dict:
    """Resident wavefronts per SIMD on gfx950 and what limits them."""
    regs = -(-vgpr // 8) * 8 + -(-agpr // 8) * 8
    by_vgpr = 512 // regs if regs else 8
    by_lds = (160 * 1024 // lds_bytes) * waves_per_wg / 4 if lds_bytes else 8
    limits = {"wave cap": 8, "VGPRs": by_vgpr, "LDS": by_lds}
    lim = min(limits, key=limits.get)
    return {"waves_per_simd": int(min(limits.values())), "limited_by": lim, "vgpr_alloc": regs}


def default_layout(n: int, v: int, family: str = "conv1d") -> str:
    """The LDS layout a plan runs by default: default_lds_layout in fufft_plan.hpp
    for the fp32 kernels; the BFP kernels take the per-exchange layouts at every
    plan (bfp_lds_layout in bfp.hip)."""
    if family == "bfp":
        return "xchg"
    if family == "wide":
        return "split"
    return "pad" if (v == 8 and n > 4096) else "xchg"


def lds_bytes_conv(n: int, v: int, layout: str) -> int:
    t = n // v
    cpb = 1 if t >= 128 else 256 // t
    return cpb * (n + (n // v if layout in ("pad", "xchg") else 0)) * 8


def conv_rows(rows=None) -> list:
    rows = load() if rows is None else rows
    out = []
    for r in rows:
        d = r["decoded"]
        if not d:
            continue
        n, v = d["n"], d["v"]
        t = n // v
        threads = t if t >= 128 else 256
        # the wide kernel's float buffer: N + N/16 slots of 4 bytes
        lds = (n + n // 16) * 4 if d["family"] == "wide" else lds_bytes_conv(n, v, d["layout"])
        occ = occupancy(r["meta"]["vgpr_count"], r["meta"].get("agpr_count", 0), lds, threads // 64)
        mod = model_conv(n, v, d["kind"], d["mid"]) if d["family"] == "conv1d" else \
            model_wide(d["mid"], d["filter"], n) if d["family"] == "wide" else None
        out.append({**d, "vgpr": r["meta"]["vgpr_count"], "sgpr": r["meta"]["sgpr_count"],
                    "scratch": r["meta"].get("private_segment_fixed_size", 0),
                    "spills": r["meta"].get("vgpr_spill_count", 0) + r["meta"].get("sgpr_spill_count", 0),
                    "lds_per_wg": lds, **{k: r["counts"][k] for k in ("valu", "fp32_arith", "lds", "lds_access_8B",
                                                                     "vmem_load", "vmem_store", "salu")},
                    "model": mod, **occ})
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--kind", default="conv")
    ap.add_argument("--layout", default="default", help="default (each plan's own), xchg, pad or xor")
    ap.add_argument("--mid", default="mul")
    ap.add_argument("--markdown", action="store_true")
    a = ap.parse_args()
    rows = [r for r in conv_rows() if r["kind"] == a.kind and r["mid"] == a.mid
            and r["layout"] == (default_layout(r["n"], r["v"], r["family"]) if a.layout == "default" else a.layout)]
    rows.sort(key=lambda r: (r["family"], r["v"], r["n"]))
    if not a.markdown:
        for r in rows:
            print(json.dumps({k: v for k, v in r.items() if k != "model"} |
                             ({"model": {k: v for k, v in r["model"].items() if k != "passes"}} if r["model"] else {})))
        return
    print("| kernel | N | V | VGPR | scratch | waves/SIMD (limit) | VALU | fp32 arith: ISA / model | "
          "LDS 8-B accesses / lane: ISA / model | VMEM load+store, static: ISA / model |")
    print("|---|---|---|---|---|---|---|---|---|---|")
    for r in rows:
        m = r["model"]
        ar = f"{r['fp32_arith']} / {m['fp32_arith_per_lane']}" if m else f"{r['fp32_arith']} / —"
        ld = f"{r['lds_access_8B']:g} / {m['lds_access_8B_per_lane']}" if m else f"{r['lds_access_8B']:g} / —"
        vm = (f"{r['vmem_load']}+{r['vmem_store']} / {m['vmem_loads_per_wave'] + m['untaken_branch']['loads']}"
              f"+{m['vmem_stores_per_wave'] + m['untaken_branch']['stores']}") if m else \
            f"{r['vmem_load']}+{r['vmem_store']} / —"
        label = f"{r['family']} {r['kind']}" + (f" ({r['filter']} filter)" if r["family"] == "wide" else "")
        print(f"| {label} | {r['n']} | {r['v']} | {r['vgpr']} | {r['scratch']} | "
              f"{r['waves_per_simd']} ({r['limited_by']}) | {r['valu']} | {ar} | {ld} | {vm} |")


if __name__ == "__main__":
    main()
