"""LDS bank model of gfx950, measured.

The conv kernels exchange data through LDS with 8-byte accesses
(ds_read2_b64 / ds_write2_b64 / ds_read2st64_b64, and ds_read_b64 or
ds_write_b64 where an offset does not fit the paired form).  Their layouts are
designed against the model below, which this module both states and measures.

Model (slots are float2 indices, i.e. byte address / 8):

- ``read_b64``: the wavefront is serviced 32 lanes at a time; two lanes of a
  half-wavefront conflict when their slots differ but agree modulo 32.
- ``write_b64``, ``write2_b64``, ``read2_b64``, ``read2st64_b64``: each 8-byte
  access (two for the paired forms) is serviced 16 lanes at a time; two lanes
  of a quarter-wavefront conflict when their slots differ but agree modulo 16.

A group whose most-shared residue holds d distinct slots costs d - 1 extra
cycles; the counter SQ_LDS_BANK_CONFLICT is the sum over groups and accesses.

Measurement: ``fufft_amd/libfufft_lds_probe.so`` (``csrc/probe/lds_probe.hip``)
runs one 64-lane workgroup per pattern and instruction form, many times over;
under ``rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS SQ_WAVES`` each
dispatch gives the conflict cycles per instruction.

    rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS SQ_WAVES --output-format csv \\
        -d OUT -o run -- python3 -m fufft_amd.lds_probe --order OUT/order.json
    python -m fufft_amd.lds_probe --summarize OUT/run_counter_collection.csv --order OUT/order.json

The summary lists measured and modelled cycles side by side
(profiles/lds_bank_model.md); tests/test_lds_audit.py checks every row.
"""
from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

LIB = Path(__file__).resolve().parent / "libfufft_lds_probe.so"
SLOTS = 20480                  # the probe kernel's LDS (160 KiB), float2 slots
REPS = 256
BLOCKS = 1024

FORMS = ("read_b64", "read2_b64", "write_b64", "write2_b64", "read2st64_b64")
# second access of the paired forms, in slots (offset1 = 1 in units of 8 or 512 bytes)
SECOND = {"read2_b64": 1, "write2_b64": 1, "read2st64_b64": 64}


def _patterns() -> dict:
    lane = range(64)
    p = {"contiguous": [l for l in lane]}
    for s in (2, 3, 4, 8, 16, 32, 33, 64):
        p[f"stride {s}"] = [s * l for l in lane]
    p["padded by 8 (i + i/8)"] = [l + l // 8 for l in lane]
    p["padded by 16 (i + i/16)"] = [l + l // 16 for l in lane]
    # column tiles: lane = 16 * L + column, each column its own slot of S float2
    for s in (576, 577, 578, 579, 580, 582, 584, 586, 588, 592, 600):
        p[f"16 columns x {s} + L"] = [(l % 16) * s + l // 16 for l in lane]
    for s in (2176, 2178, 2180):
        p[f"8 columns x {s} + L"] = [(l % 8) * s + l // 8 for l in lane]
    return p


PATTERNS = _patterns()


def conflict_cycles(slots, form: str) -> int:
    """Extra cycles of one instruction of `form` whose lanes access `slots`."""
    if form == "read_b64":
        accesses, group, mod = [list(slots)], 32, 32
    else:
        accesses = [list(slots)]
        if form in SECOND:
            accesses.append([s + SECOND[form] for s in slots])
        group, mod = 16, 16
    total = 0
    for acc in accesses:
        for h in range(0, len(acc), group):
            banks: dict = {}
            for s in acc[h:h + group]:
                banks.setdefault(s % mod, set()).add(s)
            total += max(len(x) for x in banks.values()) - 1
    return total


def run(order_path: Path | None) -> list:
    import ctypes as C
    import torch
    if not LIB.exists():
        raise RuntimeError(f"{LIB} is missing: run python -m fufft_amd.build")
    lib = C.CDLL(str(LIB))
    lib.fufft_lds_probe.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p]
    dev = torch.device("cuda:0")
    out = torch.empty(BLOCKS * 64, dtype=torch.float32, device=dev)
    order = []
    for name, slots in PATTERNS.items():
        if len(slots) != 64 or min(slots) < 0 or max(slots) + 64 >= SLOTS:
            raise ValueError(f"pattern {name!r} leaves the probe's LDS")
        t = torch.tensor(slots, dtype=torch.int32, device=dev)
        for fi, form in enumerate(FORMS):
            rc = lib.fufft_lds_probe(fi, t.data_ptr(), REPS, out.data_ptr(), BLOCKS, None)
            if rc != 0:
                raise RuntimeError(f"fufft_lds_probe({form}, {name}) returned {rc}")
            torch.cuda.synchronize()
            order.append([name, form])
    if order_path:
        order_path.parent.mkdir(parents=True, exist_ok=True)
        order_path.write_text(json.dumps(order))
    return order


def summarize(csv_path: Path, order_path: Path) -> str:
    import csv
    order = json.loads(order_path.read_text())
    per: dict = {}
    for r in csv.DictReader(open(csv_path)):
        if "lds_probe_kernel" not in r["Kernel_Name"]:
            continue
        d = per.setdefault(int(r["Dispatch_Id"]), {})
        d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    ids = sorted(per)
    if len(ids) != len(order):
        raise ValueError(f"{len(ids)} probe dispatches in the trace, {len(order)} in the order file")
    meas: dict = {}
    for i, (name, form) in zip(ids, order):
        meas.setdefault(name, {})[form] = per[i]["SQ_LDS_BANK_CONFLICT"] / (BLOCKS * REPS)
    lines = ["| pattern | " + " | ".join(f"{f}: measured / model" for f in FORMS) + " |",
             "|---|" + "---|" * len(FORMS)]
    for name, by in meas.items():
        cells = [f"{by[f]:g} / {conflict_cycles(PATTERNS[name], f)}" for f in FORMS]
        lines.append(f"| {name} | " + " | ".join(cells) + " |")
    return "\n".join(lines)


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--order", type=Path, help="where the dispatch order is written (run) or read (summarize)")
    ap.add_argument("--summarize", type=Path, help="rocprofv3 counter CSV of a probe run")
    a = ap.parse_args()
    if a.summarize:
        if not a.order:
            sys.exit("--summarize needs --order")
        print(summarize(a.summarize, a.order))
    else:
        order = run(a.order)
        print(f"{len(order)} probe dispatches", flush=True)


if __name__ == "__main__":
    main()
