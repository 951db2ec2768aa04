"""LDS bank model of gfx950, as measured on MI355X.

The conv kernels exchange data through LDS with 8-byte accesses
(ds_read2_b64 / ds_write2_b64 / ds_read2st64_b64, and ds_read_b64 or
ds_write_b64 where an offset does not fit the paired form).  Their layouts are
audited (tests/test_lds_audit.py) against this model.

Model (slots are float2 indices, i.e. byte address / 8):

- ``read_b64``: the wavefront is serviced 32 lanes at a time; two lanes of a
  half-wavefront conflict when their slots differ but agree modulo 32.
- ``write_b64``, ``write2_b64``, ``read2_b64``, ``read2st64_b64``: each 8-byte
  access (two for the paired forms) is serviced 16 lanes at a time; two lanes
  of a quarter-wavefront conflict when their slots differ but agree modulo 16.

A group whose most-shared residue holds d distinct slots costs d - 1 extra
cycles; the counter SQ_LDS_BANK_CONFLICT is the sum over groups and accesses.

The model was checked against SQ_LDS_BANK_CONFLICT per instruction for each
lane pattern in PATTERNS and each form in FORMS (one 64-lane workgroup per
pattern and form, many repetitions, rocprofv3 --pmc SQ_LDS_BANK_CONFLICT
SQ_INSTS_LDS SQ_WAVES): profiles/lds_bank_model.md lists measured and
modelled cycles side by side, and test_lds_audit.py checks every row of it.
"""
from __future__ import annotations

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


# ---- 4-byte forms ----------------------------------------------------------------
# The N = 32768 conv (wide.hip) exchanges one float component at a time
# (ds_read_b32 / ds_write_b32 and their paired and st64 forms).  Slots here
# are float indices (byte address / 4).  Measured the same way as the 8-byte
# forms (a one-off probe: one 64-lane workgroup per pattern and form, 256
# repetitions, rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS SQ_WAVES):
#
# - every 4-byte form is serviced 32 lanes at a time over 32 banks; two lanes
#   of a half-wavefront conflict when their slots differ but agree modulo 32;
# - a paired form (ds_read2_b32, ds_write2_b32, ds_read2st64_b32,
#   ds_write2st64_b32) costs its two accesses separately.

FORMS32 = ("read_b32", "write_b32", "read2_b32", "write2_b32", "read2st64_b32", "write2st64_b32")
# second access of the paired forms as the probe issued them, in float slots
SECOND32 = {"read2_b32": 1, "write2_b32": 1, "read2st64_b32": 64, "write2st64_b32": 64}


def _patterns32() -> dict:
    lane = range(64)
    p = {"contiguous": [l for l in lane]}
    for s in (2, 4, 8, 16, 32, 64, 17, 33):
        p[f"stride {s}"] = [s * l for l in lane]
    p["padded by 16 (i + i/16)"] = [l + l // 16 for l in lane]
    p["272 (l/16) + l%16"] = [272 * (l // 16) + l % 16 for l in lane]
    p["16 l + 16 (l/16)"] = [16 * l + 16 * (l // 16) for l in lane]
    p["16 l + l%16 + 16 (l/16)"] = [16 * l + l % 16 + 16 * (l // 16) for l in lane]
    p["two runs of 32, 64 apart"] = [l + 64 * (l // 32) for l in lane]
    return p


PATTERNS32 = _patterns32()

# SQ_LDS_BANK_CONFLICT per instruction of the single forms (read_b32 and
# write_b32 measured alike); the paired forms measured exactly twice these,
# with a second access 1 or 17 floats away, or 64 (st64)
MEASURED32 = {
    "contiguous": 0, "stride 2": 2, "stride 4": 6, "stride 8": 14, "stride 16": 30, "stride 32": 62,
    "stride 64": 62, "stride 17": 0, "stride 33": 0, "padded by 16 (i + i/16)": 2, "272 (l/16) + l%16": 0,
    "16 l + 16 (l/16)": 30, "16 l + l%16 + 16 (l/16)": 0, "two runs of 32, 64 apart": 0,
}


def conflict_cycles32(slots, form: str) -> int:
    """Extra cycles of one 4-byte instruction of `form` whose lanes access `slots`."""
    accesses = [list(slots)]
    if form in SECOND32:
        accesses.append([s + SECOND32[form] for s in slots])
    total = 0
    for acc in accesses:
        for h in range(0, len(acc), 32):
            banks: dict = {}
            for s in acc[h:h + 32]:
                banks.setdefault(s % 32, set()).add(s)
            total += max(len(x) for x in banks.values()) - 1
    return total
