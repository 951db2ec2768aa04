"""CPU audit of the LDS layouts used by the fused kernels (fufft_plan.hpp).

For every plan (V, N) and every pass, it enumerates the slot each lane touches
for each tap and checks it under the gfx950 bank model measured with
SQ_LDS_BANK_CONFLICT (tests/lds_bank_model.py, profiles/lds_bank_model.md):
ds_read_b64 is serviced 32 lanes at a time, so lanes of an aligned
half-wavefront conflict when their slots agree modulo 32; each 8-byte access
of ds_write_b64 and of the paired forms the exchanges use (ds_read2_b64,
ds_write2_b64, ds_read2st64_b64) is serviced 16 lanes at a time, so lanes of
an aligned quarter-wavefront conflict when their slots agree modulo 16.
Checked:

  - the layout is a bijection onto [0, size(N));
  - the padded layout is additive for every pass, phys(base + k*M) =
    phys(base) + phys(k*M), which the kernels rely on when they address taps
    with one register plus immediate offsets;
  - the conflict degree stays within the bound documented for the layout
    (XOR: conflict free everywhere; PAD: at most 2-way);
  - the reference's own swizzle, derived for 32 banks / 16-lane phases, is not
    conflict free under this model (why the layout was re-derived);
  - the per-exchange layouts the kernels use by default are bijections within
    the slot, additive, conflict free, and free of cross-wavefront races;
  - the model reproduces every probe measurement and the kernel counters on
    record.
"""
import itertools
import re
from pathlib import Path

import pytest

from tests import lds_bank_model as M
from tests.lds_bank_model import PATTERNS, FORMS, conflict_cycles

ROOT = Path(__file__).resolve().parent.parent


def ilog2(x):
    return x.bit_length() - 1


def phys_xor(i, v):
    lv = ilog2(v)
    hi = 5 - lv
    return i ^ ((i >> lv) & (v - 1)) ^ (((i >> (2 * lv)) & ((1 << hi) - 1)) << lv)


def phys_pad(i, v):
    return i + i // v


def plan(n, v):
    m, lv = ilog2(n), ilog2(v)
    lead = 1 << (m % lv)
    rads = ([lead] if lead > 1 else []) + [v] * (m // lv)
    out, M = [], n
    for r in rads:
        M //= r
        out.append((r, M))
    return out


def tap_pos(L, g, k, R, M, T):
    gidx = L + g * T
    j, b = gidx % M, gidx // M
    return b * R * M + j + k * M


def lane_sets(n, v):
    """(pass, group, k) -> list of logical positions, one per lane"""
    T = n // v
    for (R, M) in plan(n, v):
        G = v // R
        for g, k in itertools.product(range(G), range(R)):
            yield (R, M, g, k), [tap_pos(L, g, k, R, M, T) for L in range(T)]


def degree(slots, lanes=32, mod=32):
    """worst number of distinct slots sharing a residue within a lane group:
    lanes=32, mod=32 for ds_read_b64; lanes=16, mod=16 for the paired forms"""
    worst = 1
    for h in range(0, len(slots), lanes):
        banks = {}
        for s in slots[h:h + lanes]:
            banks.setdefault(s % mod, set()).add(s)
        worst = max(worst, max(len(x) for x in banks.values()))
    return worst


def quarter(slots):
    return degree(slots, 16, 16)


PLANS = [(16, n) for n in (256, 512, 1024, 2048, 4096, 8192, 16384)] + [(8, n) for n in (512, 1024, 2048, 4096)]


@pytest.mark.parametrize("v,n", PLANS)
def test_layouts_are_bijections(v, n):
    assert sorted(phys_xor(i, v) for i in range(n)) == list(range(n))
    pad = [phys_pad(i, v) for i in range(n)]
    assert len(set(pad)) == n and max(pad) < n + n // v


@pytest.mark.parametrize("v,n", PLANS)
def test_pad_layout_is_additive(v, n):
    T = n // v
    for (R, M), g in ((rm, g) for rm in plan(n, v) for g in range(v // rm[0])):
        for L in range(T):
            base = tap_pos(L, g, 0, R, M, T)
            for k in range(R):
                assert phys_pad(base + k * M, v) == phys_pad(base, v) + phys_pad(k * M, v), (R, M, L, g, k)


@pytest.mark.parametrize("v,n", PLANS)
def test_conflict_degree(v, n):
    for key, pos in lane_sets(n, v):
        if len(pos) < 32:          # transforms narrower than a half-wave sit side by side
            stride = n
            reps = 32 // len(pos)
            pos = [p + r * stride for r in range(reps) for p in pos]
        assert degree([phys_xor(p, v) for p in pos]) == 1, ("xor", key)
        assert degree([phys_pad(p, v) for p in pos]) <= 2, ("pad", key)
        assert quarter([phys_xor(p, v) for p in pos]) == 1, ("xor", key)
        assert quarter([phys_pad(p, v) for p in pos]) <= 2, ("pad", key)


def test_reference_swizzle_conflicts_on_gfx950():
    """SWZ16 (fufft.cuh:668) targets 32 banks x 16-lane phases; under the
    64-bank, 32-lane model its M = 1 pattern is not conflict free."""
    def swz16(i):
        return i ^ ((i >> 3) & 15) ^ ((i >> 7) & 15)
    n, v = 4096, 16
    worst = max(degree([swz16(p) for p in pos]) for _, pos in lane_sets(n, v))
    assert worst > 1


# column kernels (conv2d.hip): C columns side by side, thread = (L, col) with
# the column fastest, per-column slot skewed by 16 / C float2.  Their
# exchanges are paired ds_read2_b64 / ds_write2_b64, so the quarter-wavefront
# rule applies.
COLS = [(256, 8, 16), (512, 8, 16), (1024, 16, 16), (2048, 16, 8)]


def column_cost(h, v, c, slotc):
    """conflict cycles per wavefront of one pass over every tap, paired forms"""
    T = h // v
    total = 0
    for (R, M) in plan(h, v):
        for g, k in itertools.product(range(v // R), range(R)):
            addrs = [(tid % c) * slotc + phys_pad(tap_pos(tid // c, g, k, R, M, T), v)
                     for tid in range(c * T)]
            for w0 in range(0, len(addrs), 64):
                total += conflict_cycles(addrs[w0:w0 + 64], "write_b64")
    return total / (c * T // 64)


@pytest.mark.parametrize("h,v,c", COLS)
def test_column_tiles_conflict_free(h, v, c):
    T = h // v
    slotc = h + h // v + 16 // c
    for (R, M) in plan(h, v):
        for g, k in itertools.product(range(v // R), range(R)):
            addrs = [(tid % c) * slotc + phys_pad(tap_pos(tid // c, g, k, R, M, T), v)
                     for tid in range(c * T)]
            for w0 in range(0, len(addrs), 64):
                assert quarter(addrs[w0:w0 + 64]) == 1, (h, v, c, R, M, g, k)
    # the earlier skew of 32 / C is conflict-free only for ds_read_b64
    assert column_cost(h, v, c, h + h // v + 32 // c) > 0


def test_column_kernel_counter_matches_the_model():
    """rocprofv3 measured 256 conflict cycles per wavefront in the 512-row
    column conv (and 128 in the column apply, which runs half the passes)
    with the 32 / C skew, and 0 with 16 / C (profiles/lds_bank_model.md).
    The conv kernel scatters and gathers every pass's taps in both
    directions: 4 tap sets per direction for 3 passes."""
    h, v, c = 512, 8, 16
    per_pass_set = column_cost(h, v, c, h + h // v + 32 // c) / len(plan(h, v))
    assert per_pass_set * 8 == 256
    assert column_cost(h, v, c, h + h // v + 16 // c) == 0


# exchange_in_wave (fufft_plan.hpp): the exchange between pass p and p + 1 may
# use a wavefront fence instead of the workgroup barrier.  Brute force: every
# position a lane writes in pass p is read in pass p + 1 by a lane of the same
# wavefront (and, for WAR, every position a wavefront reads in pass p + 1 was
# written by that wavefront), whenever the predicate says so.
def exchange_in_wave(n, v, p, wl):
    T = n // v
    rads = plan(n, v)
    if T <= wl:
        return True
    (R, M), (R2, _) = rads[p], rads[p + 1]
    return M <= wl and v // R == 1 and v // R2 == 1


def owners(n, v, p):
    T = n // v
    R, M = plan(n, v)[p]
    own = {}
    for L in range(T):
        for g in range(v // R):
            for k in range(R):
                own[tap_pos(L, g, k, R, M, T)] = L
    return own


WAVE_CASES = [(16, n, 64) for n in (256, 512, 1024, 2048, 4096, 8192, 16384)] + \
             [(8, n, 64) for n in (512, 1024, 2048, 4096, 8192)] + \
             [(8, 256, 4), (8, 512, 4), (16, 1024, 4), (16, 2048, 8)]


@pytest.mark.parametrize("v,n,wl", WAVE_CASES)
def test_wave_local_exchanges(v, n, wl):
    rads = plan(n, v)
    local = 0
    for p in range(len(rads) - 1):
        if not exchange_in_wave(n, v, p, wl):
            continue
        local += 1
        a, b = owners(n, v, p), owners(n, v, p + 1)
        for pos, L in a.items():
            assert b[pos] // wl == L // wl, (n, v, wl, p, pos)
    # the plans that matter do drop barriers: R8 4096 keeps 1 of 3 per direction
    if (v, n, wl) == (8, 4096, 64):
        assert local == 2


# digit order <-> natural order exchange (digit_to_natural / natural_to_digit,
# fufft_plan.hpp): lane L writes slot L*V + k to bin lane_bin(L) + k*T and reads
# bins L + q*T.  The kernel relies on lane_bin being the plan's digit reversal
# restricted to the lane digits, and on the padded layout staying additive.
def lane_bin(L, n, v):
    f, w = 0, 1
    for (R, M) in plan(n, v)[:-1]:
        f += ((L // (M // v)) % R) * w
        w *= R
    return f


def mixedrev(s, n, v):
    f, w = 0, 1
    for (R, M) in plan(n, v):
        f += ((s // M) % R) * w
        w *= R
    return f


UNSCRAMBLE = PLANS + [(8, 8192)]


def unscramble_moves(n, v):
    """UnscrambleLds (fufft_plan.hpp): (source bit, target bit) pairs.  Lane
    bit b lands on bin bit bin_bit(b); the high ones are copied onto the bits
    0-3 the bin does not already vary, in order."""
    pl = plan(n, v)

    def bin_bit(b):
        w = 0
        for (R, M) in pl[:-1]:
            d, r = ilog2(M // v), ilog2(R)
            if d <= b < d + r:
                return w + b - d
            w += r
        return -1
    bits = [bin_bit(b) for b in range(4)]
    free = [t for t in range(4) if t not in bits]
    return [(s, free.pop(0)) for s in bits if s >= 4]


def phys_unscramble(i, moves):
    x = 0
    for s, d in moves:
        x |= ((i >> s) & 1) << d
    return i ^ x


@pytest.mark.parametrize("v,n", UNSCRAMBLE)
def test_unscramble_targets_and_conflicts(v, n):
    T = n // v
    mv = unscramble_moves(n, v)
    ph = [phys_unscramble(i, mv) for i in range(n)]
    assert sorted(ph) == list(range(n))                       # bijection within the slot
    for L in range(T):
        f = lane_bin(L, n, v)
        for k in range(v):
            assert f + k * T == mixedrev(L * v + k, n, v)
            assert phys_unscramble(f + k * T, mv) == phys_unscramble(f, mv) + k * T
            assert phys_unscramble(L + k * T, mv) == phys_unscramble(L, mv) + k * T
    # both sides conflict-free for the paired forms (quarter-wavefront rule),
    # where the padded layout was not (128 cycles per wavefront measured for
    # the radix-8 N = 4096 C2C, test_model_reproduces_kernel_counters)
    reps = max(1, 64 // T)
    for k in range(v):
        for side in ([lane_bin(L, n, v) + k * T for L in range(T)], [L + k * T for L in range(T)]):
            pos = [t * (n + n // v) + phys_unscramble(p, mv) for t in range(reps) for p in side]
            assert quarter(pos) == 1, (k, side[:4])


# ---- per-exchange layouts (XchgLds, fufft_plan.hpp) -------------------------------------
# Exchange e uses phys = i + Mb * (i // (V * Mb)), Mb = the stride of the first
# wavefront-private pass (M <= 64) after the exchange.  A pass gathers from
# exchange e - 1 and scatters into exchange e with no barrier in between, so
# beyond conflicts and additivity the audit checks by brute force that no
# wavefront's writes land on slots another wavefront still has to read, and
# that exchanges synchronised by a wavefront fence are read only by their
# writers.
def xchg_params(pl, e, v, wl=64):
    q = e + 1
    while pl[q][1] > wl:
        q += 1
    return v * pl[q][1], pl[q][1]


def xchg_phys(i, ma, mb):
    return i + mb * (i // ma)


def xchg_naive(pl, e, v, wl=64):
    """(M_e, M_{e+1}): conflict free too, but races after a pass spanning wavefronts"""
    return pl[e][1], pl[e + 1][1]


def xchg_problems(n, v, rule, wl=64):
    pl = plan(n, v)
    T, NP = n // v, len(pl)
    lay = [rule(pl, e, v) for e in range(NP - 1)]
    waves = max(1, T // wl)
    out = []

    def slots(p, e, w):
        R, M = pl[p]
        lanes = range(w * wl, min(T, (w + 1) * wl)) if T > wl else range(T)
        return {xchg_phys(tap_pos(L, g, k, R, M, T), *lay[e])
                for L in lanes for g in range(v // R) for k in range(R)}

    for e in range(NP - 1):
        ph = [xchg_phys(i, *lay[e]) for i in range(n)]
        if len(set(ph)) != n or max(ph) >= n + n // v:
            out.append(("bijection / slot size", e))
        for p in (e, e + 1):
            R, M = pl[p]
            for g, k in itertools.product(range(v // R), range(R)):
                lanes = []
                for wl_i in range(64):
                    t, L = divmod(wl_i, T) if T < 64 else (0, wl_i)
                    lanes.append(t * (n + n // v) + xchg_phys(tap_pos(L, g, k, R, M, T), *lay[e]))
                if degree(lanes) > 1 or quarter(lanes) > 1:
                    out.append(("conflict", e, p, g, k))
                for L in range(T):
                    base = tap_pos(L, g, 0, R, M, T)
                    if xchg_phys(base + k * M, *lay[e]) != xchg_phys(base, *lay[e]) + xchg_phys(k * M, *lay[e]):
                        out.append(("not additive", e, p, g, k))
                        break
    for p in range(1, NP - 1):                    # gather (e = p - 1) -> scatter (e = p), no barrier
        for w in range(waves):
            written = slots(p, p, w)
            for w2 in range(waves):
                if w2 != w and written & slots(p, p - 1, w2):
                    out.append(("clobbers another wavefront's input", p, w, w2))
    for e in range(NP - 1):
        if T > wl and exchange_in_wave(n, v, e, wl):
            for w in range(waves):
                if not slots(e + 1, e, w) <= slots(e, e, w):
                    out.append(("fence-only exchange read across wavefronts", e, w))
    return out


XCHG_PLANS = [(16, n) for n in (256, 512, 1024, 2048, 4096, 8192, 16384)] + \
             [(8, n) for n in (512, 1024, 2048, 4096, 8192)]


@pytest.mark.parametrize("v,n", XCHG_PLANS)
def test_exchange_layouts(v, n):
    assert xchg_problems(n, v, xchg_params) == []


@pytest.mark.parametrize("v,n", [(8, 8192), (16, 8192), (16, 16384)])
def test_exchange_layouts_audit_catches_the_race(v, n):
    """Switching layouts inside a pass that spans wavefronts races: the
    per-exchange (M_e, M_{e+1}) rule fails the audit exactly where it gave
    wrong results on the GPU at full batch (radix 8, N = 8192)."""
    kinds = {x[0] for x in xchg_problems(n, v, xchg_naive)}
    assert kinds == {"clobbers another wavefront's input"}


# ---- the model against its measurements --------------------------------------------------
def test_bank_model_reproduces_the_probe():
    """Every row of the committed probe summary: measured == model."""
    text = (ROOT / "profiles" / "lds_bank_model.md").read_text()
    rows = 0
    for line in text.splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) != 1 + len(FORMS) or cells[0] not in PATTERNS:
            continue
        rows += 1
        for form, cell in zip(FORMS, cells[1:]):
            measured, model = (float(x) for x in cell.split("/"))
            assert model == conflict_cycles(PATTERNS[cells[0]], form), (cells[0], form)
            assert measured == model, (cells[0], form, measured, model)
    assert rows == len(PATTERNS)


def test_model_reproduces_kernel_counters():
    """Counters on record: radix-8 N = 4096 conv with the single padded
    layout, 192 cycles per wavefront; natural-order C2C forward at N = 4096
    (per-exchange layouts for the DIF, padded digit-to-natural exchange), 128.
    Every exchange instruction of both kernels is a paired form."""
    n, v = 4096, 8
    T, pl = n // v, plan(n, v)

    def tapset(R, M, g, k, phys):
        return [phys(tap_pos(L, g, k, R, M, T)) for L in range(T)]

    def cost(slots):
        return sum(conflict_cycles(slots[w:w + 64], "write_b64") for w in range(0, len(slots), 64)) / (T // 64)

    pad = lambda i: phys_pad(i, v)
    conv = 0
    for e in range(len(pl) - 1):
        for p in (e, e + 1):
            R, M = pl[p]
            conv += sum(cost(tapset(R, M, g, k, pad)) for g in range(v // R) for k in range(R))
    assert 2 * conv == 192                    # forward and inverse
    # C2C: the DIF exchanges cost nothing (per-exchange layouts); the unscramble
    # scatters slot L*V + k to bin lane_bin(L) + k*T and gathers bins L + q*T
    scat = sum(cost([pad(lane_bin(L, n, v) + k * T) for L in range(T)]) for k in range(v))
    gath = sum(cost([pad(L + q * T) for L in range(T)]) for q in range(v))
    assert scat + gath == 128


# ---- two outer levels in one pass (large.hip: outer2_kernel) -------------------------------
# 256 threads, tid = jj + 16 * hi; slot(k1, k2, jj) = k1 * 272 + k2 * 16 + jj.
# Forward: threads (jj, k2 = hi) write slot(k1, hi, jj) for every k1, then
# threads (jj, k1 = hi) read slot(hi, k2, jj) for every k2; the inverse swaps
# the roles.  Both sides must be conflict-free under both bank rules.
def outer2_slot(k1, k2, jj):
    return k1 * 272 + k2 * 16 + jj


def test_outer2_exchange_conflict_free():
    sides = {
        "k2 fixed per thread, loop k1": lambda tid, q: outer2_slot(q, tid >> 4, tid & 15),
        "k1 fixed per thread, loop k2": lambda tid, q: outer2_slot(tid >> 4, q, tid & 15),
    }
    for name, slot in sides.items():
        for q in range(16):
            addrs = [slot(tid, q) for tid in range(256)]
            assert len(set(addrs)) == 256
            for w0 in range(0, 256, 64):
                wave = addrs[w0:w0 + 64]
                assert conflict_cycles(wave, "read_b64") == 0, (name, q)
                assert conflict_cycles(wave, "write_b64") == 0, (name, q)
    # without the 16-slot skew per k1 block the half-wavefront rule fails
    flat = [(tid >> 4) * 256 + q * 16 + (tid & 15) for q in (0,) for tid in range(64)]
    assert conflict_cycles(flat, "read_b64") > 0


# ---- the N = 32768 conv's float exchanges (wide.hip) ---------------------------------

def test_b32_model_reproduces_the_probe():
    """The 4-byte rule (32 lanes, 32 banks, paired forms per access) gives
    every measured count of the probe."""
    for name, slots in M.PATTERNS32.items():
        for form in M.FORMS32:
            want = M.MEASURED32[name] * (2 if form in M.SECOND32 else 1)
            assert M.conflict_cycles32(slots, form) == want, (name, form)


WIDE_N, WIDE_V = 32768, 32
WIDE_T = WIDE_N // WIDE_V
WIDE_RADICES = [8, 16, 16, 16]          # LEAD 8, then radix 16 at two groups per lane


def _wide_stride(p):
    m = WIDE_N
    for r in WIDE_RADICES[:p + 1]:
        m //= r
    return m


def _wide_taps(p, lane, g):
    """positions of group g of pass p for `lane` (gidx = L + g T, taps b R M + j + k M)"""
    r, m = WIDE_RADICES[p], _wide_stride(p)
    gidx = lane + g * WIDE_T
    return [(gidx // m) * r * m + gidx % m + k * m for k in range(r)]


def _pad16(i):
    return i + (i >> 4)


def _pad256(i):
    return i + ((i >> 8) << 4)


def _wide_private(p):
    """the kernel's rule: both passes at M <= 64 with the same radix"""
    return _wide_stride(p) <= 64 and _wide_stride(p + 1) <= 64 and WIDE_RADICES[p] == WIDE_RADICES[p + 1]


def test_wide_private_exchange_rule_matches_brute_force():
    for p in range(len(WIDE_RADICES) - 1):
        private = True
        for w in range(WIDE_T // 64):
            a = {x for lane in range(64 * w, 64 * w + 64) for g in range(WIDE_V // WIDE_RADICES[p])
                 for x in _wide_taps(p, lane, g)}
            b = {x for lane in range(64 * w, 64 * w + 64) for g in range(WIDE_V // WIDE_RADICES[p + 1])
                 for x in _wide_taps(p + 1, lane, g)}
            private &= a == b
        assert private == _wide_private(p), p


def _wide_conflicts(layout_of):
    """conflict cycles per wavefront over a transform: every exchange, both
    sides, both components, forward and inverse (single 4-byte accesses)"""
    total = 0
    for p in range(len(WIDE_RADICES) - 1):
        lay = layout_of(p)
        for side in (p, p + 1):
            for g in range(WIDE_V // WIDE_RADICES[side]):
                for k in range(WIDE_RADICES[side]):
                    for w in (0, 5, WIDE_T // 64 - 1):          # every wavefront has the same pattern
                        slots = [lay(_wide_taps(side, lane, g)[k]) for lane in range(64 * w, 64 * w + 64)]
                        c = M.conflict_cycles32(slots, "read_b32")
                        if w == 0:
                            first = c
                        assert c == first
                    total += first * 2 * 2
    return total


def test_wide_layouts_conflict_free_and_old_layout_matches_counter():
    """Pad256 on the cross-wavefront exchanges, Pad16 on the private one: no
    conflict cycle.  Pad16 everywhere (the first build) gives the 768 cycles
    per wavefront that rocprofv3 counted on it."""
    assert _wide_conflicts(lambda p: _pad16 if _wide_private(p) else _pad256) == 0
    assert _wide_conflicts(lambda p: _pad16) == 768


def test_wide_layouts_keep_wavefront_ranges():
    """Both layouts put the 1024-aligned block c of positions inside slots
    [1088c, 1088c + 1088): a private pass that reads one layout and writes the
    other never reaches another wavefront's slots; and both fit the buffer."""
    size = WIDE_N + WIDE_N // 16
    for c in range(WIDE_N // 1024):
        for lay in (_pad16, _pad256):
            s = [lay(i) for i in range(1024 * c, 1024 * c + 1024)]
            assert len(set(s)) == 1024 and min(s) >= 1088 * c and max(s) < 1088 * (c + 1) <= size
    # every wavefront's positions of the private passes form whole 1024-blocks
    for w in range(WIDE_T // 64):
        pos = {x for lane in range(64 * w, 64 * w + 64) for g in range(2) for x in _wide_taps(3, lane, g)}
        blocks = {x // 1024 for x in pos}
        assert len(pos) == 1024 * len(blocks)


def test_wide_layouts_additive():
    """the kernel addresses a tap as layout(base) + layout(k M)"""
    for p in range(len(WIDE_RADICES) - 1):
        lay = _pad16 if _wide_private(p) else _pad256
        for side in (p, p + 1):
            m = _wide_stride(side)
            for lane in (0, 1, 17, 63, 64, 515, WIDE_T - 1):
                for g in range(WIDE_V // WIDE_RADICES[side]):
                    taps = _wide_taps(side, lane, g)
                    assert all(lay(t) == lay(taps[0]) + lay(k * m) for k, t in enumerate(taps))
