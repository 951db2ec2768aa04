"""CPU audit of the LDS layouts used by the fused kernels (fufft_plan.hpp).

For every plan (V, N) and every pass, it enumerates the slot each lane touches
for each tap and checks, under the gfx950 bank model measured with
SQ_LDS_BANK_CONFLICT (64 banks x 4 B; an 8-byte access is serviced 32 lanes
at a time, so lanes of an aligned half-wave conflict when their slots agree
modulo 32):

  - the layout is a bijection onto [0, size(N));
  - the padded layout is additive for every pass, phys(base + k*M) =
    phys(base) + phys(k*M), which the kernels rely on when they address taps
    with one register plus immediate offsets;
  - the conflict degree stays within the bound documented for the layout
    (XOR: conflict free everywhere; PAD: at most 2-way);
  - the reference's own swizzle, derived for 32 banks / 16-lane phases, is not
    conflict free under this model (why the layout was re-derived);
  - the per-exchange layouts the kernels use by default are bijections within
    the slot, additive, conflict free, and free of cross-wavefront races.
"""
import itertools

import pytest


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


def degree(slots, lanes=32):
    worst = 1
    for h in range(0, len(slots), lanes):
        banks = {}
        for s in slots[h:h + lanes]:
            banks.setdefault(s % 32, set()).add(s)
        worst = max(worst, max(len(x) for x in banks.values()))
    return worst


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


def test_reference_swizzle_conflicts_on_gfx950():
    """SWZ16 (fufft.cuh:668) targets 32 banks x 16-lane phases; under the
    64-bank, 32-lane model its M = 1 pattern is not conflict free."""
    def swz16(i):
        return i ^ ((i >> 3) & 15) ^ ((i >> 7) & 15)
    n, v = 4096, 16
    worst = max(degree([swz16(p) for p in pos]) for _, pos in lane_sets(n, v))
    assert worst > 1


# column kernels (conv2d.hip): C columns side by side, thread = (L, col) with
# the column fastest, per-column slot skewed by 32 / C float2
COLS = [(256, 8, 16), (512, 8, 16), (1024, 16, 16), (2048, 16, 8)]


@pytest.mark.parametrize("h,v,c", COLS)
def test_column_tiles_conflict_free(h, v, c):
    T = h // v
    slotc = h + h // v + 32 // c
    for (R, M) in plan(h, v):
        for g, k in itertools.product(range(v // R), range(R)):
            addrs = [(tid % c) * slotc + phys_pad(tap_pos(tid // c, g, k, R, M, T), v)
                     for tid in range(c * T)]
            for w0 in range(0, len(addrs), 64):
                assert degree(addrs[w0:w0 + 64]) == 1, (h, v, c, R, M, g, k)
    # without the skew the C columns of a half-wavefront share banks
    addrs = [(tid % c) * (h + h // v) + phys_pad(tap_pos(tid // c, 0, 0, *plan(h, v)[0], T), v)
             for tid in range(64)]
    assert degree(addrs) > 1


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


@pytest.mark.parametrize("v,n", UNSCRAMBLE)
def test_unscramble_targets_and_conflicts(v, n):
    T = n // v
    for L in range(T):
        f = lane_bin(L, n, v)
        for k in range(v):
            assert f + k * T == mixedrev(L * v + k, n, v)
            assert phys_pad(f + k * T, v) == phys_pad(f, v) + phys_pad(k * T, v)
    worst = 1
    for k in range(v):
        pos = [lane_bin(L, n, v) + k * T for L in range(T)]
        if len(pos) < 32:
            pos = [p + r * n for r in range(32 // len(pos)) for p in pos]
        worst = max(worst, degree([phys_pad(p, v) for p in pos]))
    # measured bound of the scattered side; the natural side is pass 0's pattern
    assert worst <= (2 if n <= 4096 and (v, n) != (8, 1024) else 4), worst


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
                if degree(lanes) > 1:
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
