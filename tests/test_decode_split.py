"""Index math of the balanced decode split (DecodeSplit in
pto-wsp_amd/csrc/device/ptowsp_device.h and the wave ranges emitted by
emit_decode in pto-wsp_amd/csrc/host/emit.cpp), checked by brute force.

Units' pages are laid end to end (page prefix pre) and so are their
scheduling costs (cost prefix cpre: a non-empty unit costs its pages plus
UNIT_COST leading positions that hold no page).  Wave w of W = min(resident
waves, TC) owns cost positions [w*TC/W, (w+1)*TC/W), i.e. the pages
[page_at(w*TC/W), page_at((w+1)*TC/W)); a wave writes the partial of unit u
into slot u + w, and unit u's partials are the slots u + wf .. u + wl, wf and
wl the waves of the cost positions of its first and last page.  The checks:
every page is folded exactly once, slots are distinct and below U + W, each
unit's slots are consecutive and as many as the waves that touch it (the
count its completion counter waits for), and the cost split bounds every
wave's pages plus unit starts."""
import numpy as np
import pytest

UNIT_COST = 3


def wave_of(p, T, W):
    return ((p + 1) * W - 1) // T


def unit_of(pre, U, s):
    lo, hi = 0, U
    while hi - lo > 1:
        mid = (lo + hi) >> 1
        if pre[mid] <= s:
            lo = mid
        else:
            hi = mid
    return lo


def cost(n):
    return n + UNIT_COST if n > 0 else 0


def prefixes(counts):
    pre, cpre = [0], [0]
    for n in counts:
        pre.append(pre[-1] + n)
        cpre.append(cpre[-1] + cost(n))
    return pre, cpre


def page_at(pre, cpre, U, v):
    if v >= cpre[U]:
        return pre[U]
    u = unit_of(cpre, U, v)
    return pre[u] + max(0, v - cpre[u] - UNIT_COST)


def walk(counts, W):
    """The emitted wave ranges and DecodeStream's unit walk: yields (wave, unit, first page, end page)."""
    U = len(counts)
    pre, cpre = prefixes(counts)
    TC = cpre[U]
    W = min(W, TC)  # active waves: no empty cost range
    for w in range(W):
        s, b = page_at(pre, cpre, U, w * TC // W), page_at(pre, cpre, U, (w + 1) * TC // W)
        if s >= b:
            continue
        u = unit_of(pre, U, s)
        while True:
            su, eu = pre[u], pre[u + 1]
            e = min(eu, b)
            assert su <= s < eu, (w, u, s)
            yield w, u, s - su, e - su
            s = e
            if s >= b:
                break
            u += 1
            while pre[u + 1] <= s:
                u += 1


def check(counts, W):
    U = len(counts)
    pre, cpre = prefixes(counts)
    TC = cpre[U]
    W = min(W, TC)
    seen = [np.zeros(n, dtype=np.int64) for n in counts]
    slots = {}
    per_unit = {}
    load = {}
    for w, u, p0, p1 in walk(counts, W):
        assert 0 <= p0 < p1 <= counts[u]
        seen[u][p0:p1] += 1
        slot = u + w
        assert 0 <= slot < U + W and slot not in slots
        slots[slot] = (w, u)
        per_unit.setdefault(u, []).append(slot)
        load[w] = load.get(w, 0) + (p1 - p0) + (UNIT_COST if p0 == 0 else 0)
    for u in range(U):
        assert (seen[u] == 1).all(), u
        if counts[u] == 0:
            assert u not in per_unit
            continue
        wf, wl = wave_of(cpre[u] + UNIT_COST, TC, W), wave_of(cpre[u + 1] - 1, TC, W)
        assert per_unit[u] == list(range(u + wf, u + wl + 1)), (u, per_unit[u], wf, wl)
    # a wave's pages plus the units it starts never exceed its cost range
    for w, c in load.items():
        assert c <= (w + 1) * TC // W - w * TC // W + UNIT_COST, (w, c)
    return len(slots)


def test_wave_of_is_the_owner_of_each_page():
    for T in range(1, 60):
        for W in range(1, 70):
            for p in range(T):
                w = wave_of(p, T, W)
                assert w * T // W <= p < (w + 1) * T // W


@pytest.mark.parametrize("seed", range(40))
def test_split_covers_every_page_once(seed):
    rng = np.random.default_rng(seed)
    U = int(rng.integers(1, 300))
    counts = rng.integers(0, 40, size=U)
    counts[rng.random(U) < 0.3] = 0  # empty units
    W = int(rng.integers(1, 800))
    if counts.sum() == 0:
        counts[0] = 1
    check(counts.tolist(), W)


def test_split_edge_cases():
    check([5], 1)
    check([5], 64)            # more waves than pages
    check([0, 0, 3, 0], 7)    # empty units around one
    check([1] * 100, 3)       # many units per wave
    check([1000, 1, 1000], 3072)
    check([0] * 4095 + [17], 3072)
