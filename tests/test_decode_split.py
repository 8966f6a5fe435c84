"""Index math of the balanced decode split (DecodeSplit in
pto-wsp_amd/csrc/device/ptowsp_device.h and the wave loop emitted by
emit_decode in pto-wsp_amd/csrc/host/emit.cpp), checked by brute force.

Wave w of W = min(resident waves, T) folds global pages [w*T/W, (w+1)*T/W)
of the T pages of all units laid end to end (so each active wave holds at
least one page); a wave writes the partial of unit u into slot u + w, and unit u's
partials are the slots u + wave_of(pre[u]) .. u + wave_of(pre[u+1]-1).  The
checks: every page is folded exactly once, slots are distinct and below
U + W, each unit's slots are consecutive and as many as the waves that touch
it (the count its completion counter waits for)."""
import numpy as np
import pytest


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


def walk(counts, W):
    """The emitted wave loop: yields (wave, unit, first page, end page)."""
    U = len(counts)
    pre = [0]
    for n in counts:
        pre.append(pre[-1] + n)
    T = pre[U]
    W = min(W, T)  # active waves: each holds at least one page
    for w in range(W):
        s, b = w * T // W, (w + 1) * T // W
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
    pre = np.concatenate([[0], np.cumsum(counts)]).tolist()
    T = pre[-1]
    W = min(W, T)
    seen = [np.zeros(n, dtype=np.int64) for n in counts]
    slots = {}
    per_unit = {}
    for w, u, p0, p1 in walk(counts, W):
        assert 0 <= p0 < p1 <= counts[u]
        seen[u][p0:p1] += 1
        slot = u + w
        assert 0 <= slot < U + W and slot not in slots
        slots[slot] = (w, u)
        per_unit.setdefault(u, []).append(slot)
    for u in range(U):
        assert (seen[u] == 1).all(), u
        if counts[u] == 0:
            assert u not in per_unit
            continue
        wf, wl = wave_of(pre[u], T, W), wave_of(pre[u + 1] - 1, T, W)
        assert per_unit[u] == list(range(u + wf, u + wl + 1)), (u, per_unit[u], wf, wl)
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
