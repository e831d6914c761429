"""CPU restatement of the reference's token sampling (src/lib/sample.f90).

TEST INFRASTRUCTURE ONLY: imported by tests/ to check the device results. The product
library never imports it.

fp32 arithmetic in the reference's order (numpy float32 scalars); ids are
0-based, positions in the reference are 1-based. Functions follow
sample.f90: rand_u01 :15-28, apply_penalties :33-51, apply_rep_penalty
:56-71, apply_windowed_penalties :77-104, block_ngram :109-130,
apply_byte_mask :141-151, sample_next :153-177, sample_top_p :180-233,
sort_desc :236-257, sample_token :260-296.

Pinned by the reference's known answers (src/test/test_kernels.f90
test_sample :677-720, test_valid_mask :1026-1065, test_decode :2180-2233),
by the xorshift64* recurrence restated over Python integers, and by the
sampled distribution against the closed-form softmax / nucleus
probabilities (chi-square, tests/test_sample_host.py). One deliberate
difference: sample_top_p orders equal probabilities by id
(sort_desc_ties_by_id) where the reference's quicksort has its own order;
parity of draws that land inside a run of equal probabilities is unpinned.
"""
from __future__ import annotations

import numpy as np

F = np.float32
MASK64 = (1 << 64) - 1
XS_MULT = 2685821657736338717
HUGE = np.finfo(np.float32).max


def _signed64(x: int) -> int:
    return x - (1 << 64) if x >= (1 << 63) else x


def rand_u01(state: int):
    """xorshift64* step (sample.f90:15-28): returns (u in [0,1) as float32,
    new state). state is a signed int64 value as the reference holds it."""
    x = state & MASK64
    if x == 0:
        x = XS_MULT
    x ^= (x << 13) & MASK64
    x ^= x >> 7  # ishft(x, -7): logical shift
    x ^= (x << 17) & MASK64
    new_state = _signed64(x)
    y = (x * XS_MULT) & MASK64
    u = F((y >> 40) & 0xFFFFFF) / F(16777216.0)
    return F(u), new_state


def apply_penalties(w, gen, ngen, pres, freq):
    V = w.size
    seen = set()
    for i in range(ngen):
        g = int(gen[i])
        if g < 0 or g >= V or g in seen:
            continue
        seen.add(g)
        cnt = sum(1 for j in range(ngen) if int(gen[j]) == g)
        w[g] = F(F(w[g] - F(pres)) - F(F(freq) * F(cnt)))


def apply_rep_penalty(w, gen, ngen, theta):
    V = w.size
    if F(theta) <= F(1.0) or ngen == 0:
        return
    seen = set()
    for i in range(ngen):
        g = int(gen[i])
        if g < 0 or g >= V or g in seen:
            continue
        seen.add(g)
        w[g] = F(w[g] / F(theta))


def apply_windowed_penalties(w, gen, ngen, pres, freq, win, plen):
    V = w.size
    if win <= 0 or ngen == 0:
        return
    start = max(0, ngen - win)
    if abs(F(pres)) > 0 or abs(F(freq)) > 0:
        seen = set()
        for i in range(start, ngen):
            g = int(gen[i])
            if g < 0 or g >= V or g in seen:
                continue
            seen.add(g)
            cnt = sum(1 for j in range(start, ngen) if int(gen[j]) == g)
            w[g] = F(F(w[g] - F(pres)) - F(F(freq) * F(cnt)))
    if abs(F(plen)) > 0 and ngen < win:
        w[0] = F(w[0] - F(F(F(plen) * F(win - ngen)) / F(win)))


def block_ngram(w, gen, ngen, nn):
    """Ban every id that would complete an n-gram already in gen[0:ngen]."""
    if nn < 2 or ngen < nn:
        return
    tail = [int(x) for x in gen[ngen - nn + 1:ngen]]
    for s in range(0, ngen - nn + 1):
        if [int(x) for x in gen[s:s + nn - 1]] == tail:
            t = int(gen[s + nn - 1])
            if 0 <= t < w.size:
                w[t] = F(-HUGE)


def apply_byte_mask(w):
    V = w.size
    ids = np.arange(V)
    keep = (ids < 128) | ((ids >= 256) & (ids < 512))
    w[~keep] = F(-HUGE)


def sort_desc(pr, ox):
    """sort_desc (sample.f90:236-257): Lomuto quicksort, middle pivot, pr
    descending with ox alongside, in place on python lists (the recursion
    kept as an explicit stack of disjoint ranges)."""
    todo = [(0, len(pr))]
    while todo:
        lo, n = todo.pop()
        if n < 2:
            continue
        mid = lo + (n + 1) // 2 - 1
        last = lo + n - 1
        pr[mid], pr[last] = pr[last], pr[mid]
        ox[mid], ox[last] = ox[last], ox[mid]
        pv = pr[last]
        i = lo - 1
        for j in range(lo, last):
            if pr[j] > pv:
                i += 1
                pr[i], pr[j] = pr[j], pr[i]
                ox[i], ox[j] = ox[j], ox[i]
        pr[i + 1], pr[last] = pr[last], pr[i + 1]
        ox[i + 1], ox[last] = ox[last], ox[i + 1]
        todo.append((lo, i + 1 - lo))
        todo.append((i + 2, lo + n - (i + 2)))


def sort_desc_ties_by_id(pr):
    """The descending order sample_top_p uses here: probability descending,
    equal probabilities in id order. It equals sort_desc's permutation
    whenever no two probabilities are equal (tests/test_sample_host.py); the
    reference's quicksort leaves runs of equal values in an order of its own,
    and the quadratic time it takes on long runs (every id but one at zero
    probability, say) is out of reach in Python."""
    ox = sorted(range(len(pr)), key=lambda i: (-float(pr[i]), i))
    return [pr[i] for i in ox], ox


def argmax_first(w) -> int:
    best = 0
    for i in range(1, w.size):
        if w[i] > w[best]:
            best = i
    return best


def sample_top_p(w, temp, topp, state):
    """Returns (0-based id, new state, detail) where detail holds the draw
    and the sorted cumulative sums (for margin checks in tests)."""
    V = w.size
    t = F(temp)
    if t <= 0:
        return argmax_first(w), state, None
    if t < F(1e-6):
        t = F(1e-6)
    m = w[0]
    for i in range(1, V):
        if w[i] > m:
            m = w[i]
    # (w - m) / t overflows to -inf for tiny temperatures, as it does in the
    # reference's single precision; exp then gives 0
    with np.errstate(over="ignore"):
        sc = np.exp(((w - m) / t).astype(np.float32)).astype(np.float32)
    s = F(0.0)
    for i in range(V):
        s = F(s + sc[i])
    pr, ox = sort_desc_ties_by_id([F(sc[i] / s) for i in range(V)])
    if F(topp) >= 1:
        cut = V
    else:
        acc = F(0.0)
        cut = 1
        for k in range(V):
            acc = F(acc + pr[k])
            cut = k + 1
            if acc >= F(topp):
                break
    tot = F(0.0)
    for k in range(cut):
        tot = F(tot + pr[k])
    u01, state = rand_u01(state)
    u = F(u01 * tot)
    acc = F(0.0)
    cums = []
    pick = ox[cut - 1]
    for k in range(cut):
        acc = F(acc + pr[k])
        cums.append(acc)
        if acc >= u:
            pick = ox[k]
            break
    return pick, state, {"u": float(u), "cums": cums, "cut": cut, "total": float(tot)}


def sample_next(logits, temp, topp, pres, freq, rep, pwin, plen, gen, ngen, nblock, state,
                byte_space=False):
    """sample_next (sample.f90:153-177): returns (0-based id, new state,
    detail)."""
    w = np.array(logits, dtype=np.float32).copy()
    gen = [int(x) for x in gen]
    if pwin > 0:
        apply_windowed_penalties(w, gen, ngen, pres, freq, pwin, plen)
    elif abs(F(pres)) > 0 or abs(F(freq)) > 0:
        apply_penalties(w, gen, ngen, pres, freq)
    if F(rep) > F(1.0):
        apply_rep_penalty(w, gen, ngen, rep)
    if nblock >= 2:
        block_ngram(w, gen, ngen, nblock)
    if byte_space:
        apply_byte_mask(w)
    return sample_top_p(w, temp, topp, state)


def sample_token(logits, temp, state):
    """sample_token (sample.f90:260-296): argmax at temp <= 0, else a draw
    from softmax(logits / temp) scanned in id order. Returns (0-based id, new
    state)."""
    w = np.asarray(logits, dtype=np.float32)
    V = w.size
    t = F(temp)
    if t <= 0:
        return argmax_first(w), state
    if t < F(1e-6):
        t = F(1e-6)
    m = w[0]
    for i in range(1, V):
        if w[i] > m:
            m = w[i]
    e = np.exp(((w - m) / t).astype(np.float32)).astype(np.float32)
    s = F(0.0)
    for i in range(V):
        s = F(s + e[i])
    u01, state = rand_u01(state)
    u = F(u01 * s)
    acc = F(0.0)
    for i in range(V):
        acc = F(acc + e[i])
        if acc >= u:
            return i, state
    return V - 1, state
