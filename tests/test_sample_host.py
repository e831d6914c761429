"""Token sampling, the oracle (oracle/sample.py) on the CPU.

Pins: the reference's known answers (src/test/test_kernels.f90 test_sample
:677-720, test_valid_mask :1026-1065, test_decode :2180-2233); the
xorshift64* recurrence restated independently over numpy uint64; windowed
and repetition penalties and the n-gram ban on hand-worked cases; and the
sampled distribution against the closed-form softmax and nucleus
probabilities (chi-square).
"""
import numpy as np
import pytest

from oracle import sample as S

F = np.float32


def test_sample_token_kats():
    lg = np.array([-1.0, 2.0, 0.5, -0.5], np.float32)
    assert S.sample_token(lg, 0.0, 1)[0] == 1  # greedy argmax (position 2)
    st, hits = 42, [0] * 4
    for _ in range(400):
        pos, st = S.sample_token(lg, 1.0, st)
        hits[pos] += 1
    assert sum(h > 0 for h in hits) > 1  # samples spread
    assert hits[1] > 200  # argmax dominates
    assert S.sample_token(lg, 1.0, 7)[0] == S.sample_token(lg, 1.0, 7)[0]  # seeded


def test_decode_kats():
    w = np.zeros(5, np.float32)
    S.apply_penalties(w, [1, 1, 2], 3, 1.0, 0.5)
    assert w[1] == F(-2.0) and w[2] == F(-1.5) and w[0] == w[3] == w[4] == 0
    lg = np.array([0, 1, 2, 3, 4], np.float32)
    # bigram (4,4) seen; tail [4] + t=4 would repeat it: 4 banned, argmax falls to 3
    assert S.sample_next(lg, 0.0, 1.0, 0, 0, 1.0, 0, 0.0, [3, 4, 4], 3, 2, 9)[0] == 3
    assert S.sample_next(lg, 0.0, 1.0, 0, 0, 1.0, 0, 0.0, [3, 4, 4], 3, 0, 9)[0] == 4
    st = 3
    for _ in range(50):  # top-p 0: always the argmax
        pos, st, _ = S.sample_next(lg, 1.0, 0.0, 0, 0, 1.0, 0, 0.0, [], 0, 0, st)
        assert pos == 4
    st, hits = 11, [0] * 5
    for _ in range(200):  # top-p 1 spreads
        pos, st, _ = S.sample_next(lg, 1.0, 1.0, 0, 0, 1.0, 0, 0.0, [], 0, 0, st)
        hits[pos] += 1
    assert hits[4] > 100 and sum(hits[:4]) > 0
    pr = [F(3.0), F(1.0), F(2.0), F(0.5)]
    ox = [0, 1, 2, 3]
    S.sort_desc(pr, ox)
    assert pr == [3.0, 2.0, 1.0, 0.5] and ox == [0, 2, 1, 3]


def test_valid_mask_kats():
    V = 8192
    lg = np.ones(V, np.float32)
    lg[5000] = 100.0
    assert S.sample_next(lg, 0.0, 1.0, 0, 0, 1.0, 0, 0.0, [1], 1, 0, 42)[0] == 5000
    tok = S.sample_next(lg, 0.0, 1.0, 0, 0, 1.0, 0, 0.0, [1], 1, 0, 42, byte_space=True)[0]
    assert tok != 5000 and (tok < 128 or 256 <= tok < 512)
    w = lg.copy()
    w[5000] = 1.0
    S.apply_byte_mask(w)
    assert np.all(w[:128] == 1) and np.all(w[256:512] == 1)
    assert np.all(w[128:256] == -S.HUGE) and np.all(w[512:] == -S.HUGE)


def _xs_numpy(state, n):
    """xorshift64* over numpy uint64 (wrapping), the top 24 bits of the
    scrambled word as u."""
    with np.errstate(over="ignore"):
        x = np.uint64(state & ((1 << 64) - 1))
        if x == 0:
            x = np.uint64(2685821657736338717)
        out = []
        for _ in range(n):
            x ^= x << np.uint64(13)
            x ^= x >> np.uint64(7)
            x ^= x << np.uint64(17)
            y = x * np.uint64(2685821657736338717)
            out.append(int(y >> np.uint64(40)) & 0xFFFFFF)
        return out, int(x)


@pytest.mark.parametrize("seed", [0, 1, 42, 12345, -7, (1 << 62) + 3])
def test_rng_restated(seed):
    want, last = _xs_numpy(seed, 500)
    st = seed
    for w in want:
        u, st = S.rand_u01(st)
        assert u == F(w) / F(16777216.0)
    assert st & ((1 << 64) - 1) == last


def test_rng_uniform():
    st, us = 99, []
    for _ in range(20000):
        u, st = S.rand_u01(st)
        us.append(float(u))
    h, _ = np.histogram(us, bins=20, range=(0, 1))
    chi2 = float(((h - 1000.0) ** 2 / 1000.0).sum())
    assert chi2 < 60  # 19 dof: p ~ 3e-6 at 60


def test_windowed_penalties_and_rep():
    w = np.zeros(6, np.float32)
    # window of 2 over [1, 2, 1, 3]: ids 1 and 3 once each
    S.apply_windowed_penalties(w, [1, 2, 1, 3], 4, 1.0, 0.5, 2, 0.0)
    assert list(w) == [0, -1.5, 0, -1.5, 0, 0]
    w = np.zeros(6, np.float32)
    # window of 8 over 4 ids: counts over all four, and id 0 pays plen * 4 / 8
    S.apply_windowed_penalties(w, [1, 2, 1, 3], 4, 1.0, 0.5, 8, 2.0)
    assert list(w) == [-1.0, -2.0, -1.5, -1.5, 0, 0]
    w = np.array([2.0, -2.0, 4.0, 1.0], np.float32)
    S.apply_rep_penalty(w, [0, 1, 1], 3, 2.0)
    assert list(w) == [1.0, -1.0, 4.0, 1.0]
    w = np.zeros(8, np.float32)
    # trigram ban: tail [5, 6]; [5, 6, 7] and [5, 6, 2] occurred
    S.block_ngram(w, [5, 6, 7, 1, 5, 6, 2, 5, 6], 9, 3)
    assert set(np.nonzero(w)[0].tolist()) == {2, 7}


def _closed_form(lg, temp, topp):
    p = np.exp((lg.astype(np.float64) - lg.max()) / temp)
    p /= p.sum()
    order = sorted(range(lg.size), key=lambda i: (-p[i], i))
    keep, acc = [], 0.0
    for i in order:
        keep.append(i)
        acc += p[i]
        if topp < 1 and acc >= topp:
            break
    q = np.zeros_like(p)
    q[keep] = p[keep]
    return q / q.sum()


@pytest.mark.parametrize("temp,topp", [(1.0, 1.0), (0.6, 1.0), (1.3, 0.7)])
def test_sampled_distribution(temp, topp):
    rng = np.random.default_rng(17)
    lg = rng.normal(0, 1.5, 12).astype(np.float32)
    q = _closed_form(lg, temp, topp)
    st, n = 5, 6000
    hits = np.zeros(lg.size)
    for _ in range(n):
        i, st, _ = S.sample_top_p(lg, temp, topp, st)
        hits[i] += 1
    assert np.all(hits[q == 0] == 0)  # nothing outside the nucleus
    m = q > 0
    exp = q[m] * n
    chi2 = float(((hits[m] - exp) ** 2 / exp).sum())
    assert chi2 < 3 * m.sum() + 30


def test_sort_orders_agree_without_ties():
    rng = np.random.default_rng(4)
    for n in (1, 2, 3, 7, 64, 513):
        pr = [F(x) for x in rng.permutation(n * 3)[:n] / 7.0]  # distinct values
        a, oa = list(pr), list(range(n))
        S.sort_desc(a, oa)
        b, ob = S.sort_desc_ties_by_id(pr)
        assert oa == ob and a == b
    # with ties the two may order equal values differently, never the values
    pr = [F(1.0), F(0.5), F(1.0), F(0.5), F(2.0)]
    a, oa = list(pr), list(range(5))
    S.sort_desc(a, oa)
    b, ob = S.sort_desc_ties_by_id(pr)
    assert a == b and ob == [4, 0, 2, 1, 3]
