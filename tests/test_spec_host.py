"""Greedy speculative decoding, host side: the accept rule, the prompt-lookup
drafter and the draft/verify loop's schedule, on the CPU.

Pinned by the reference's own known-answer tests (src/test/test_kernels.f90
test_accept_prefix :1556-1616, test_lookup_draft :1623-1650), run against
both the oracle restatement and the library's host functions
(fg_spec_accept / fg_spec_draft through the C ABI), and by cross-checking
the two on random inputs.
"""
import numpy as np
import pytest

from autoresearch_amd import engine
from oracle import spec as S

IMPLS = {
    "oracle": (S.accept_prefix, lambda ids, p, m, k: S.lookup_draft(ids, p, m, k)),
    "lib": (lambda d, t, k: engine.spec_accept(list(d)[:k], list(t)[:k + 1]),
            engine.spec_draft),
}


@pytest.fixture(params=sorted(IMPLS))
def impl(request):
    if request.param == "lib":
        engine.load_library()
    return IMPLS[request.param]


def test_accept_prefix_table(impl):
    acc, _ = impl
    assert acc([1, 2, 3, 4], [1, 2, 9, 9, 7], 4) == (2, 9)  # partial match
    assert acc([1, 2, 3], [1, 2, 3, 5], 3) == (3, 5)  # all match: bonus row
    assert acc([1, 2], [7, 8, 9], 2) == (0, 7)  # first rejected
    assert acc([], [4], 0) == (0, 4)  # k = 0 is a plain step


def test_accept_prefix_protocol(impl):
    """The reference's protocol simulation: a drafter that agrees except at a
    planted mismatch every 7th window reproduces the target stream exactly,
    committing >= 1 token per pass."""
    acc, _ = impl
    K, NT = 5, 40
    tg = [(j * 7 + 3) % 11 for j in range(1, NT + K + 2)]  # tg(j), j = 1..NT+K+1
    p, buf, npass, ncorr = 1, [], 0, 0
    while len(buf) < NT and p <= NT:
        draft = [tg[p + j - 1 - 1] for j in range(1, K + 1)]
        if p % 7 == 0:
            draft[2] = (draft[2] + 1) % 11
        targ = [tg[p + j - 1 - 1] for j in range(1, K + 2)]
        na, corr = acc(draft, targ, K)
        assert corr == targ[na]
        buf += draft[:na] + [corr]
        ncorr += na < K
        p += na + 1
        npass += 1
    assert len(buf) >= NT
    assert buf == tg[:len(buf)]
    assert ncorr > 0
    assert npass < len(buf)  # drafts were accepted: fewer passes than tokens


def test_lookup_draft_kats(impl):
    _, draft = impl
    ids = [5, 1, 2, 3, 9, 1, 2, 3, 7]
    assert draft(ids, 8, 3, 6) == [9, 1, 2, 3]  # continuation capped at known ids
    assert draft(ids, 8, 3, 2) == [9, 1]  # k truncates
    assert draft([5, 1, 2], 3, 5, 4) == []  # m > p-1: a miss, not a bad read
    assert draft([1, 2, 3, 4, 5, 6], 6, 2, 3) == []  # no earlier occurrence
    assert draft([7, 8, 9, 7, 8, 9], 6, 3, 5) == [7, 8, 9]  # match at position 1


def test_lookup_draft_edges(impl):
    _, draft = impl
    assert draft([4], 1, 2, 3) == []  # a single known id: nothing to match
    # the search window stops at s = p - mm: the suffix never matches itself
    # through an overlapping window, so a run of one id proposes from the
    # window ending mm earlier
    assert draft([3, 3, 3, 3], 4, 2, 8) == [3, 3]
    # the most recent occurrence wins
    assert draft([1, 2, 5, 1, 2, 6, 1, 2], 8, 2, 1) == [6]


def test_lib_matches_oracle_random():
    engine.load_library()
    rng = np.random.default_rng(3)
    for _ in range(3000):
        n = int(rng.integers(1, 14))
        ids = rng.integers(0, 3, n).tolist()
        p = int(rng.integers(1, n + 1))
        m = int(rng.integers(1, 5))
        k = int(rng.integers(0, 6))
        assert engine.spec_draft(ids, p, m, k) == S.lookup_draft(ids, p, m, k)
        kk = int(rng.integers(0, 6))
        d = rng.integers(0, 2, kk).tolist()
        t = rng.integers(0, 2, kk + 1).tolist()
        assert engine.spec_accept(d, t) == S.accept_prefix(d, t, kk)


def test_schedule_worked_example():
    # prompt [1 2 3 1 2]: the last two ids occur at the start, so the first
    # pass proposes [3 1 2] (capped at known ids); all three are accepted and
    # the bonus row commits the fourth id
    out, st = S.spec_schedule([1, 2, 3, 1, 2], [3, 1, 2, 3], k=8, match=2, probe=8,
                              min_acc=0.5)
    assert out == [3, 1, 2, 3]
    assert st == dict(passes=1, accepted=3, proposed=3, plain=0, pauses=0)


def test_schedule_commits_the_stream_and_pauses():
    rng = np.random.default_rng(5)
    for trial in range(200):
        prompt = rng.integers(0, 4, int(rng.integers(1, 12))).tolist()
        stream = rng.integers(0, 4, int(rng.integers(0, 40))).tolist()
        k, match, probe = int(rng.integers(1, 9)), int(rng.integers(1, 4)), int(rng.integers(1, 5))
        min_acc = float(rng.choice([0.0, 0.5, 1.5, 9.0]))
        out, st = S.spec_schedule(prompt, stream, k, match, probe, min_acc)
        assert out == stream
        # every round commits na+1 (pass) or 1 (plain) ids
        assert st["accepted"] + st["passes"] + st["plain"] == len(stream)
        assert st["accepted"] <= st["proposed"] <= k * st["passes"]
        if min_acc == 0.0:
            assert st["pauses"] == 0
    # a window that accepts nothing pauses drafting for `probe` plain rounds
    out, st = S.spec_schedule([0, 0, 0, 0], [1] * 6, k=4, match=2, probe=1, min_acc=0.5)
    assert out == [1] * 6 and st["pauses"] >= 1 and st["plain"] >= 1
