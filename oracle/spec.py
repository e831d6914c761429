"""CPU restatement of greedy speculative decoding (temperature 0).

TEST INFRASTRUCTURE ONLY: imported by tests/ to check the device results. The product
library never imports it.

Follows src/lib/fortran_spec.f90 (accept_prefix :41-52, lookup_draft
:62-92) and the draft/verify/commit loop with its sliding-window controller
in src/app/chat_text.f90:293-422. Indices here are 0-based; `p` keeps the
reference's meaning, the number of known tokens ids[0:p], so the pending
token is ids[p-1] and the cache holds p-1 positions.

Pinned by the reference's own known-answer tests (src/test/test_kernels.f90
test_accept_prefix :1556-1616, test_lookup_draft :1623-1650) and, for the
loop, by the invariant the reference asserts (src/app/spec_bench.f90:165-171):
the committed stream equals the target's plain greedy stream.
"""
from __future__ import annotations

import numpy as np


def accept_prefix(draft, targmax, k: int):
    """src/lib/fortran_spec.f90:41-52: the longest prefix of draft[0:k] equal
    to targmax, and the target token right after it (targmax[n_accept])."""
    n = 0
    while n < k and draft[n] == targmax[n]:
        n += 1
    return n, targmax[n]


def lookup_draft(ids, p: int, m: int, k: int):
    """src/lib/fortran_spec.f90:62-92: the continuation (at most k ids, capped
    at known ids) of the most recent earlier occurrence of the last
    mm = min(m, p-1) ids of ids[0:p]. Candidate match ends s run from p-mm
    down to mm (1-based), the window ids(s-mm+1:s) against ids(p-mm+1:p)."""
    mm = min(m, p - 1)
    if mm < 1:
        return []
    tail = list(ids[p - mm:p])
    for s in range(p - mm, mm - 1, -1):  # 1-based end position of the window
        if list(ids[s - mm:s]) == tail:
            kk = min(k, p - s)
            return [int(x) for x in ids[s:s + kk]]
    return []


def spec_schedule(prompt, stream, k: int, match: int, probe: int, min_acc: float):
    """Replay src/app/chat_text.f90:293-422 for a target whose greedy
    continuation of `prompt` is `stream` (every verification row's argmax is
    then the stream's token at that position, which is exactly what the
    accept rule commits). Returns the committed ids and the loop's counters:
    passes (verification rounds), accepted, proposed (sum of clamped k_eff),
    plain (plain steps), pauses (controller switches to plain)."""
    ids = [int(x) for x in prompt] + [-1] * len(stream)
    ntot = len(ids)
    full = [int(x) for x in prompt] + [int(x) for x in stream]
    pp = len(prompt)
    mode_spec, nplain_left = True, 0
    npass_w = nacc_w = 0
    st = dict(passes=0, accepted=0, proposed=0, plain=0, pauses=0)
    while pp < ntot:
        round_spec = mode_spec
        draft = []
        if round_spec:
            draft = lookup_draft(ids, pp, match, k)
            if not draft:
                round_spec = False
        if round_spec:
            keff = len(draft)
            if pp + keff > ntot:
                keff = max(0, ntot - pp)
            # rows of the verification pass: target tokens for pp .. pp+keff;
            # the last row can predict position ntot, past the stream, and is
            # then never committed (the clamp below)
            targ = full[pp:pp + keff + 1]
            targ += [-1] * (keff + 1 - len(targ))
            na, corr = accept_prefix(draft, targ, keff)
            if pp + na + 1 > ntot:
                na = ntot - pp - 1
                corr = targ[na]
            ids[pp:pp + na] = draft[:na]
            ids[pp + na] = corr
            pp += na + 1
            npass_w += 1
            nacc_w += na
            st["passes"] += 1
            st["accepted"] += na
            st["proposed"] += keff
        else:
            ids[pp] = full[pp]
            pp += 1
            st["plain"] += 1
        if mode_spec:
            if npass_w >= probe:
                # single precision, as the reference compares real(sp) values
                if np.float32(nacc_w) < np.float32(min_acc) * np.float32(npass_w):
                    mode_spec = False
                    nplain_left = probe
                    st["pauses"] += 1
                npass_w = nacc_w = 0
        else:
            nplain_left -= 1
            if nplain_left <= 0:
                mode_spec = True
                npass_w = nacc_w = 0
    return ids[len(prompt):], st
