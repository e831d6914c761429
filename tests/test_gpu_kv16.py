"""The bf16 KV cache (fg_kv_create_ex with FG_KV_BF16) on the GPU.

The reference's cache is fp32 (src/lib/fortran_kv.f90:9-12); a bf16 cache
rounds K and V (RNE) where they are stored, so attention reads the rounded
values. Bars: layer 0's cache rows, whose inputs nothing rounded, are
exactly the bf16 rounding of the fp32 cache's rows; logits within
2e-3 x max|logit| of the fp32 oracle; greedy ids equal the oracle's, or the
first differing step is one whose oracle top-2 logit margin is a near-tie
(below 2 x the logit error bar), and the flip is recorded with its margin.
"""
import numpy as np
import pytest

from autoresearch_amd import engine
from autoresearch_amd.weights import D12, Dims, rope_tables, seeded_weights, uniform_ids
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 2e-3
SMALL = Dims(n_layer=2, d_model=128, n_head=2, n_kv_head=1, head_dim=64, vocab=512)
SMALL_MHA = Dims(n_layer=2, d_model=256, n_head=2, n_kv_head=2, head_dim=128, vocab=1024)
GQA5 = Dims(n_layer=2, d_model=640, n_head=5, n_kv_head=1, head_dim=128, vocab=1024)


def record(name, **kv):
    print(name, kv, flush=True)


def relerr(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / np.max(np.abs(b)))


def bf16_round(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def model(d, seed, n):
    m = engine.Model(d, stacks=seeded_weights(d, seed))
    c, s = rope_tables(n, d.head_dim)
    m.set_rope(c.reshape(-1), s.reshape(-1))
    return m, c.reshape(-1), s.reshape(-1)


@pytest.mark.parametrize("d", [SMALL, SMALL_MHA, GQA5], ids=["gqa2", "mha", "gqa5"])
@pytest.mark.parametrize("chunk", [True, False], ids=["chunk", "steps"])
def test_layer0_rows_are_rounded_fp32_rows(d, chunk):
    T = 21
    m, _, _ = model(d, 5, T)
    ids = uniform_ids(9, T, d.vocab)
    caches = []
    for bf in (False, True):
        kv = m.kv(1, T, bf16=bf)
        if chunk:
            kv.step_multi(ids)
        else:
            for t in range(T):
                kv.step(ids[t:t + 1])
        caches.append(kv.read())
        kv.close()
    n0 = T * d.n_kv_head * d.head_dim  # layer 0 of a B=1 cache
    for t32, t16 in zip(caches[0], caches[1]):
        assert np.array_equal(t16[:n0], bf16_round(t32[:n0]))
        # later layers: close to the fp32 cache (their inputs saw rounded K/V)
        assert relerr(t16[n0:], t32[n0:]) < 2e-2
    m.close()


@pytest.mark.parametrize("d", [SMALL, GQA5], ids=["gqa2", "gqa5"])
def test_bf16_cache_chunks_equal_steps(d):
    """Chunked prefill and per-token steps read the same rounded cache."""
    T = 19
    m, _, _ = model(d, 6, T)
    ids = uniform_ids(10, T, d.vocab)
    kv = m.kv(1, T, bf16=True)
    lg_c, _ = kv.step_multi(ids)
    kv.len = 0
    lg_s = np.stack([kv.step(ids[t:t + 1])[0][0] for t in range(T)])
    assert relerr(lg_s, lg_c[0]) < 1e-3
    kv.close()
    m.close()


def test_bf16_cache_d12_decode_vs_oracle():
    """The B=1 decode workload (16-id prompt, 32 steps) on a bf16 cache
    against the fp32 oracle."""
    d = D12
    m, c, s = model(d, 1234, 48)
    prompt = uniform_ids(42, 16, d.vocab)
    ref_ids, ref_lg = O.greedy_decode(prompt, seeded_weights(d, 1234), d, 32, c, s, maxT=48)
    kv = m.kv(1, 48, bf16=True)
    kv.step_multi(prompt[None, :-1], want_logits=False)
    ids, lg = kv.decode_greedy(prompt[-1:], 32, want_logits=True)
    e = relerr(lg[:, 0], ref_lg)
    srt = np.sort(ref_lg, -1)
    marg = srt[:, -1] - srt[:, -2]
    diff = np.nonzero(ids[:, 0] != ref_ids)[0]
    first = int(diff[0]) if diff.size else -1
    record("bf16_cache_greedy_d12", relerr=e, first_flip=first,
           margin_at_flip=float(marg[first]) if first >= 0 else None,
           min_top2_margin=float(marg.min()))
    assert e < TOL
    if first >= 0:
        assert marg[first] < 2 * 2 * TOL * np.abs(ref_lg).max()
    kv.close()
    m.close()


def test_batched_bf16_chunks_merged():
    """B=96 at the small MHA dims over a 1152-position bf16 cache (9 blocks
    of 128, 8 per workgroup) runs the looped decode attention on 8
    wavefronts of 256-position blocks, split into two chunks per sequence
    and head that a merge combines; the fp32 cache at the same shape runs
    the single-block kernel over 9 chunks. Layer 0's appended rows are
    exactly the bf16 rounding of the fp32 ones; the step's logits agree
    within the bar, and every id matches but at near-ties."""
    d, B, P, maxT, n = SMALL_MHA, 96, 1000, 1152, 1
    m, c, s = model(d, 8, maxT)
    ids = uniform_ids(23, B * P, d.vocab).reshape(B, P)
    out = []
    for bf in (False, True):
        kv = m.kv(B, maxT, bf16=bf)
        kv.step_multi(ids[:, :-1], want_logits=False)
        nxt, lg = kv.decode_greedy(ids[:, -1], n, want_logits=True)
        out.append((nxt, lg, kv.read()))
        kv.close()
    n0 = B * maxT * d.n_kv_head * d.head_dim
    for t32, t16 in zip(out[0][2], out[1][2]):
        assert np.array_equal(t16[:n0], bf16_round(t32[:n0]))
    (i32, l32, _), (i16, l16, _) = out
    e = relerr(l16, l32)
    srt = np.sort(l32[0], -1)
    flips = np.flatnonzero(i16[0] != i32[0])
    record("bf16_chunks_merged", relerr=e, first_step_flips=flips.tolist())
    assert e < TOL
    assert np.all(srt[flips, -1] - srt[flips, -2] < 2 * TOL * np.abs(l32).max())
    m.close()


def test_batched_qkv_fold_gqa_vs_single_rows():
    """B=40 sequences of the 5:1 GQA shape (5 query heads over one KV head,
    head_dim 128) on a bf16 cache, 400-id prompts: 200 (sequence, head)
    rows take the looped decode attention (3 blocks of 128 positions per
    workgroup, 2 chunks and a merge), which also finishes the QKV's split-K
    sums (five workgroups per KV head fold the query, one of them appends
    k/v). One plain step and two graph-replayed steps, against each
    sequence decoded alone (single-row GEMV path, no fold): the appended
    layer-0 rows within one bf16 unit (the two paths sum the projection in
    different orders; elements near zero within 1e-5 of the row's largest),
    the logits within the bar, ids equal but at near-ties."""
    d, B, P, n = GQA5, 40, 400, 2
    maxT = P + 1 + n
    m, _, _ = model(d, 11, maxT)
    prompts = uniform_ids(29, B * P, d.vocab).reshape(B, P)
    kv = m.kv(B, maxT, bf16=True)
    kv.step_multi(prompts[:, :-1], want_logits=False)
    lg0, nxt = kv.step(prompts[:, -1])
    ids, lg = kv.decode_greedy(nxt, n, want_logits=True)
    kb, vb = kv.read()
    kv.close()
    got_ids = np.vstack([nxt[None, :], ids])              # [n+1, B]
    got_lg = np.concatenate([lg0[None], lg])               # [n+1, B, V]
    kvd = d.n_kv_head * d.head_dim
    worst, flips = 0.0, []
    for b in range(B):
        one = m.kv(1, maxT, bf16=True)
        one.step_multi(prompts[b:b + 1, :-1], want_logits=False)
        l1, x1 = one.step(prompts[b, -1:])
        i1, l2 = one.decode_greedy(x1, n, want_logits=True)
        k1, v1 = one.read()
        one.close()
        ref_ids = np.concatenate([x1, i1[:, 0]])
        ref_lg = np.concatenate([l1, l2[:, 0]])
        diff = np.flatnonzero(got_ids[:, b] != ref_ids)
        first = int(diff[0]) if diff.size else n + 1
        if first <= n:
            srt = np.sort(ref_lg[first])
            flips.append((b, first, float(srt[-1] - srt[-2])))
        # steps t <= first see the same context in both runs: their logits,
        # and the layer-0 rows they append at position P-1+t
        for t in range(min(first, n) + 1):
            worst = max(worst, relerr(got_lg[t, b], ref_lg[t]))
            p = P - 1 + t
            for big, small in ((kb, k1), (vb, v1)):
                a = big[(b * maxT + p) * kvd:(b * maxT + p + 1) * kvd]
                r = small[p * kvd:(p + 1) * kvd]
                # one bf16 unit of the element, plus the fp32 summation-order
                # difference of the projection (elements near zero)
                bar = 2.0 ** -7 * np.abs(r) + 1e-5 * np.abs(r).max()
                assert np.all(np.abs(a - r) <= bar), (b, p, float(np.abs(a - r).max()))
    record("qkv_fold_gqa5_b40", relerr=worst, flips=flips)
    assert worst < TOL
    for b, t, marg in flips:
        assert marg < 2 * TOL * np.abs(got_lg).max(), (b, t, marg)
    m.close()
