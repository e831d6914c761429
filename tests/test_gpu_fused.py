"""The persistent B=1 greedy decode (one launch for the whole loop) against
the CPU oracle and against the captured per-kernel path, through the C ABI.

Bars: logits within 2e-3 x max|logit| of the oracle, greedy ids identical,
the KV cache rows the loop writes equal to the oracle's within the same
bar; against the per-kernel path (same arithmetic, other fp32 summation
orders) ids identical and logits within 1e-5 x max|logit|; the persistent
loop itself deterministic (a replay from the same cache state is bit for bit
the same).
"""
import numpy as np
import pytest

from autoresearch_amd import engine
from autoresearch_amd.weights import D12, Dims, rope_tables, seeded_weights, uniform_ids
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 2e-3
SMALL_MHA = Dims(n_layer=2, d_model=256, n_head=2, n_kv_head=2, head_dim=128, vocab=1024)
SMALL_GQA = Dims(n_layer=2, d_model=128, n_head=2, n_kv_head=1, head_dim=64, vocab=512)
# the grouped-KV persistent kernel's small build: 4 heads over 2 KV heads
SMALL_GQA2 = Dims(n_layer=2, d_model=512, n_head=4, n_kv_head=2, head_dim=128, vocab=1024)


def relerr(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / np.max(np.abs(b)))


def setup(d, seed, n_pos):
    w = seeded_weights(d, seed)
    m = engine.Model(d, stacks=w)
    c, s = rope_tables(n_pos, d.head_dim)
    c, s = c.reshape(-1), s.reshape(-1)
    m.set_rope(c, s)
    return w, m, c, s


def oracle_cache(prompt, w, d, n_gen, c, s, maxT):
    """The oracle's cache after the prompt and n_gen greedy steps."""
    kv = O.KVCache(d, maxT)
    ids = list(prompt)
    for t in range(len(prompt) + n_gen - 1):
        lg = O.gpt_step(np.array([ids[t]], np.int32), c[t * (d.head_dim // 2):],
                        s[t * (d.head_dim // 2):], w, d, kv)
        if t >= len(prompt) - 1:
            ids.append(int(np.argmax(lg)))
    return kv.k.copy(), kv.v.copy()


@pytest.fixture(scope="module")
def d12():
    w, m, c, s = setup(D12, 1234, 2304)
    yield D12, w, m, c, s
    m.close()


def test_fused_is_active_on_mi355x(d12):
    d, w, m, c, s = d12
    on, why = m.fused_decode()
    print("persistent decode active:", on, why)
    assert on, why


def test_fused_d12_prompt16_steps32_vs_oracle(d12):
    """The B=1 workload: 16 uniform prompt ids, 32 greedy steps."""
    d, w, m, c, s = d12
    prompt = uniform_ids(42, 16, d.vocab)
    ref_ids, ref_lg = O.greedy_decode(prompt, w, d, 32, c, s, maxT=48)
    kv = m.kv(1, 48)
    kv.step_multi(prompt[:-1], want_logits=False)
    ids, lg = kv.decode_greedy(prompt[-1:], 32, want_logits=True)
    e = relerr(lg[:, 0], ref_lg)
    print("fused d12: ids equal", np.array_equal(ids[:, 0], ref_ids), "relerr", e)
    assert np.array_equal(ids[:, 0], ref_ids)
    assert e < TOL
    # the cache rows the loop wrote (positions 15..46) match the oracle's
    k, v = kv.read()
    rk, rv = oracle_cache(prompt, w, d, 32, c, s, 48)
    kd = d.n_kv_head * d.head_dim
    k = k.reshape(d.n_layer, 48, kd)[:, :47]
    v = v.reshape(d.n_layer, 48, kd)[:, :47]
    rk = rk.reshape(d.n_layer, 48, kd)[:, :47]
    rv = rv.reshape(d.n_layer, 48, kd)[:, :47]
    assert relerr(k, rk) < TOL and relerr(v, rv) < TOL
    kv.close()


def test_fused_equals_per_kernel_path(d12):
    d, w, m, c, s = d12
    prompt = uniform_ids(7, 16, d.vocab)
    kv = m.kv(1, 48)
    kv.step_multi(prompt[:-1], want_logits=False)
    ids_f, lg_f = kv.decode_greedy(prompt[-1:], 32, want_logits=True)
    kf, vf = kv.read()
    m.set_fused_decode(False)
    try:
        assert m.fused_decode() == (False, "disabled by fg_set_option")
        kv.len = 15
        ids_g, lg_g = kv.decode_greedy(prompt[-1:], 32, want_logits=True)
        kg, vg = kv.read()
    finally:
        m.set_fused_decode(True)
    assert np.array_equal(ids_f, ids_g)
    e = relerr(lg_f, lg_g)
    print("fused vs per-kernel: logits relerr", e)
    assert e < 1e-5
    assert relerr(kf, kg) < 1e-5 and relerr(vf, vg) < 1e-5
    kv.close()


def test_fused_replay_and_chained_calls(d12):
    """A replay from the same cache state is bit for bit the same (later
    launches run on fresh epochs over the same exchange slots), and 12 + 20
    steps in two calls equal 32 in one."""
    d, w, m, c, s = d12
    prompt = uniform_ids(11, 16, d.vocab)
    kv = m.kv(1, 48)
    kv.step_multi(prompt[:-1], want_logits=False)
    a_ids, a_lg = kv.decode_greedy(prompt[-1:], 32, want_logits=True)
    for _ in range(3):
        kv.len = 15
        b_ids, b_lg = kv.decode_greedy(prompt[-1:], 32, want_logits=True)
        assert np.array_equal(a_ids, b_ids)
        assert np.array_equal(a_lg, b_lg)
    kv.len = 15
    c1, l1 = kv.decode_greedy(prompt[-1:], 12, want_logits=True)
    c2, l2 = kv.decode_greedy(c1[-1], 20, want_logits=True)
    assert np.array_equal(np.concatenate([c1, c2]), a_ids)
    assert np.array_equal(np.concatenate([l1, l2]), a_lg)
    kv.close()


def test_fused_small_mha_across_split():
    """Small MHA dims (d_model 256, 2 heads of 128): one persistent call
    through the positions below FUSED_SPLIT_MIN (128: each workgroup of a
    head's XCD runs the whole attention) and on past it (the attention split
    over 8 workgroups, partials merged after one more hand-over), against
    the oracle and the per-kernel path."""
    d = SMALL_MHA
    w, m, c, s = setup(d, 21, 200)
    on, why = m.fused_decode()
    assert on, why
    prompt = uniform_ids(5, 7, d.vocab)
    n = 180
    ref_ids, ref_lg = O.greedy_decode(prompt, w, d, n, c, s, maxT=200)
    kv = m.kv(1, 200)
    kv.step_multi(prompt[:-1], want_logits=False)
    ids, lg = kv.decode_greedy(prompt[-1:], n, want_logits=True)   # positions 6..185
    e = relerr(lg[:, 0], ref_lg)
    print("small mha across the split: ids equal", np.array_equal(ids[:, 0], ref_ids), "relerr", e)
    assert np.array_equal(ids[:, 0], ref_ids)
    assert e < TOL
    m.set_fused_decode(False)
    try:
        kv.len = 6
        ids_g, lg_g = kv.decode_greedy(prompt[-1:], n, want_logits=True)
    finally:
        m.set_fused_decode(True)
    assert np.array_equal(ids, ids_g)
    print("vs per-kernel path: logits relerr", relerr(lg, lg_g))
    assert relerr(lg, lg_g) < 1e-5
    kv.close()
    m.close()


def test_fused_d12_long_context_vs_oracle(d12):
    """chat_text's context length: a 1008-id prompt (cached by one chunked
    pass), then 40 greedy steps at positions 1007..1046 in one persistent
    call (the split attention over 16 workgroups: one batch of cache rows
    per position group below 1024 positions, a second one from there),
    against the oracle (ids identical, logits within the bar) and the
    per-kernel path; a replay is bit for bit the same."""
    d, w, m, c, s = d12
    P, n, maxT = 1008, 40, 1080
    prompt = uniform_ids(77, P, d.vocab)
    ref_ids, ref_lg = O.greedy_decode(prompt, w, d, n, c, s, maxT=maxT, prefill_multi=True)
    kv = m.kv(1, maxT)
    kv.step_multi(prompt[:-1], want_logits=False)
    ids, lg = kv.decode_greedy(prompt[-1:], n, want_logits=True)
    e = relerr(lg[:, 0], ref_lg)
    srt = np.sort(ref_lg, -1)
    print("fused d12 at 1007..1046: ids equal", np.array_equal(ids[:, 0], ref_ids), "relerr", e,
          "min oracle top-2 margin", float((srt[:, -1] - srt[:, -2]).min()))
    assert np.array_equal(ids[:, 0], ref_ids)
    assert e < TOL
    kv.len = P - 1
    ids2, lg2 = kv.decode_greedy(prompt[-1:], n, want_logits=True)
    assert np.array_equal(ids, ids2) and np.array_equal(lg, lg2)
    m.set_fused_decode(False)
    try:
        kv.len = P - 1
        ids_g, lg_g = kv.decode_greedy(prompt[-1:], n, want_logits=True)
    finally:
        m.set_fused_decode(True)
    assert np.array_equal(ids, ids_g)
    assert relerr(lg, lg_g) < 1e-5
    kv.close()


def test_fused_not_for_unsupported_dims():
    """head_dim 64 with grouped KV heads keeps the per-kernel path, which
    still matches the oracle."""
    d = SMALL_GQA
    w, m, c, s = setup(d, 3, 40)
    on, why = m.fused_decode()
    assert not on and why
    prompt = uniform_ids(9, 8, d.vocab)
    ref_ids, _ = O.greedy_decode(prompt, w, d, 20, c, s, maxT=40)
    kv = m.kv(1, 40)
    kv.step_multi(prompt[:-1], want_logits=False)
    ids, _ = kv.decode_greedy(prompt[-1:], 20)
    assert np.array_equal(ids[:, 0], ref_ids)
    kv.close()
    m.close()


def test_fused_gqa_small_vs_oracle():
    """The grouped-KV persistent kernel (4 heads over 2 KV heads): one call
    from position 6 to 305, so the group's positions first sit in the first
    quarter's 32 workgroups only (the other three quarters' partials empty),
    then in all 128 and on past 256 (two and three positions per
    workgroup); against the oracle (ids identical, logits and the cache rows
    the loop wrote within the bar), the per-kernel path (ids identical,
    logits within 1e-5 x max|logit|), and a replay bit for bit."""
    d = SMALL_GQA2
    w, m, c, s = setup(d, 31, 320)
    on, why = m.fused_decode()
    print("grouped-KV persistent decode active:", on, why)
    assert on, why
    prompt = uniform_ids(13, 7, d.vocab)
    n, maxT = 300, 320
    ref_ids, ref_lg = O.greedy_decode(prompt, w, d, n, c, s, maxT=maxT)
    kv = m.kv(1, maxT)
    kv.step_multi(prompt[:-1], want_logits=False)
    ids, lg = kv.decode_greedy(prompt[-1:], n, want_logits=True)   # positions 6..305
    e = relerr(lg[:, 0], ref_lg)
    first = int(np.argmax(ids[:, 0] != ref_ids)) if not np.array_equal(ids[:, 0], ref_ids) else -1
    print("small gqa: ids equal", first < 0, "first mismatch", first, "relerr", e)
    assert np.array_equal(ids[:, 0], ref_ids)
    assert e < TOL
    k, v = kv.read()
    rk, rv = oracle_cache(prompt, w, d, n, c, s, maxT)
    kd = d.n_kv_head * d.head_dim
    P = len(prompt) + n - 1
    k = k.reshape(d.n_layer, maxT, kd)[:, :P]
    v = v.reshape(d.n_layer, maxT, kd)[:, :P]
    rk = rk.reshape(d.n_layer, maxT, kd)[:, :P]
    rv = rv.reshape(d.n_layer, maxT, kd)[:, :P]
    print("cache rows relerr", relerr(k, rk), relerr(v, rv))
    assert relerr(k, rk) < TOL and relerr(v, rv) < TOL
    kv.len = 6
    ids2, lg2 = kv.decode_greedy(prompt[-1:], n, want_logits=True)
    assert np.array_equal(ids, ids2) and np.array_equal(lg, lg2)
    m.set_fused_decode(False)
    try:
        kv.len = 6
        ids_g, lg_g = kv.decode_greedy(prompt[-1:], n, want_logits=True)
    finally:
        m.set_fused_decode(True)
    assert np.array_equal(ids, ids_g)
    print("vs per-kernel path: logits relerr", relerr(lg, lg_g))
    assert relerr(lg, lg_g) < 1e-5
    kv.close()
    m.close()


def test_fused_gqa_small_long_context():
    """The grouped-KV persistent kernel past 512 positions (a 600-id prompt
    cached by one chunked pass, then 80 steps at positions 599..678): a
    workgroup then holds up to six of the group's positions, so its waves
    weigh slots on more than one 16-lane row; against the oracle and the
    per-kernel path."""
    d = SMALL_GQA2
    P, n, maxT = 600, 80, 700
    w, m, c, s = setup(d, 37, maxT)
    prompt = uniform_ids(19, P, d.vocab)
    ref_ids, ref_lg = O.greedy_decode(prompt, w, d, n, c, s, maxT=maxT, prefill_multi=True)
    kv = m.kv(1, maxT)
    kv.step_multi(prompt[:-1], want_logits=False)
    ids, lg = kv.decode_greedy(prompt[-1:], n, want_logits=True)
    e = relerr(lg[:, 0], ref_lg)
    print("small gqa at 599..678: ids equal", np.array_equal(ids[:, 0], ref_ids), "relerr", e)
    assert np.array_equal(ids[:, 0], ref_ids)
    assert e < TOL
    m.set_fused_decode(False)
    try:
        kv.len = P - 1
        ids_g, lg_g = kv.decode_greedy(prompt[-1:], n, want_logits=True)
    finally:
        m.set_fused_decode(True)
    assert np.array_equal(ids, ids_g)
    assert relerr(lg, lg_g) < 1e-5
    kv.close()
    m.close()
