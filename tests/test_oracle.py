"""Pins for the CPU oracle (oracle/fgpt_oracle.c) before it is trusted.

What fixes each oracle routine (reference = 14NGiestas/autoresearch):
  or_relu2          reference KAT, src/test/test_kernels.f90:342-367
  or_argmax         reference greedy KAT, src/test/test_kernels.f90:677-688;
                    first-max tie rule of src/lib/sample.f90:271-277
  or_rmsnorm0       closed form in float64 (reference tolerance 1e-4,
                    src/test/test_kernels.f90:177-204)
  or_linear         float64 matmul at model shapes (tol of test_linear_blas,
                    src/test/test_kernels.f90:2156-2177)
  or_rope           complex rotation x*exp(-i angle) in float64, plus norm
                    preservation (reference tolerance 1e-5, :302-339)
  or_rope_tables    float64 cos/sin of the closed-form angle
  or_causal_attn    masked-softmax attention in float64, MHA and GQA H=4/KH=2
                    (the reference's own GQA case, :370-510)
  or_attn_step      bit-equal to the last causal_attn row
                    (src/lib/fortran_attn.f90:316)
  or_attn_chunk     bit-equal to causal_attn at TC_PREV=0 and to attn_step at
                    TB=1 (src/lib/fortran_attn.f90:370-374)
  or_wte_lookup     exact gather
  or_gpt_forward    float64 whole-tensor forward (tests/np_ref.py) at tiny
                    dims and at depth-12 dims with short T; causal-prefix and
                    batch-row independence invariants
  or_gpt_step       4 cached steps == forward, the reference's test_kv_equiv
                    (src/test/test_kernels.f90:720-779, tol 1e-6)
  or_gpt_step_multi chunked == per-token == forward (:1466-1550); cache-full
                    and TB<1 errors (src/lib/fortran_kv.f90:74-77,209-216)
  or_nll            float64 logsumexp - logit[target]
  or_attn_pos_count closed forms (scores all > 0, all < 0, exactly 0 on some
                    rows: the strict >), the GQA head -> kv head mapping,
                    float64 counts on random inputs
  or_gpt_forward_pos  logits bit-equal to or_gpt_forward; per-layer counts
                    equal to the float64 forward's (tests/np_ref.py)
  or_frand_fill     input generator only (no parity claim): range and
                    determinism
"""
import numpy as np
import pytest

from autoresearch_amd.weights import Dims, D12, round_bf16, seeded_weights, uniform_ids
from oracle import oracle as O
from tests import np_ref

TINY = Dims(n_layer=1, d_model=8, n_head=2, n_kv_head=2, head_dim=4, vocab=16)
TINY_GQA = Dims(n_layer=2, d_model=16, n_head=4, n_kv_head=2, head_dim=4, vocab=32)


def frand_weights(d: Dims, seed=42):
    """Stacked buffers filled as test_kv_equiv fills them (scale 0.1 / 0.05)."""
    from autoresearch_amd.weights import stack_sizes
    sizes = stack_sizes(d)
    out, s = {}, seed
    for name in ("wte", "c_q", "c_k", "c_v", "c_proj", "c_fc", "c_proj2", "lm_head"):
        x, s = O.frand(s, sizes[name], 0.1 if name == "wte" else 0.05)
        out[name] = x
    return out


def test_relu2_kat():
    x = np.array([-2.0, -1.0, -0.5, 0.0, 0.5, 1.0, 2.0], np.float32)
    y = O.relu2(x)
    assert np.max(np.abs(y - np.array([0, 0, 0, 0, 0.25, 1.0, 4.0], np.float32))) < 1e-6


def test_argmax_kat_and_ties():
    assert O.argmax([-1.0, 2.0, 0.5, -0.5]) == 1  # reference: 1-based position 2
    assert O.argmax([3.0, 1.0, 3.0]) == 0          # first maximum wins
    assert O.argmax([-5.0, -1.0, -1.0, -7.0]) == 1


def test_frand_generator():
    a, s1 = O.frand(42, 1000)
    b, s2 = O.frand(42, 1000)
    assert np.array_equal(a, b) and s1 == s2
    assert np.all(np.abs(a) <= 1.5)  # wrapped LCG may go negative: r in [-1.5, 0.5)
    assert len(np.unique(a)) > 900


def test_rmsnorm0_closed_form():
    x, _ = O.frand(42, 4 * 32)
    y = O.rmsnorm0(x, 32, 1e-5)
    x64 = x.astype(np.float64).reshape(4, 32)
    ref = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-5)
    assert np.max(np.abs(y.reshape(4, 32) - ref)) < 1e-6


@pytest.mark.parametrize("BT,IF,OF", [(10, 8, 6), (3, 768, 2304), (5, 3072, 768), (2, 768, 8192)])
def test_linear_vs_float64(BT, IF, OF):
    rng = np.random.default_rng(BT + IF)
    x = rng.standard_normal(BT * IF).astype(np.float32)
    w = round_bf16((rng.standard_normal(OF * IF) * 0.02).astype(np.float32))
    y = O.linear(x, w, IF, OF).reshape(BT, OF)
    ref = x.astype(np.float64).reshape(BT, IF) @ w.astype(np.float64).reshape(OF, IF).T
    assert np.max(np.abs(y - ref)) < 1e-4 * max(1.0, np.abs(ref).max())


def test_rope_complex_rotation_and_norm():
    B, T, H, D = 1, 4, 2, 8
    x, s = O.frand(42, B * T * H * D)
    c, s = O.frand(s, T * D // 2)
    sn, _ = O.frand(s, T * D // 2)
    y = O.rope(x, c, sn, B, T, H, D)
    ref = np_ref.rope(x.astype(np.float64).reshape(T, H, D), c.reshape(T, -1).astype(np.float64),
                      sn.reshape(T, -1).astype(np.float64))
    assert np.max(np.abs(y.reshape(T, H, D) - ref)) < 1e-6
    # with a true (cos, sin) table the rotation preserves each pair's norm
    ct, st = O.rope_tables(T, D)
    y2 = O.rope(x, ct, st, B, T, H, D).reshape(T, H, 2, D // 2)
    x2 = x.reshape(T, H, 2, D // 2)
    assert np.allclose((y2 ** 2).sum(2), (x2 ** 2).sum(2), rtol=1e-5, atol=1e-7)


def test_rope_tables_closed_form():
    T, hd = 64, 128
    c, s = O.rope_tables(T, hd)
    j = np.arange(hd // 2)
    ang = np.arange(T)[:, None] * 10000.0 ** (-2.0 * j / hd)[None, :]
    assert np.max(np.abs(c.reshape(T, -1) - np.cos(ang))) < 5e-5
    assert np.max(np.abs(s.reshape(T, -1) - np.sin(ang))) < 5e-5
    assert c[0] == 1.0 and s[0] == 0.0


@pytest.mark.parametrize("H,KH", [(1, 1), (2, 2), (4, 2), (6, 6), (10, 2)])
def test_causal_attn_vs_masked_softmax(H, KH):
    B, T, D = 2, 7, 16
    rng = np.random.default_rng(H * 10 + KH)
    q = rng.standard_normal((B, T, H, D)).astype(np.float32)
    k = rng.standard_normal((B, T, KH, D)).astype(np.float32)
    v = rng.standard_normal((B, T, KH, D)).astype(np.float32)
    y = O.causal_attn(q, k, v, B, T, H, KH, D).reshape(B, T, H, D)
    for b in range(B):
        ref = np_ref.attention(q[b].astype(np.float64), k[b].astype(np.float64), v[b].astype(np.float64))
        assert np.max(np.abs(y[b] - ref)) < 1e-5


def test_gqa_reduces_to_mha():
    B, T, H, KH, D = 1, 6, 4, 2, 8
    rng = np.random.default_rng(5)
    q = rng.standard_normal((B, T, H, D)).astype(np.float32)
    k = rng.standard_normal((B, T, KH, D)).astype(np.float32)
    v = rng.standard_normal((B, T, KH, D)).astype(np.float32)
    y = O.causal_attn(q, k, v, B, T, H, KH, D)
    y_mha = O.causal_attn(q, np.repeat(k, H // KH, axis=2), np.repeat(v, H // KH, axis=2), B, T, H, H, D)
    assert np.array_equal(y, y_mha)


def test_attn_step_and_chunk_equal_causal_rows():
    B, T, H, KH, D = 1, 9, 4, 2, 8
    rng = np.random.default_rng(11)
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    k = rng.standard_normal((T, KH, D)).astype(np.float32)
    v = rng.standard_normal((T, KH, D)).astype(np.float32)
    full = O.causal_attn(q, k, v, 1, T, H, KH, D).reshape(T, H, D)
    step = O.attn_step(q[T - 1], k, v, 1, H, KH, D, T).reshape(H, D)
    assert np.array_equal(step, full[T - 1])
    chunk0 = O.attn_chunk(q, k, v, 1, H, KH, D, 0, T).reshape(T, H, D)
    assert np.array_equal(chunk0, full)
    chunk1 = O.attn_chunk(q[T - 1], k, v, 1, H, KH, D, T - 1, 1).reshape(H, D)
    assert np.array_equal(chunk1, step)
    tail = O.attn_chunk(q[5:], k, v, 1, H, KH, D, 5, T - 5).reshape(T - 5, H, D)
    assert np.array_equal(tail, full[5:])


def test_wte_lookup_gather():
    V, D = 16, 8
    wte, _ = O.frand(7, V * D)
    ids = np.array([3, 0, 15, 3], np.int32)
    out = np.empty(4 * D, np.float32)
    O.lib().or_wte_lookup(O.ip(ids), O.fp(wte), O.fp(out), 1, 4, D)
    assert np.array_equal(out.reshape(4, D), wte.reshape(V, D)[ids])


@pytest.mark.parametrize("d", [TINY, TINY_GQA])
def test_forward_vs_float64_tiny(d):
    B, T = 2, 5
    w = frand_weights(d)
    ids = (np.arange(B * T) * 5 + 1) % d.vocab
    c, s = O.rope_tables(T, d.head_dim)
    out = O.gpt_forward(ids, c, s, w, d, B, T)
    ref = np_ref.forward(ids, c, s, w, d, B, T)
    assert np.max(np.abs(out - ref)) < 1e-5 * max(1.0, np.abs(ref).max())


def test_forward_vs_float64_depth12_short():
    d, T = D12, 6
    w = seeded_weights(d, seed=1234)
    ids = uniform_ids(1234, T, d.vocab)
    c, s = O.rope_tables(T, d.head_dim)
    out = O.gpt_forward(ids, c, s, w, d, 1, T)
    ref = np_ref.forward(ids, c, s, w, d, 1, T)
    assert np.max(np.abs(out - ref)) < 2e-4 * np.abs(ref).max()


def test_transposed_weight_cache_changes_nothing():
    """or_wt_cache(1) (transposed weights kept between calls, for timing the
    CPU baseline) gives the same bits as transposing on every call."""
    d, B, T = TINY_GQA, 2, 5
    w = frand_weights(d, seed=13)
    ids = ((np.arange(B * T) * 3 + 1) % d.vocab).astype(np.int32)
    c, s = O.rope_tables(T, d.head_dim)
    ref = O.gpt_forward(ids, c, s, w, d, B, T)
    O.lib().or_wt_cache(1)
    try:
        a = O.gpt_forward(ids, c, s, w, d, B, T)
        b = O.gpt_forward(ids, c, s, w, d, B, T)
    finally:
        O.lib().or_wt_cache(0)
    assert np.array_equal(a, ref) and np.array_equal(b, ref)


def test_forward_causal_prefix_and_rows():
    d, B, T = TINY_GQA, 3, 6
    w = frand_weights(d, seed=9)
    ids = ((np.arange(B * T) * 7 + 3) % d.vocab).astype(np.int32)
    c, s = O.rope_tables(T, d.head_dim)
    out = O.gpt_forward(ids, c, s, w, d, B, T)
    ids2 = ids.copy().reshape(B, T)
    ids2[:, 4:] = (ids2[:, 4:] + 5) % d.vocab
    out2 = O.gpt_forward(ids2, c, s, w, d, B, T)
    assert np.array_equal(out[:, :4], out2[:, :4])
    assert not np.array_equal(out[:, 4:], out2[:, 4:])
    for b in range(B):
        ob = O.gpt_forward(ids.reshape(B, T)[b], c, s, w, d, 1, T)
        assert np.array_equal(ob[0], out[b])


def test_kv_equiv_steps_equal_forward():
    """The reference's test_kv_equiv: BR=1, TC=4, V=16, D=8, H=KH=2, hd=4."""
    d, T = TINY, 4
    w = frand_weights(d)
    ids = np.array([1 + (i + 1) % 7 for i in range(T)], np.int32)
    c, s = O.frand(123, T * 2)
    sn, _ = O.frand(456, T * 2)
    full = O.gpt_forward(ids, c, sn, w, d, 1, T)[0]
    kv = O.KVCache(d, T)
    steps = np.stack([O.gpt_step(ids[t:t + 1], c[t * 2:], sn[t * 2:], w, d, kv) for t in range(T)])
    assert kv.len[0] == T
    assert np.max(np.abs(full - steps)) < 1e-6
    with pytest.raises(RuntimeError):
        O.gpt_step(ids[:1], c, sn, w, d, kv)


def test_kv_chunk_equiv():
    d, T = TINY_GQA, 7
    w = frand_weights(d, seed=3)
    ids = ((np.arange(T) * 3 + 2) % d.vocab).astype(np.int32)
    c, s = O.rope_tables(T, d.head_dim)
    hd2 = d.head_dim // 2
    full = O.gpt_forward(ids, c, s, w, d, 1, T)[0]
    kv = O.KVCache(d, T)
    a = O.gpt_step_multi(ids[:3], c, s, w, d, kv)
    b = O.gpt_step_multi(ids[3:], c[3 * hd2:], s[3 * hd2:], w, d, kv)
    assert kv.len[0] == T
    assert np.max(np.abs(np.concatenate([a, b]) - full)) < 1e-6
    kv2 = O.KVCache(d, T)
    steps = np.stack([O.gpt_step(ids[t:t + 1], c[t * hd2:], s[t * hd2:], w, d, kv2) for t in range(T)])
    assert np.max(np.abs(steps - full)) < 1e-6
    assert np.array_equal(kv.k, kv2.k) and np.array_equal(kv.v, kv2.v)
    with pytest.raises(RuntimeError):
        O.gpt_step_multi(ids[:1], c, s, w, d, kv)
    with pytest.raises(ValueError):
        O.gpt_step_multi(ids[:0], c, s, w, d, O.KVCache(d, T))


def test_nll_vs_logsumexp():
    rng = np.random.default_rng(2)
    lg = (rng.standard_normal((5, 300)) * 3).astype(np.float32)
    tg = rng.integers(0, 300, 5).astype(np.int32)
    out = O.nll(lg, tg, 300)
    ref = np_ref.nll(lg, tg)
    assert np.max(np.abs(out - ref)) < 1e-5


def test_attn_pos_count_closed_forms():
    """attn_sgemm's positive-score count (src/lib/fortran_attn.f90:249-254):
    q = k with positive entries makes every causal score > 0 (T(T+1)/2 per
    row and head), q = -k none; query rows of zeros give scores of exactly
    0, which the strict > does not count."""
    B, T, H, D = 2, 7, 2, 4
    k = np.full((B, T, H, D), 0.5, np.float32)
    n, _ = O.attn_pos_count(k, k, B, T, H, H, D)
    assert np.all(n == T * (T + 1) // 2)
    n, _ = O.attn_pos_count(-k, k, B, T, H, H, D)
    assert np.all(n == 0)
    q = k.copy()
    q[:, 1::2] = 0.0  # odd query positions: scores exactly 0
    n, amb = O.attn_pos_count(q, k, B, T, H, H, D)
    assert np.all(n == sum(t + 1 for t in range(0, T, 2)))
    assert np.all(amb == sum(t + 1 for t in range(1, T, 2)))  # the zeros sit at 0


def test_attn_pos_count_gqa_mapping():
    """Query head h reads kv head h / (H/KH) (src/lib/fortran_attn.f90:226):
    with kv head 0 positive and kv head 1 negative, heads 0-1 count every
    score and heads 2-3 none."""
    B, T, H, KH, D = 1, 5, 4, 2, 4
    q = np.ones((B, T, H, D), np.float32)
    k = np.ones((B, T, KH, D), np.float32)
    k[:, :, 1] = -1.0
    n, _ = O.attn_pos_count(q, k, B, T, H, KH, D)
    assert n.tolist() == [[T * (T + 1) // 2] * 2 + [0, 0]]


def test_attn_pos_count_random_vs_float64():
    rng = np.random.default_rng(3)
    B, T, H, KH, D = 2, 33, 4, 2, 16
    q = rng.standard_normal((B, T, H, D)).astype(np.float32)
    k = rng.standard_normal((B, T, KH, D)).astype(np.float32)
    n, amb = O.attn_pos_count(q, k, B, T, H, KH, D)
    kk = np.repeat(k.astype(np.float64), H // KH, axis=2)
    s = np.einsum("bqhd,bkhd->bhqk", q.astype(np.float64), kk)
    causal = np.tril(np.ones((T, T), bool))
    ref = ((s > 0) & causal).sum(axis=(2, 3))
    assert np.all(np.abs(n - ref) <= amb)
    assert 0 < n.min() and n.max() < T * (T + 1) // 2


@pytest.mark.parametrize("d", [TINY, TINY_GQA])
def test_gpt_forward_pos_vs_float64(d):
    w = frand_weights(d, 19)
    B, T = 2, 9
    ids = uniform_ids(4, B * T, d.vocab)
    c, s = O.rope_tables(T, d.head_dim)
    lg, npos, namb = O.gpt_forward_pos(ids, c, s, w, d, B, T)
    assert np.array_equal(lg, O.gpt_forward(ids, c, s, w, d, B, T))
    ref, closest = np_ref.pos_counts(ids, c, s, w, d, B, T)
    assert np.all(np.abs(npos - ref) <= namb)
    assert closest > 1e-4 or namb.sum() > 0
    assert npos.shape == (d.n_layer, B, d.n_head)
