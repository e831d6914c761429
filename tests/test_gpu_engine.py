"""GPU parity of the gfx950 engine against the CPU oracle, through the C ABI.

Bars (from the engine's contract): logits within max|d| <= 2e-3 * max|logit|
of the oracle on identical seeded bf16-exact weights and ids; greedy ids
identical over the decode horizon; everything else (steps == forward,
chunked == per-token, load == create) exact or at fp32 reordering level.
"""
import json
import os

import numpy as np
import pytest

from autoresearch_amd import engine
from autoresearch_amd.weights import (D12, Dims, rope_tables, seeded_weights, uniform_ids,
                                      write_npy_dir, write_safetensors, zipf_ids, BOS_ID)
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 2e-3  # max|d logit| / max|logit|
SMALL = Dims(n_layer=2, d_model=128, n_head=2, n_kv_head=1, head_dim=64, vocab=512)
SMALL_MHA = Dims(n_layer=2, d_model=256, n_head=2, n_kv_head=2, head_dim=128, vocab=1024)


def record(name, **kv):
    """Print a parity figure; also append it as a JSON line to the file
    $FGPT_PARITY_LOG names, when set."""
    print(name, kv, flush=True)
    path = os.environ.get("FGPT_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps({"test": name, **kv}) + "\n")


def relerr(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / np.max(np.abs(b)))


def tables(d, T):
    c, s = rope_tables(T, d.head_dim)
    return c.reshape(-1), s.reshape(-1)


@pytest.fixture(scope="module")
def d12():
    w = seeded_weights(D12, 1234)
    m = engine.Model(D12, stacks=w)
    c, s = tables(D12, 2304)
    m.set_rope(c, s)
    yield D12, w, m, c, s
    m.close()


@pytest.mark.parametrize("d", [SMALL, SMALL_MHA], ids=["gqa", "mha"])
@pytest.mark.parametrize("B,T", [(1, 1), (1, 4), (2, 3), (2, 37), (3, 130), (3, 500)])
def test_forward_small_vs_oracle(d, B, T):
    w = seeded_weights(d, 7)
    ids = uniform_ids(B * 100 + T, B * T, d.vocab)
    c, s = tables(d, T)
    m = engine.Model(d, stacks=w)
    m.set_rope(c, s)
    tg = np.roll(ids, -1)
    lg, nll = m.forward(ids, B, T, targets=tg)
    ref = O.gpt_forward(ids, c, s, w, d, B, T)
    e = relerr(lg, ref)
    record("forward_small", dims=str(d), B=B, T=T, relerr=e)
    assert e < TOL
    ref_nll = O.nll(ref.reshape(-1, d.vocab), tg, d.vocab)
    assert np.max(np.abs(nll.reshape(-1) - ref_nll)) < 2 * TOL * np.abs(ref).max()
    m.close()


@pytest.mark.parametrize("d,B,T,f16", [(SMALL, 2, 37, False), (SMALL, 3, 500, False),
                                       (SMALL_MHA, 1, 700, False), (SMALL, 2, 300, True)],
                         ids=["gqa-2x37", "gqa-3x500", "mha-1x700", "gqa-2x300-f16"])
def test_forward_pos_counts_vs_oracle(d, B, T, f16):
    """attn_sgemm's positive-score statistic (fg_forward_pos): per layer, row
    and head, the engine's count of causal scores > 0 against the oracle's
    count from its fp32 scores, within the scores whose sign sits within
    rounding (|q.k| <= tol * sum |q_d k_d|: 1e-4 for the split operands'
    ~16 significant bits, 2e-3 for single-term fp16's 11). The logits are
    fg_forward's, bit for bit (the count changes no arithmetic)."""
    w = seeded_weights(d, 8)
    ids = uniform_ids(B * 7 + T, B * T, d.vocab)
    c, s = tables(d, T)
    m = engine.Model(d, stacks=w)
    m.set_rope(c, s)
    m.set_forward_f16(f16)
    lg, npos = m.forward_pos(ids, B, T)
    lg0, _ = m.forward(ids, B, T)
    assert np.array_equal(lg, lg0)
    _, ref, amb = O.gpt_forward_pos(ids, c, s, w, d, B, T, rel_tol=2e-3 if f16 else 1e-4)
    diff = np.abs(npos.astype(np.int64) - ref)
    record("forward_pos_counts", dims=str(d), B=B, T=T, f16=f16, total=int(ref.sum()),
           max_diff=int(diff.max()), ambiguous=int(amb.sum()),
           frac_positive=float(ref.sum() / (d.n_layer * B * d.n_head * T * (T + 1) / 2)))
    assert np.all(diff <= amb)
    m.close()


def test_forward_d12_vs_oracle(d12):
    d, w, m, c, s = d12
    T = 256
    ids = uniform_ids(5, T, d.vocab)
    lg, _ = m.forward(ids, 1, T)
    ref = O.gpt_forward(ids, c, s, w, d, 1, T)
    e = relerr(lg, ref)
    record("forward_d12", T=T, relerr=e)
    assert e < TOL
    assert e < 1e-4  # the split-bf16 GEMMs keep ~fp32 accuracy
    assert np.array_equal(lg[0].argmax(-1), ref[0].argmax(-1))


@pytest.mark.parametrize("B,T", [(1, 48), (1, 1500), (2, 700)])
def test_forward_d12_gemm_shapes(d12, B, T):
    """Row counts that reach the other GEMM tilings: split-K partials and their
    reduce (48 rows), and the 64x96 residual tiles whose K is split over
    wavefront groups, with a partial last row tile (1400 and 1500 rows) and,
    at B=2, a sequence boundary inside a tile."""
    d, w, m, c, s = d12
    ids = uniform_ids(40 + T, B * T, d.vocab).reshape(B, T)
    lg, _ = m.forward(ids, B, T)
    for b in range(B):
        ref = O.gpt_forward(ids[b], c, s, w, d, 1, T)
        e = relerr(lg[b], ref[0])
        record("forward_d12_shape", B=B, T=T, row=b, relerr=e)
        assert e < 1e-4
        assert np.array_equal(lg[b].argmax(-1), ref[0].argmax(-1))


def test_prefill_d12_T2048_vs_oracle(d12):
    """The prefill workload's own size: T = 2048 logits and per-token CE."""
    d, w, m, c, s = d12
    T = 2048
    ids = uniform_ids(2, T + 1, d.vocab)
    lg, nll = m.forward(ids[:T], 1, T, targets=ids[1:])
    ref = O.gpt_forward(ids[:T], c, s, w, d, 1, T)
    e = relerr(lg, ref)
    ref_nll = O.nll(ref.reshape(T, -1), ids[1:], d.vocab)
    dn = float(np.max(np.abs(nll.reshape(-1) - ref_nll)))
    record("prefill_d12_T2048", relerr=e, max_dnll=dn, bits_mean=float(ref_nll.mean() / np.log(2)))
    assert e < TOL
    assert dn < 2 * TOL * np.abs(ref).max()
    # every cross-workgroup sum (K groups, key chunks, row sums of squares)
    # runs in a fixed order: a second forward gives the same bits
    lg2, nll2 = m.forward(ids[:T], 1, T, targets=ids[1:])
    assert np.array_equal(lg, lg2) and np.array_equal(nll, nll2)


def test_eval_rows_zipf_bos(d12):
    """bpb-style rows: Zipf ids, BOS at position 0, summed nats per row; rows
    batched on the GPU equal rows run one by one on the CPU."""
    d, w, m, c, s = d12
    B, T = 2, 192
    rows = zipf_ids(9, B * (T + 1), d.vocab).reshape(B, T + 1)
    rows[:, 0] = BOS_ID
    _, nll = m.forward(rows[:, :T], B, T, targets=rows[:, 1:])
    for b in range(B):
        ref = O.gpt_forward(rows[b, :T], c, s, w, d, 1, T)
        ref_sum = float(O.nll(ref.reshape(T, -1), rows[b, 1:], d.vocab).astype(np.float64).sum())
        got = float(nll[b].astype(np.float64).sum())
        record("eval_row", row=b, nats=got, ref=ref_sum)
        assert abs(got - ref_sum) < 2 * TOL * np.abs(ref).max() * T


def test_steps_equal_forward_and_oracle():
    d = SMALL
    w = seeded_weights(d, 11)
    T = 9
    ids = uniform_ids(3, T, d.vocab)
    c, s = tables(d, T)
    m = engine.Model(d, stacks=w)
    m.set_rope(c, s)
    full, _ = m.forward(ids, 1, T)
    kv = m.kv(1, T)
    steps = np.stack([kv.step(ids[t:t + 1])[0][0] for t in range(T)])
    assert kv.len == T
    assert relerr(steps, full[0]) < 1e-5
    okv = O.KVCache(d, T)
    hd2 = d.head_dim // 2
    ref = np.stack([O.gpt_step(ids[t:t + 1], c[t * hd2:], s[t * hd2:], w, d, okv) for t in range(T)])
    assert relerr(steps, ref) < TOL
    # the cache the engine wrote is the reference cache (rotated k, raw v)
    k, v = kv.read()
    assert relerr(k, okv.k) < 1e-4 and relerr(v, okv.v) < 1e-4
    with pytest.raises(engine.CacheFull):
        kv.step(ids[:1])
    kv.close()
    m.close()


@pytest.mark.parametrize("chunks", [[5, 1, 7], [1, 1, 1, 10], [13]])
def test_step_multi_vs_oracle(chunks):
    d = SMALL
    w = seeded_weights(d, 12)
    T = sum(chunks)
    ids = uniform_ids(4, T, d.vocab)
    c, s = tables(d, T)
    hd2 = d.head_dim // 2
    m = engine.Model(d, stacks=w)
    m.set_rope(c, s)
    kv = m.kv(1, T)
    okv = O.KVCache(d, T)
    p = 0
    for tb in chunks:
        lg, nxt = kv.step_multi(ids[p:p + tb])
        ref = O.gpt_step_multi(ids[p:p + tb], c[p * hd2:], s[p * hd2:], w, d, okv)
        assert relerr(lg[0], ref) < TOL
        assert nxt[0] == O.argmax(ref[-1])
        p += tb
    assert kv.len == T
    kv.close()
    m.close()


def test_greedy_depth12_prompt16_steps32(d12):
    """16 uniform prompt ids, then 32 greedy cached steps: ids must be identical."""
    d, w, m, c, s = d12
    prompt = uniform_ids(42, 16, d.vocab)
    ref_ids, ref_lg = O.greedy_decode(prompt, w, d, 32, c, s, maxT=48)
    kv = m.kv(1, 48)
    kv.step_multi(prompt[:-1], want_logits=False)
    ids, lg = kv.decode_greedy(prompt[-1:], 32, want_logits=True)
    srt = np.sort(ref_lg, -1)
    margin = float((srt[:, -1] - srt[:, -2]).min())
    e = relerr(lg[:, 0], ref_lg)
    record("greedy_d12", ids_equal=bool(np.array_equal(ids[:, 0], ref_ids)), relerr=e,
           min_top2_margin=margin, ids=ids[:, 0].tolist())
    assert np.array_equal(ids[:, 0], ref_ids)
    assert e < TOL
    # replaying the captured loop from a reset cache gives the same ids
    kv.len = 0
    kv.step_multi(prompt[:-1], want_logits=False)
    ids2, _ = kv.decode_greedy(prompt[-1:], 32)
    assert np.array_equal(ids2, ids)
    # the Python drop-in loop (chunked prompt of 4) agrees as well
    gen = engine.greedy_generate(m, prompt, 32, c, s, pchunk=4)
    assert np.array_equal(gen, ref_ids)
    kv.close()


def test_set_len_within_computed_positions():
    """set_len rolls back and forward again within the positions the cache
    has computed (a rejected draft's rows are recomputed before use); past
    them it fails instead of reading rows nothing wrote."""
    d = SMALL
    w = seeded_weights(d, 9)
    m = engine.Model(d, stacks=w)
    c, s = tables(d, 32)
    m.set_rope(c, s)
    kv = engine.KV(m, 1, 32)
    ids = uniform_ids(77, 12, d.vocab)
    ref, _ = kv.step_multi(ids[:8])
    kv.len = 3
    kv.len = 8
    with pytest.raises(engine.FgptError, match="computed only 8"):
        kv.len = 9
    assert kv.len == 8
    kv.len = 5
    again, _ = kv.step_multi(ids[5:8])
    assert relerr(again.reshape(3, -1), ref.reshape(8, -1)[5:8]) < 1e-5
    kv.close()
    m.close()


@pytest.mark.parametrize("B", [3, 6])
def test_batched_decode_rows_independent(B):
    """B sequences decoded together equal B independent B=1 oracle runs
    (B=6 runs the MFMA GEMM path for the per-step linears)."""
    d = SMALL
    w = seeded_weights(d, 13)
    P, n = 7, 12
    prompts = uniform_ids(77, B * P, d.vocab).reshape(B, P)
    c, s = tables(d, P + n)
    m = engine.Model(d, stacks=w)
    m.set_rope(c, s)
    kv = m.kv(B, P + n)
    kv.step_multi(prompts[:, :-1], want_logits=False)
    ids, lg = kv.decode_greedy(prompts[:, -1], n, want_logits=True)
    for b in range(B):
        ref_ids, ref_lg = O.greedy_decode(prompts[b], w, d, n, c, s, maxT=P + n)
        assert np.array_equal(ids[:, b], ref_ids)
        assert relerr(lg[:, b], ref_lg) < TOL
    kv.close()
    m.close()


@pytest.mark.parametrize("d,B,mode", [(SMALL, 1, "step"), (SMALL, 6, "step"),
                                      (SMALL_MHA, 1, "decode"), (SMALL_MHA, 6, "decode")],
                         ids=["step-b1", "step-b6", "fused-b1", "loop-b6"])
def test_argmax_ties_take_the_first_index(d, B, mode):
    """Exact ties in the logits: lm_head rows copied from sequence 0's winner
    give the same bits at every copy (the same dot product). The step's id
    must be the lowest tied index, as sample_token's strict > scan returns
    it, on every argmax the step can run (per-row kernel, single-block tail,
    the persistent loop's two-level exchange)."""
    w = seeded_weights(d, 31)
    P = 5
    prompts = uniform_ids(5, B * P, d.vocab).reshape(B, P)
    c, s = tables(d, P + 1)

    def run(weights):
        m = engine.Model(d, stacks=weights)
        m.set_rope(c, s)
        kv = m.kv(B, P + 1)
        kv.step_multi(prompts[:, :-1], want_logits=False)
        if mode == "step":
            lg, nxt = kv.step(prompts[:, -1])
        else:
            ids, lgs = kv.decode_greedy(prompts[:, -1], 1, want_logits=True)
            lg, nxt = lgs[0], ids[0]
        kv.close()
        m.close()
        return lg, nxt

    _, nxt0 = run(w)
    r = int(nxt0[0])
    lm = w["lm_head"].reshape(d.vocab, d.d_model).copy()
    copies = sorted({(r + k) % d.vocab for k in (-1, 1, 4, 129, 258)} - {r})
    for t in copies:
        lm[t] = lm[r]
    w2 = dict(w, lm_head=lm.reshape(-1))
    lg, nxt = run(w2)
    row = lg[0]
    tied = np.flatnonzero(row == row.max())
    record("argmax_ties", mode=mode, B=B, winner=r, tied=tied.tolist(), got=int(nxt[0]))
    assert len(tied) >= len(copies)  # the copies reproduce the winner's bits
    assert nxt[0] == tied[0]
    for b in range(B):
        assert nxt[b] == int(np.argmax(lg[b]))  # numpy's argmax: the first maximum


def test_errors_are_loud():
    d = SMALL
    w = seeded_weights(d, 14)
    m = engine.Model(d, stacks=w)
    with pytest.raises(engine.FgptError) as e:      # no RoPE rows yet
        m.forward(np.zeros(4, np.int32), 1, 4)
    assert e.value.code == -6
    c, s = tables(d, 8)
    m.set_rope(c, s)
    with pytest.raises(engine.FgptError) as e:      # id out of range
        m.forward(np.array([0, d.vocab], np.int32), 1, 2)
    assert e.value.code == -1
    kv = m.kv(1, 3)
    kv.step_multi(np.array([1, 2, 3], np.int32))
    with pytest.raises(engine.CacheFull):
        kv.step(np.array([1], np.int32))
    kv.close()
    bad = dict(w)
    bad["c_fc"] = w["c_fc"].copy()
    bad["c_fc"][5] = np.float32(0.1)  # 0.1 is not bf16-representable
    with pytest.raises(engine.FgptError) as e:
        engine.Model(d, stacks=bad)
    assert e.value.code == -3 and "c_fc" in str(e.value)
    m.close()


def test_load_npy_dir_equals_create(tmp_path):
    d = SMALL
    w = seeded_weights(d, 15)
    write_npy_dir(str(tmp_path), d, w, ctx=64)
    c, s = tables(d, 16)
    ids = uniform_ids(8, 16, d.vocab)
    a = engine.Model(d, stacks=w)
    b = engine.load_gpt_weights(str(tmp_path), d)
    a.set_rope(c, s)
    b.set_rope(c, s)
    la, _ = a.forward(ids, 1, 16)
    lb, _ = b.forward(ids, 1, 16)
    assert np.array_equal(la, lb)
    wrong = Dims(n_layer=2, d_model=128, n_head=2, n_kv_head=2, head_dim=64, vocab=512)
    with pytest.raises(engine.FgptError) as e:     # arch.txt says n_kv = 1
        engine.load_gpt_weights(str(tmp_path), wrong)
    assert e.value.code == -9
    os.remove(str(tmp_path / "transformer_h_1_mlp_c_fc_weight.npy"))
    with pytest.raises(engine.FgptError) as e:
        engine.load_gpt_weights(str(tmp_path), d)
    assert e.value.code == -3 and "missing" in str(e.value)
    # a model.safetensors beside them is read instead, and loads the same model
    write_safetensors(str(tmp_path), d, w, ctx=64)
    st = engine.load_gpt_weights(str(tmp_path), d)
    st.set_rope(c, s)
    ls, _ = st.forward(ids, 1, 16)
    assert np.array_equal(la, ls)
    st.close()
    a.close()
    b.close()


def test_eval_bpb_small_vs_oracle():
    """fg_eval_bpb: per-position NLL and the byte-weighted sums of
    scripts/eval_driver.py:174-190 (positions whose target has 0 bytes are
    left out) against the oracle's NLL weighted in float64 on the host."""
    d = SMALL
    w = seeded_weights(d, 17)
    N, T = 5, 130
    rows = uniform_ids(5, N * (T + 1), d.vocab).reshape(N, T + 1)
    tb = (uniform_ids(6, d.vocab, 5)).astype(np.int32)   # 0..4 bytes, zeros included
    assert (tb == 0).any()
    c, s = tables(d, T)
    m = engine.Model(d, stacks=w)
    m.set_rope(c, s)
    got = m.eval_bpb(rows, tb, batch=2, want_nll=True)       # batches of 2, 2, 1
    tot_n, tot_b = 0.0, 0
    for r in range(N):
        lg = O.gpt_forward(rows[r, :T], c, s, w, d, 1, T).reshape(T, d.vocab)
        nl = O.nll(lg, rows[r, 1:], d.vocab).astype(np.float64)
        keep = tb[rows[r, 1:]] > 0
        rn, rb = float(nl[keep].sum()), int(tb[rows[r, 1:]][keep].sum())
        assert got["row_bytes"][r] == rb
        assert abs(got["row_nats"][r] - rn) <= 2 * TOL * np.abs(lg).max() * T
        assert abs(got["row_nats"][r] - rn) <= 1e-4 * T
        assert np.abs(got["nll"][r] - nl).max() <= 2 * TOL * np.abs(lg).max()
        tot_n += rn
        tot_b += rb
    assert got["bytes"] == tot_b
    bpb_ref = tot_n / tot_b / np.log(2)
    record("eval_bpb_small", bpb=got["bpb"], ref=bpb_ref)
    assert abs(got["bpb"] - bpb_ref) <= 1e-4 * bpb_ref
    # the sums do not depend on how rows are batched
    again = m.eval_bpb(rows, tb, batch=5)
    assert np.allclose(again["row_nats"], got["row_nats"], rtol=1e-6, atol=0)
    # a target outside the table stops before any work
    with pytest.raises(engine.FgptError) as e:
        m.eval_bpb(rows, tb[:100], batch=2)
    assert e.value.code == -1 and "token_bytes" in str(e.value)
    with pytest.raises(engine.FgptError):
        m.eval_bpb(rows, tb, batch=65)
    m.close()


@pytest.mark.parametrize("B,T", [(1, 255), (1, 256), (1, 257), (2, 613)])
def test_host_logits_staged_copy_exact(d12, B, T):
    """Logits copied to host memory equal the device-pointer forward's bit
    for bit: below one 8 MiB staging chunk (255 rows of 8192 fp32), exactly
    one, one plus a row, and a ragged four-plus chunks; twice, so the second
    call reuses the staging buffers."""
    from .devbuf import DevBuf
    d, w, m, c, s = d12
    ids = uniform_ids(5 + T, B * T, d.vocab)
    di = DevBuf(ids)
    dl = DevBuf(np.zeros(B * T * d.vocab, np.float32))
    try:
        m.forward_dev(di.ptr, B, T, dl.ptr)
        ref = dl.get()
        for _ in range(2):
            lg, _ = m.forward(ids, B, T)
            assert np.array_equal(lg.reshape(-1), ref)
    finally:
        di.free()
        dl.free()


def test_decode_logits_over_staging_chunks(d12):
    """decode_greedy's logits for 64 sequences x 8 steps (16 MiB, two
    staging chunks) agree with per-step step_multi logits (2 MiB each, a
    direct copy) and give the same ids."""
    d, w, m, c, s = d12
    B, P, n = 64, 5, 8
    prompts = uniform_ids(31, B * P, d.vocab).reshape(B, P)
    a, b = m.kv(B, P + n), m.kv(B, P + n)
    a.step_multi(prompts[:, :-1], want_logits=False)
    b.step_multi(prompts[:, :-1], want_logits=False)
    ids, lg = a.decode_greedy(prompts[:, -1], n, want_logits=True)
    cur = prompts[:, -1]
    for k in range(n):
        one, nxt = b.step_multi(cur.reshape(B, 1))
        assert np.array_equal(nxt, ids[k])
        assert relerr(lg[k], one.reshape(B, d.vocab)) < 1e-5
        cur = nxt
    a.close()
    b.close()
