"""The full-size workloads on the GPU against the oracle's committed results.

tests/golden/make_fixtures.py ran the CPU oracle once on the same seeded
weights and ids (regenerated here bit for bit by the repository's own
generators) and stored: the per-row NLL sums of the B=8 x 2048 Zipf eval
rows, the greedy ids and per-step top-2 logit margins of all 64
batched-decode sequences (1024-id prompts, 512 steps), and the depth-20 GQA
model's prefill rows 0, 128, ..., 1920, 2047 and 256 greedy ids. Bars:
logits within 2e-3 x max|logit|, NLL sums within 2 x max|d logit| per
token, greedy ids identical (on the fp32 cache; the bf16 cache is reported
against the same ids with the margin of each first flip).
"""
import functools
import json
import os

import numpy as np
import pytest

from autoresearch_amd import engine
from autoresearch_amd.weights import D12, GQA20, rope_tables, seeded_weights, uniform_ids, zipf_ids

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
TOL = 2e-3


def fixture(name):
    with open(os.path.join(GOLD, name + ".json")) as f:
        return json.load(f)


def model(d, seed, n_pos):
    m = engine.Model(d, stacks=seeded_weights(d, seed))
    c, s = rope_tables(n_pos, d.head_dim)
    m.set_rope(c.reshape(-1), s.reshape(-1))
    return m


def test_eval_rows_b8_t2048():
    """bpb-style evaluation, B=8 independent rows of T=2048 in one batch."""
    g = fixture("eval_rows_d12")
    d, B, T = D12, g["B"], g["T"]
    rows = zipf_ids(g["seed"], B * (T + 1), d.vocab).reshape(B, T + 1)
    rows[:, 0] = g["bos"]
    m = model(d, g["weights_seed"], T)
    lg, nll = m.forward(rows[:, :T], B, T, targets=rows[:, 1:])
    maxlogit = float(np.abs(lg).max())
    got = nll.astype(np.float64).sum(axis=1)
    ref = np.array(g["nats"])
    print("eval rows: max |d nats| per row", np.abs(got - ref).max(), "max|logit|", maxlogit)
    # |d nll| <= 2 max|d logit| per token, max|d logit| <= TOL * max|logit|
    assert np.all(np.abs(got - ref) <= 2 * TOL * maxlogit * T)
    # and far inside that bar: below 1e-4 nats per token on average
    assert np.all(np.abs(got - ref) <= 1e-4 * T)
    # one row alone gives the same sums as inside the batch
    _, nll1 = m.forward(rows[B - 1:, :T], 1, T, targets=rows[B - 1:, 1:])
    assert abs(float(nll1.astype(np.float64).sum()) - got[B - 1]) <= 1e-6 * T
    # the device bpb path with every token one byte long: bytes = T per row
    # and nats = the row sums
    bp = m.eval_bpb(rows, np.ones(d.vocab, np.int32), batch=B)
    assert np.all(bp["row_bytes"] == T)
    assert np.all(np.abs(bp["row_nats"] - ref) <= 1e-4 * T)
    m.close()


# Steps of the batched decode whose logits the tests keep (64 steps x 64
# sequences x 8192 fp32 = 128 MiB a run).
B64_LOGIT_STEPS = 64


@functools.lru_cache(maxsize=2)
def b64_run(bf16):
    """The batched-decode workload: 64 sequences, their 1023-id prompts
    through one chunked pass, then 512 greedy steps. Returns the ids [B, n]
    and the logits of the first B64_LOGIT_STEPS steps [steps, B, V]."""
    g = fixture("decode_b64_d12")
    d, B, P, n = D12, g["B"], g["P"], g["steps"]
    prompts = uniform_ids(g["seed"], B * P, d.vocab).reshape(B, P)
    m = model(d, g["weights_seed"], P + n)
    kv = m.kv(B, P + n, bf16=bf16)
    kv.step_multi(prompts[:, :-1], want_logits=False)
    ids1, lg = kv.decode_greedy(prompts[:, -1], B64_LOGIT_STEPS, want_logits=True)
    ids2, _ = kv.decode_greedy(ids1[-1], n - B64_LOGIT_STEPS)
    kv.close()
    m.close()
    return np.concatenate([ids1, ids2]).T, lg  # [B, n], [steps, B, V]


def first_flips(got, ref):
    out = {}
    for b in range(ref.shape[0]):
        diff = np.nonzero(got[b] != ref[b])[0]
        if diff.size:
            out[b] = int(diff[0])
    return out


def top2(lg):
    """Indices of the largest and second-largest logit along the last axis
    (first index on ties, as the argmax takes it) and their margin."""
    a = np.argmax(lg, axis=-1)
    rest = lg.copy()
    np.put_along_axis(rest, a[..., None], -np.inf, axis=-1)
    b = np.argmax(rest, axis=-1)
    la = np.take_along_axis(lg, a[..., None], -1)[..., 0]
    lb = np.take_along_axis(lg, b[..., None], -1)[..., 0]
    return a, b, la - lb


def agree_mask(got, ref, steps):
    """[steps, B]: True where every id of sequence b before step t agrees
    (the input of step t is the id of step t - 1), so both runs decode the
    same context at step t and their logits there are comparable."""
    same = (got[:, :steps] == ref[:, :steps]).T  # [steps, B]
    ok = np.cumprod(same, axis=0).astype(bool)
    return np.vstack([np.ones((1, same.shape[1]), bool), ok[:-1]])


# Top-2 logit margin below which two fp32 evaluations of the same logits in
# different summation orders can rank the two ids either way: the engine's
# logits sit within ~5e-6 x max|logit| of the oracle's (|logit| < 20 here),
# and the reference itself accepts 1e-4 between two GEMM orders
# (test_linear_blas, src/test/test_kernels.f90:2156-2177).
FP32_TIE = 1e-4


def test_decode_b64_prompt1024_steps512():
    """Batched greedy decode: 64 sequences, 1024-id prompts, 512 steps, every
    sequence's ids against the oracle's (fp32 cache). A sequence may leave
    the oracle's stream only at a step whose oracle top-2 margin is an fp32
    tie (below FP32_TIE); every such flip is printed. Over the first
    B64_LOGIT_STEPS steps the engine's top-2 margin of every sequence must
    also equal the oracle's within FP32_TIE / 2, so an error in the cached
    prompt shows up even where it flips no id."""
    ref = np.load(os.path.join(GOLD, "decode_b64_d12_ids.npy"))
    marg = np.load(os.path.join(GOLD, "decode_b64_d12_margins.npy"))
    got, lg = b64_run(False)
    flips = first_flips(got, ref)
    print(f"fp32 cache: {64 - len(flips)} of 64 sequences identical over 512 steps;",
          "first flips (seq: step, oracle margin):",
          {b: (t, float(marg[b, t])) for b, t in flips.items()},
          "smallest oracle margin", float(marg.min()))
    S = lg.shape[0]
    ok = agree_mask(got, ref, S)
    _, _, mg = top2(lg)
    dm = np.abs(mg - marg[:, :S].T)[ok]
    print(f"fp32 cache: top-2 margin vs the oracle's over {int(ok.sum())} steps: "
          f"max |d| {dm.max():.3g}, mean {dm.mean():.3g}")
    assert dm.max() < FP32_TIE / 2
    assert len(flips) <= 2
    for b, t in flips.items():
        assert marg[b, t] < FP32_TIE, (b, t, float(marg[b, t]))


def test_decode_b64_bf16_cache_vs_oracle():
    """The same workload on the bf16 cache the workload states. The bar is
    measured here: over the first B64_LOGIT_STEPS steps, the change that the
    bf16 cache alone makes to each sequence's top-2 margin (bf16-cache run
    against the fp32-cache run, the fp32 run's top-2 ids, steps whose
    context both runs share). A sequence may leave the fp32 oracle's ids only
    at a step whose oracle margin is below 1.5 x the largest such change;
    every first flip is printed with its margin."""
    ref = np.load(os.path.join(GOLD, "decode_b64_d12_ids.npy"))
    marg = np.load(os.path.join(GOLD, "decode_b64_d12_margins.npy"))
    got, lg16 = b64_run(True)
    got32, lg32 = b64_run(False)
    S = lg16.shape[0]
    a, b2, m32 = top2(lg32)
    m16 = (np.take_along_axis(lg16, a[..., None], -1) - np.take_along_axis(lg16, b2[..., None], -1))[..., 0]
    both = agree_mask(got, got32, S) & agree_mask(got32, ref, S)
    dmax = float(np.abs(m16 - m32)[both].max())
    bar = 1.5 * dmax
    flips = first_flips(got, ref)
    same = 64 - len(flips)
    print(f"bf16 cache: top-2 margin change from the bf16 cache, max over {int(both.sum())} "
          f"steps {dmax:.3g}: flip bar {bar:.3g};",
          f"{same} of 64 sequences identical over 512 steps;",
          "first flips (seq: step, oracle margin):",
          {b: (t, round(float(marg[b, t]), 6)) for b, t in flips.items()})
    for b, t in flips.items():
        assert marg[b, t] < bar, (b, t, float(marg[b, t]), bar)


def test_gqa20_prefill2048_decode256():
    """Depth-20 GQA (10 query heads over 2 KV heads): prefill and 256 steps."""
    g = fixture("gqa20_decode")
    d, P, n = GQA20, g["P"], g["steps"]
    prompt = uniform_ids(g["seed"], P, d.vocab)
    m = model(d, g["weights_seed"], P + n)
    lg, _ = m.forward(prompt, 1, P)
    lg = lg.reshape(P, d.vocab)
    last = np.load(os.path.join(GOLD, "gqa20_prefill_last.npy"))
    rel = float(np.abs(lg[-1].astype(np.float64) - last).max() / np.abs(last).max())
    print("gqa20 last prefill row rel err", rel)
    assert rel < TOL
    rows = np.load(os.path.join(GOLD, "gqa20_prefill_rows.npy"))
    idx = list(range(0, P, 128)) + [P - 1]
    relr = float(np.abs(lg[idx].astype(np.float64) - rows).max() / np.abs(rows).max())
    print(f"gqa20 prefill rows {idx[0]}..{idx[-1]} (every 128th + last) rel err", relr)
    assert relr < TOL
    kv = m.kv(1, P + n)
    kv.step_multi(prompt[None, :-1], want_logits=False)
    ids = kv.decode_greedy(prompt[None, -1:], n)[0][:, 0]
    ref = np.array(g["ids"], dtype=np.int32)
    first = int(np.argmax(ids != ref)) if not np.array_equal(ids, ref) else -1
    print(f"gqa20 decode: first mismatch {first}, oracle min top-2 margin {g['min_top2_margin']:.3g}")
    assert np.array_equal(ids, ref)
    kv.close()
    m.close()
