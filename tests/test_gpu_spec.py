"""Greedy speculative decoding on the GPU (fg_decode_spec), through the C ABI.

The reference's invariant (src/app/spec_bench.f90:165-171): the committed
stream equals the target's plain greedy stream. Here it is checked bit for
bit against fg_decode_greedy on the same weights and prefill, the greedy
stream against the CPU oracle, the cache left behind against the greedy
run's, and the loop's counters against the oracle's replay of the
chat_text.f90:293-422 schedule over that stream.
"""
import time

import numpy as np
import pytest

from autoresearch_amd import engine
from autoresearch_amd.weights import D12, Dims, rope_tables, seeded_weights, uniform_ids
from oracle import oracle as O
from oracle import spec as S

pytestmark = pytest.mark.gpu

SMALL = Dims(n_layer=2, d_model=128, n_head=2, n_kv_head=1, head_dim=64, vocab=512)
SMALL_MHA = Dims(n_layer=2, d_model=256, n_head=2, n_kv_head=2, head_dim=128, vocab=1024)


def repetitive_prompt(seed, vocab, period=12, reps=3, extra=5):
    base = uniform_ids(seed, period, vocab)
    return np.concatenate([np.tile(base, reps), base[:extra]]).astype(np.int32)


def prefill(m, prompt, maxT):
    kv = m.kv(1, maxT)
    n = prompt.size - 1
    s = 0
    while s < n:
        tb = min(64, n - s)
        kv.step_multi(prompt[s:s + tb], want_logits=False)
        s += tb
    return kv


def greedy_and_spec(d, m, prompt, n_gen, runs=1, **cfg):
    """Greedy and speculative continuations from the same prefill; with
    runs > 1 each is repeated from the prefill state (graphs captured by the
    first run) and the last run is timed. The greedy run takes the
    per-kernel steps (the persistent loop off): the verification pass
    computes every row as that step does, so stream and cache must be equal
    bit for bit; the persistent loop sums in another order (logits within
    ~1e-6 relative of the steps)."""
    ntot = prompt.size + n_gen
    kv = prefill(m, prompt, ntot)
    m.set_fused_decode(False)
    try:
        for _ in range(runs):
            kv.len = prompt.size - 1
            t0 = time.perf_counter()
            g, _ = kv.decode_greedy(prompt[-1:], n_gen)
            t_g = time.perf_counter() - t0
    finally:
        m.set_fused_decode(True)
    gk, gv = kv.read()
    kv.close()
    kv = prefill(m, prompt, ntot)
    for _ in range(runs):
        kv.len = prompt.size - 1
        t0 = time.perf_counter()
        out, st = kv.decode_spec(prompt, n_gen, **cfg)
        t_s = time.perf_counter() - t0
    assert kv.len == ntot - 1
    sk, sv = kv.read()
    kv.close()
    shape = (d.n_layer, ntot, d.n_kv_head * d.head_dim)
    used = slice(0, ntot - 1)
    dk = np.abs(gk.reshape(shape)[:, used] - sk.reshape(shape)[:, used]).max()
    dv = np.abs(gv.reshape(shape)[:, used] - sv.reshape(shape)[:, used]).max()
    return g[:, 0], out, st, (dk, dv), (t_g, t_s)


@pytest.mark.parametrize("d", [SMALL, SMALL_MHA], ids=["gqa", "mha"])
@pytest.mark.parametrize("k,probe,min_acc", [(8, 8, 0.5), (3, 1, 2.0), (15, 4, 0.0)])
def test_spec_equals_greedy_small(d, k, probe, min_acc):
    w = seeded_weights(d, 11)
    prompt = repetitive_prompt(d.vocab + k, d.vocab)
    n_gen = 100
    ntot = prompt.size + n_gen
    c, s = rope_tables(ntot, d.head_dim)
    m = engine.Model(d, stacks=w)
    m.set_rope(c.reshape(-1), s.reshape(-1))
    g, out, st, (dk, dv), _ = greedy_and_spec(d, m, prompt, n_gen, k=k, match=2, probe=probe,
                                              min_acc=min_acc)
    m.close()
    print(f"spec {d} k={k} probe={probe} min_acc={min_acc}: {st} cache dk={dk} dv={dv}",
          flush=True)
    assert np.array_equal(out, g)
    # every verification row is computed as the step at its position
    assert dk == 0 and dv == 0
    _, want = S.spec_schedule(prompt.tolist(), g.tolist(), k, 2, probe, min_acc)
    assert st == want
    assert st["passes"] > 0
    # the greedy stream itself against the CPU oracle
    ref, _ = O.greedy_decode(prompt, w, d, n_gen, c.reshape(-1), s.reshape(-1), ntot)
    assert np.array_equal(ref, g)


def test_spec_equals_greedy_d12():
    d = D12
    w = seeded_weights(d, 1234)
    prompt = repetitive_prompt(77, d.vocab, period=24, reps=3, extra=16)
    n_gen = 256
    ntot = prompt.size + n_gen
    c, s = rope_tables(ntot, d.head_dim)
    m = engine.Model(d, stacks=w)
    m.set_rope(c.reshape(-1), s.reshape(-1))
    g, out, st, (dk, dv), (t_g, t_s) = greedy_and_spec(d, m, prompt, n_gen, runs=2, k=8,
                                                       match=2, probe=8, min_acc=0.5)
    m.close()
    print(f"spec d12 prompt={prompt.size} gen={n_gen}: {st} greedy {n_gen / t_g:.0f} tok/s, "
          f"spec {n_gen / t_s:.0f} tok/s, cache dk={dk} dv={dv}", flush=True)
    assert np.array_equal(out, g)
    assert dk == 0 and dv == 0
    _, want = S.spec_schedule(prompt.tolist(), g.tolist(), 8, 2, 8, 0.5)
    assert st == want


def test_spec_errors_are_loud():
    d = SMALL
    m = engine.Model(d, stacks=seeded_weights(d, 3))
    c, s = rope_tables(64, d.head_dim)
    m.set_rope(c.reshape(-1), s.reshape(-1))
    prompt = repetitive_prompt(1, d.vocab)[:20]
    kv2 = m.kv(2, 64)
    with pytest.raises(engine.FgptError, match="B=1"):
        kv2.decode_spec(prompt, 4)
    kv2.close()
    kv = prefill(m, prompt, 64)
    for bad in (dict(k=0), dict(k=16), dict(match=0), dict(probe=0)):
        with pytest.raises(engine.FgptError):
            kv.decode_spec(prompt, 4, **bad)
    with pytest.raises(engine.FgptError, match="n_known-1"):
        kv.decode_spec(prompt[:-1], 4)
    with pytest.raises(engine.CacheFull):
        kv.decode_spec(prompt, 64)
    # nothing above ran a pass: the cache is where the prefill left it
    assert kv.len == prompt.size - 1
    out, st = kv.decode_spec(prompt, 0)
    assert out.size == 0 and st["passes"] == 0 and kv.len == prompt.size - 1
    kv.close()
    m.close()
