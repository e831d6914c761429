"""FG_OPT_FORWARD_F16, the single-term fp16 forward, against the CPU oracle.

With the option on, forward and eval passes of more than 128 token rows run
their GEMMs and chunk attention as one fp16 MFMA per product (activations
rounded once to fp16, weights an exact fp16 copy scaled by a power of 2).
The bar is the engine's contract, logits within 2e-3 x max|logit| of the
oracle; a row's argmax may differ from the oracle's only where the oracle's
own top-2 margin is below twice the largest logit error measured, the
bound under which a flip is possible at all. Passes of 128 rows or fewer,
cached steps and chunked prefill keep the split format bit for bit.
"""
import json
import os

import numpy as np
import pytest

from autoresearch_amd import engine
from autoresearch_amd.weights import (D12, GQA20, Dims, rope_tables, seeded_weights, uniform_ids,
                                      zipf_ids)
from oracle import oracle as O

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
TOL = 2e-3
SMALL = Dims(n_layer=2, d_model=128, n_head=2, n_kv_head=1, head_dim=64, vocab=512)
SMALL_MHA = Dims(n_layer=2, d_model=256, n_head=2, n_kv_head=2, head_dim=128, vocab=1024)


def relerr(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / np.max(np.abs(b)))


def tables(d, T):
    c, s = rope_tables(T, d.head_dim)
    return c.reshape(-1), s.reshape(-1)


def flips_within_bound(got, ref):
    """Rows whose argmax differs, and whether each such row's oracle top-2
    margin is below 2 x the largest |logit error| (else the flip is a bug)."""
    got = np.asarray(got, np.float64).reshape(ref.shape)
    err = float(np.abs(got - ref).max())
    srt = np.sort(ref, -1)
    margin = srt[..., -1] - srt[..., -2]
    bad = got.argmax(-1) != ref.argmax(-1)
    return int(bad.sum()), bool(np.all(margin[bad] <= 2 * err)), err


@pytest.fixture(scope="module")
def d12():
    w = seeded_weights(D12, 1234)
    m = engine.Model(D12, stacks=w)
    c, s = tables(D12, 2304)
    m.set_rope(c, s)
    yield D12, w, m, c, s
    m.close()


def test_option_round_trip(d12):
    d, w, m, c, s = d12
    assert m.forward_f16() is False
    wb0, _ = m.bytes()
    m.set_forward_f16(True)
    assert m.forward_f16() is True
    wb1, _ = m.bytes()
    assert wb1 == 2 * wb0  # the fp16 copy has the arena's size
    m.set_forward_f16(False)
    assert m.forward_f16() is False
    assert m.bytes()[0] == wb0  # the copy is released with the option
    with pytest.raises(engine.FgptError):
        engine._check(engine._LIB.fg_set_option(m._h, 99, 1))


def test_prefill_d12_T2048_f16_vs_oracle(d12):
    """The prefill workload's own size, T = 2048, logits and per-token CE."""
    d, w, m, c, s = d12
    T = 2048
    ids = uniform_ids(2, T + 1, d.vocab)
    lg_split, nll_split = m.forward(ids[:T], 1, T, targets=ids[1:])
    m.set_forward_f16(True)
    try:
        lg, nll = m.forward(ids[:T], 1, T, targets=ids[1:])
        lg2, nll2 = m.forward(ids[:T], 1, T, targets=ids[1:])
    finally:
        m.set_forward_f16(False)
    ref = O.gpt_forward(ids[:T], c, s, w, d, 1, T).reshape(T, d.vocab)
    e = relerr(lg, ref)
    ref_nll = O.nll(ref, ids[1:], d.vocab)
    dn = float(np.max(np.abs(nll.reshape(-1) - ref_nll)))
    nflip, bounded, err = flips_within_bound(lg, ref)
    print(f"f16 prefill T=2048: relerr {e:.3g} (split {relerr(lg_split, ref):.3g}), "
          f"max|d nll| {dn:.3g}, argmax flips {nflip} of {T} (within the margin bound: {bounded})",
          flush=True)
    assert e < TOL
    assert dn < 2 * TOL * np.abs(ref).max()
    assert bounded
    # fixed summation order: a second pass gives the same bits
    assert np.array_equal(lg, lg2) and np.array_equal(nll, nll2)
    # and turning the option off restores the split results exactly
    lg3, _ = m.forward(ids[:T], 1, T, targets=ids[1:])
    assert np.array_equal(lg3, lg_split)


def test_eval_rows_b8_t2048_f16():
    """B=8 x 2048 Zipf rows with BOS, the summed nats per row against the
    oracle's committed sums, and the device bpb path with the option on."""
    with open(os.path.join(GOLD, "eval_rows_d12.json")) as f:
        g = json.load(f)
    d, B, T = D12, g["B"], g["T"]
    rows = zipf_ids(g["seed"], B * (T + 1), d.vocab).reshape(B, T + 1)
    rows[:, 0] = g["bos"]
    m = engine.Model(d, stacks=seeded_weights(d, g["weights_seed"]))
    c, s = tables(d, T)
    m.set_rope(c, s)
    m.set_forward_f16(True)
    lg, nll = m.forward(rows[:, :T], B, T, targets=rows[:, 1:])
    maxlogit = float(np.abs(lg).max())
    got = nll.astype(np.float64).sum(axis=1)
    ref = np.array(g["nats"])
    print("f16 eval rows: max |d nats| per row", np.abs(got - ref).max(), "per token",
          np.abs(got - ref).max() / T, "max|logit|", maxlogit, flush=True)
    assert np.all(np.abs(got - ref) <= 2 * TOL * maxlogit * T)
    bp = m.eval_bpb(rows, np.ones(d.vocab, np.int32), batch=B)
    assert np.all(bp["row_bytes"] == T)
    assert np.allclose(bp["row_nats"], got, rtol=0, atol=1e-6 * T)
    m.close()


@pytest.mark.parametrize("d", [SMALL, SMALL_MHA], ids=["gqa", "mha"])
@pytest.mark.parametrize("B,T", [(1, 100), (2, 64), (3, 130), (1, 300), (2, 257), (3, 500)])
def test_forward_small_f16(d, B, T):
    """Small models: above 128 rows within the bar, at or below 128 rows the
    split format's exact bits."""
    w = seeded_weights(d, 7)
    ids = uniform_ids(B * 100 + T, B * T, d.vocab)
    c, s = tables(d, T)
    m = engine.Model(d, stacks=w)
    m.set_rope(c, s)
    tg = np.roll(ids, -1)
    lg0, nll0 = m.forward(ids, B, T, targets=tg)
    m.set_forward_f16(True)
    lg, nll = m.forward(ids, B, T, targets=tg)
    if B * T <= 128:
        assert np.array_equal(lg, lg0) and np.array_equal(nll, nll0)
    ref = O.gpt_forward(ids, c, s, w, d, B, T)
    e = relerr(lg, ref)
    print(f"f16 small {d} B={B} T={T}: relerr {e:.3g}", flush=True)
    assert e < TOL
    ref_nll = O.nll(ref.reshape(-1, d.vocab), tg, d.vocab)
    assert np.max(np.abs(nll.reshape(-1) - ref_nll)) < 2 * TOL * np.abs(ref).max()
    nflip, bounded, _ = flips_within_bound(lg.reshape(ref.shape), ref)
    assert bounded
    m.close()


def test_cached_paths_keep_split_format(d12):
    """fg_step_multi (chunked prefill into the cache) and greedy decode give
    the same bits with the option on as with it off."""
    d, w, m, c, s = d12
    prompt = uniform_ids(42, 300, d.vocab)
    out = []
    for on in (False, True):
        m.set_forward_f16(on)
        kv = m.kv(1, 340)
        lg, nxt = kv.step_multi(prompt[:-1])
        ids, _ = kv.decode_greedy(prompt[-1:], 8)
        k, v = kv.read()
        out.append((lg, nxt, ids, k, v))
        kv.close()
    m.set_forward_f16(False)
    for a, b in zip(out[0], out[1]):
        assert np.array_equal(a, b)


def test_gqa20_prefill2048_f16_rows():
    """Depth-20 GQA model (10 query heads over 2 KV heads), T=2048 prefill:
    the oracle's committed rows 0, 128, ..., 1920 and 2047."""
    with open(os.path.join(GOLD, "gqa20_decode.json")) as f:
        g = json.load(f)
    d, P = GQA20, g["P"]
    prompt = uniform_ids(g["seed"], P, d.vocab)
    m = engine.Model(d, stacks=seeded_weights(d, g["weights_seed"]))
    c, s = tables(d, P)
    m.set_rope(c, s)
    m.set_forward_f16(True)
    lg, _ = m.forward(prompt, 1, P)
    lg = lg.reshape(P, d.vocab)
    rows = np.load(os.path.join(GOLD, "gqa20_prefill_rows.npy"))
    idx = list(range(0, P, 128)) + [P - 1]
    e = relerr(lg[idx], rows)
    nflip, bounded, _ = flips_within_bound(lg[idx], rows)
    print(f"f16 gqa20 prefill rows: relerr {e:.3g}, argmax flips {nflip} of {len(idx)}",
          flush=True)
    assert e < TOL
    assert bounded
    m.close()


def test_f16_overflow_is_an_error():
    """An activation beyond fp16's range fails the pass with FG_ERANGE
    instead of returning inf / NaN logits. c_fc scaled by 2^10 (still
    bf16-exact) puts relu^2 of the fc outputs far above 65504: fg_forward,
    fg_eval_bpb and a device-pointer pass (reported at the next fg_sync)
    refuse with the option on; the split path computes the same rows with
    finite logits, and the flag does not outlive its report."""
    from tests.devbuf import DevBuf
    d = SMALL
    w = seeded_weights(d, 9)
    w["c_fc"] = (w["c_fc"] * np.float32(1024.0)).astype(np.float32)
    B, T = 2, 200
    ids = uniform_ids(10, B * T, d.vocab)
    c, s = tables(d, T)
    m = engine.Model(d, stacks=w)
    m.set_rope(c, s)
    lg, _ = m.forward(ids, B, T)
    assert np.isfinite(lg).all()
    m.set_forward_f16(True)
    with pytest.raises(engine.FgptError) as e:
        m.forward(ids, B, T)
    assert e.value.code == -10 and "fp16" in str(e.value)
    rows = np.concatenate([ids.reshape(B, T), ids.reshape(B, T)[:, :1]], axis=1)
    with pytest.raises(engine.FgptError) as e:
        m.eval_bpb(rows, np.ones(d.vocab, np.int32), batch=B)
    assert e.value.code == -10
    d_ids = DevBuf(ids.astype(np.int32))
    d_lg = DevBuf(np.zeros(B * T * d.vocab, np.float32))
    m.forward_dev(d_ids.ptr, B, T, d_lg.ptr)
    with pytest.raises(engine.FgptError) as e:
        m.sync()
    assert e.value.code == -10
    m.sync()  # reported once
    d_ids.free()
    d_lg.free()
    # the same weights without the scale pass on the fp16 path
    m.close()
    w["c_fc"] = (w["c_fc"] / np.float32(1024.0)).astype(np.float32)
    m = engine.Model(d, stacks=w)
    m.set_rope(c, s)
    m.set_forward_f16(True)
    lg16, _ = m.forward(ids, B, T)
    assert np.isfinite(lg16).all()
    m.close()
