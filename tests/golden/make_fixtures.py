#!/usr/bin/env python3
"""Write the oracle's outputs for the full-size workloads as fixtures.

The CPU oracle (oracle/, a restatement of the reference loops) is too slow to
run inside the GPU test session at these sizes, so its results are computed
once here, on seeded inputs the tests regenerate bit for bit, and committed:

- eval_rows_d12.json   B=8 rows of 2049 Zipf(1.1) ids, BOS at position 0;
                       summed NLL (nats) of each row, depth-12 seeded model
                       (rows run one at a time, as eval_bpb --batch 1 does).
- decode_b64_d12.json  64 prompts of 1024 uniform ids; for sequences 0 and
                       63: chunked prefill of prompt[:-1], then 512 greedy
                       gpt_step ids (one sequence at a time).
- decode_b64_d12_ids.npy, decode_b64_d12_margins.npy  the same for all 64
                       sequences: int32 ids [64, 512] and the float32 top-2
                       logit margin of every step [64, 512]; sequences 0
                       and 63 must equal the run above.
- gqa20_decode.json    depth-20 GQA model, a 2048-id uniform prompt: chunked
                       prefill of prompt[:-1], then 256 greedy ids.
- gqa20_prefill_last.npy  the last row of gpt_forward logits for that prompt
                       (T = 2048), float32.
- gqa20_prefill_rows.npy  rows 0, 128, ..., 1920 and 2047 of those logits,
                       float32 [17, 8192].

    python tests/golden/make_fixtures.py [--only NAME]

(--only decode_b64_all and --only gqa20_rows each run a few minutes on 8
cores; the default runs every job.)
"""
import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from autoresearch_amd.weights import (BOS_ID, D12, GQA20, rope_tables, seeded_weights,  # noqa: E402
                                      uniform_ids, zipf_ids)
from oracle import oracle as O  # noqa: E402

SEED_D12, SEED_GQA = 1234, 4321
EVAL = dict(seed=31, B=8, T=2048)
B64 = dict(seed=64, B=64, P=1024, steps=512, seqs=[0, 63])
GQA = dict(seed=20, P=2048, steps=256)


def tables(d, n):
    c, s = rope_tables(n, d.head_dim)
    return c.reshape(-1), s.reshape(-1)


def eval_rows():
    d, w = D12, seeded_weights(D12, SEED_D12)
    B, T = EVAL["B"], EVAL["T"]
    rows = zipf_ids(EVAL["seed"], B * (T + 1), d.vocab).reshape(B, T + 1)
    rows[:, 0] = BOS_ID
    c, s = tables(d, T)
    nats = []
    for b in range(B):
        lg = O.gpt_forward(rows[b, :T], c, s, w, d, 1, T).reshape(T, d.vocab)
        nats.append(float(O.nll(lg, rows[b, 1:], d.vocab).astype(np.float64).sum()))
    return {**EVAL, "weights_seed": SEED_D12, "bos": BOS_ID, "nats": nats}


def decode_b64():
    d, w = D12, seeded_weights(D12, SEED_D12)
    B, P, n = B64["B"], B64["P"], B64["steps"]
    prompts = uniform_ids(B64["seed"], B * P, d.vocab).reshape(B, P)
    c, s = tables(d, P + n)
    out = {}
    for b in B64["seqs"]:
        ids, lg = O.greedy_decode(prompts[b], w, d, n, c, s, maxT=P + n, prefill_multi=True)
        top2 = np.sort(lg, axis=1)[:, -2:]
        out[str(b)] = {"ids": ids.tolist(), "min_top2_margin": float((top2[:, 1] - top2[:, 0]).min())}
    return {**B64, "weights_seed": SEED_D12, "sequences": out}


def gqa20():
    d, w = GQA20, seeded_weights(GQA20, SEED_GQA)
    P, n = GQA["P"], GQA["steps"]
    prompt = uniform_ids(GQA["seed"], P, d.vocab)
    c, s = tables(d, P + n)
    lg = O.gpt_forward(prompt, c, s, w, d, 1, P).reshape(P, d.vocab)
    np.save(os.path.join(HERE, "gqa20_prefill_last.npy"), lg[-1].astype(np.float32))
    ids, slg = O.greedy_decode(prompt, w, d, n, c, s, maxT=P + n, prefill_multi=True)
    top2 = np.sort(slg, axis=1)[:, -2:]
    return {**GQA, "weights_seed": SEED_GQA, "ids": ids.tolist(),
            "min_top2_margin": float((top2[:, 1] - top2[:, 0]).min())}


def decode_b64_all():
    """All 64 sequences, each run alone as decode_b64 runs two of them (the
    reference's cache layout serves one sequence per call), with the
    transposed weight copies kept between calls (or_wt_cache)."""
    d, w = D12, seeded_weights(D12, SEED_D12)
    B, P, n = B64["B"], B64["P"], B64["steps"]
    prompts = uniform_ids(B64["seed"], B * P, d.vocab).reshape(B, P)
    c, s = tables(d, P + n)
    ws = {k: O.f32(v) for k, v in w.items()}
    ids = np.zeros((B, n), np.int32)
    margins = np.zeros((B, n), np.float32)
    O.lib().or_wt_cache(1)
    try:
        for b in range(B):
            got, lg = O.greedy_decode(prompts[b], ws, d, n, c, s, maxT=P + n, prefill_multi=True)
            top2 = np.sort(lg, axis=1)[:, -2:]
            ids[b] = got
            margins[b] = top2[:, 1] - top2[:, 0]
            print(f"  sequence {b}: min margin {margins[b].min():.3g}", flush=True)
    finally:
        O.lib().or_wt_cache(0)
    old = json.load(open(os.path.join(HERE, "decode_b64_d12.json")))
    for b, rec in old["sequences"].items():
        assert np.array_equal(ids[int(b)], rec["ids"]), f"sequence {b} differs from the earlier run"
    np.save(os.path.join(HERE, "decode_b64_d12_ids.npy"), ids)
    np.save(os.path.join(HERE, "decode_b64_d12_margins.npy"), margins)
    return None


GQA_ROWS = list(range(0, 2048, 128)) + [2047]


def gqa20_rows():
    d, w = GQA20, seeded_weights(GQA20, SEED_GQA)
    P = GQA["P"]
    prompt = uniform_ids(GQA["seed"], P, d.vocab)
    c, s = tables(d, P)
    lg = O.gpt_forward(prompt, c, s, w, d, 1, P).reshape(P, d.vocab)
    last = np.load(os.path.join(HERE, "gqa20_prefill_last.npy"))
    assert np.array_equal(lg[-1], last)
    np.save(os.path.join(HERE, "gqa20_prefill_rows.npy"), lg[GQA_ROWS].astype(np.float32))
    return None


JOBS = {"eval_rows_d12": eval_rows, "decode_b64_d12": decode_b64, "gqa20_decode": gqa20,
        "decode_b64_all": decode_b64_all, "gqa20_rows": gqa20_rows}

if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", choices=sorted(JOBS))
    a = ap.parse_args()
    for name, fn in JOBS.items():
        if a.only and a.only != name:
            continue
        t0 = time.time()
        rec = fn()
        if rec is not None:  # (the others write .npy files)
            rec["oracle_threads"] = int(O.lib().or_num_threads())
            with open(os.path.join(HERE, name + ".json"), "w") as f:
                json.dump(rec, f)
        print(f"{name}: {time.time() - t0:.1f} s", flush=True)
