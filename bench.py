#!/usr/bin/env python3
"""Benchmark of the MI355X engine for the fortran_gpt forward path.

One JSON line on stdout. `value` is the prefill throughput of the depth-12
model at B=1, T=2048 (logits [2048, 8192] plus per-token cross-entropy, ids
and targets already resident in HBM), one "step" being one full forward, with
FG_OPT_FORWARD_F16 on (one fp16 MFMA per product: activations rounded once
to fp16, weights an exact fp16 copy; logits within ~4e-4 x max|logit| of the
fp32 forward), the split-bf16 default (2 MFMAs per product, ~5e-6) beside it
under "split"; the B=8 eval rows likewise. Beside it, each with its own
roofline and the profiles/ summary it reproduces from: the B=1 greedy decode (16-id prompt, 32 cached steps), the
B=8 x 2048 Zipf eval rows, the B=64 batched decode (1024-id prompts, 512
steps, on the bf16 KV cache the workload states, and on the fp32 cache
beside it), the depth-20 GQA model (2048-id prefill, 256 steps), speculative and
sampled decoding; and the CPU oracle timed on this host's cores on a bounded
sample.

Rooflines use algorithmic units: bf16 weights read once per step, K and V of
a cached position as bf16 (36 864 B per position at depth 12), 2 M N K flops
per linear and the causal half of attention for prefill.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--skip NAME]
                    [--only NAME] [--operands both|f16|split] [--no-pmc]
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import math
import os
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tok/s (B=1, B=64) + prefill tok/s, depth-12; % HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_BF16_PEAK_TFS = 2516.6    # 256 CU x 2.4 GHz x 4096 bf16 flop/clk, dense (fp16: the same)
SEED = 1234                    # depth-12 weights
SEED_GQA = 4321                # depth-20 GQA weights
# executed MFMA work per algorithmic flop: the linears multiply the exact
# bf16 weights by the activation's hi and lo planes (2 MFMAs), the chunk
# attention takes hi*hi + hi*lo + lo*hi (3)
MFMA_EXEC = {"gemm": 2.0, "attn_chunk": 3.0}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# --- algorithmic units: bf16 weights read once per step, bf16 KV positions
def kv_pos_bytes(d) -> int:
    """K and V of one position over all layers, bf16 (the unit of the
    decode rooflines; the engine's default cache holds them in fp32)."""
    return 2 * d.n_layer * d.n_kv_head * d.head_dim * 2


def decode_step_bytes(d, B: int, n: int) -> float:
    """One greedy step of B sequences whose caches hold n positions before
    it: every weight but the embedding table once, one embedding row per
    sequence, n+1 cached positions read and one written per sequence."""
    return 2.0 * (d.params - d.vocab * d.d_model) + B * (2.0 * d.d_model + kv_pos_bytes(d) * (n + 2))


def prefill_flops(d, B: int, T: int) -> float:
    """2 T (params - V D) for the linears plus 4 hd H L T(T+1)/2 for the
    causal half of attention, per row."""
    lin = 2.0 * T * (d.params - d.vocab * d.d_model)
    att = 4.0 * d.head_dim * d.n_head * d.n_layer * T * (T + 1) / 2
    return B * (lin + att)


def roofline(rec, alg_total: float, bound: str, kind: str, profile: str,
             mfma_exec: float = None) -> dict:
    """achieved = algorithmic bytes (or flops) per launch / mean launch time,
    the launches of one kernel kind from a pass with every launch bracketed
    by HIP events on its stream (fg_timing)."""
    n, ms = rec[0], rec[1]
    per_s = ms * 1e-3 / max(n, 1)
    per_unit = alg_total / max(n, 1)
    if bound == "mfma":
        achieved, peak, unit = per_unit / per_s / 1e12, MFMA_BF16_PEAK_TFS, "TFLOP/s"
    else:
        achieved, peak, unit = per_unit / per_s / 1e9, HBM_PEAK_GBS, "GB/s"
    out = {"bound": bound, "kernel_kind": kind, "launches": n, "avg_launch_us": per_s * 1e6,
           ("alg_flop_per_launch" if bound == "mfma" else "alg_bytes_per_launch"): per_unit,
           "achieved": achieved, "peak": peak, "unit": unit, "frac": achieved / peak,
           "traffic": None, "profile": profile}
    ex = mfma_exec if mfma_exec is not None else MFMA_EXEC.get(kind)
    if ex is not None:
        out["mfma_executed_frac"] = out["frac"] * ex
    return out


def timing_pass(m, fn, reps: int = 1) -> dict:
    m.timing(True)
    for _ in range(reps):
        fn()
    m.sync()
    tm = m.timing_read()
    m.timing(False)
    return tm


def dominant(tm: dict) -> str:
    return max(tm, key=lambda k: tm[k][1])


def event_time(torch, st, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(st):
        e0.record(st)
        for _ in range(steps):
            fn()
        e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def bench_forward(m, d, torch, B, T, ids, steps, warmup, profile, f16=False):
    """Forward of B rows of T ids with per-token NLL against ids shifted by
    one, ids/targets/logits/NLL resident in HBM, timed with HIP events on the
    stream the engine launches on; then an fg_timing pass for the kernels.
    f16: with FG_OPT_FORWARD_F16 on (one fp16 MFMA per product instead of
    the split format's 2 in the linears and 3 in attention)."""
    m.set_forward_f16(f16)
    try:
        return _bench_forward(m, d, torch, B, T, ids, steps, warmup, profile, f16)
    finally:
        m.set_forward_f16(False)


_FWD_STREAM = []


def forward_stream(torch):
    """The one stream every forward measurement runs on. Each stream a process
    has used takes a hardware queue (GPU_MAX_HW_QUEUES is 4 here); with two
    more than torch's and the engine's in use, the sampled decode's queued
    single-step launches ran ~40 % slower, so the benches share one."""
    if not _FWD_STREAM:
        _FWD_STREAM.append(torch.cuda.Stream())
    return _FWD_STREAM[0]


def _bench_forward(m, d, torch, B, T, ids, steps, warmup, profile, f16):
    dev = torch.device("cuda:0")
    ids = np.asarray(ids, np.int32).reshape(B, T + 1)
    d_ids = torch.from_numpy(np.ascontiguousarray(ids[:, :T])).to(dev)
    d_tgt = torch.from_numpy(np.ascontiguousarray(ids[:, 1:])).to(dev)
    d_lg = torch.empty(B * T * d.vocab, dtype=torch.float32, device=dev)
    d_nll = torch.empty(B * T, dtype=torch.float32, device=dev)
    st = forward_stream(torch)  # a real stream handle: events and kernels share it
    run = lambda: m.forward_dev(d_ids.data_ptr(), B, T, d_lg.data_ptr(), d_tgt.data_ptr(),
                                d_nll.data_ptr(), st.cuda_stream)
    ms = event_time(torch, st, run, steps, warmup)
    nats = d_nll.double().reshape(B, T).sum(1).cpu().numpy()
    nt = min(steps, 5)
    tm = timing_pass(m, run, nt)
    g = tm["gemm"]
    ex = {"gemm": 1.0, "attn_chunk": 1.0} if f16 else MFMA_EXEC
    out = {"B": B, "T": T, "operands": "fp16 single-term" if f16 else "bf16 hi+lo split",
           "ms_per_step": ms, "tok_s": B * T / (ms * 1e-3),
           "alg_gflop": prefill_flops(d, B, T) / 1e9,
           "achieved_tflops_whole": prefill_flops(d, B, T) / (ms * 1e-3) / 1e12,
           "nats_per_row": nats.tolist(), "ce_bits_mean": float(nats.sum() / (B * T) / math.log(2)),
           "kernel_ms_per_step": {k: v[1] / nt for k, v in tm.items()},
           # the GEMM launches' flops are 2 M N K each: the algorithmic count
           "roofline": roofline(g, g[2], "mfma", "gemm", profile, ex["gemm"])}
    at = tm["attn_chunk"]
    if at[0]:
        out["roofline_attention"] = roofline(at, at[2], "mfma", "attn_chunk", profile,
                                             ex["attn_chunk"])
    out["whole_frac"] = out["achieved_tflops_whole"] / MFMA_BF16_PEAK_TFS
    return out


def forward_pair(m, d, torch, B, T, ids, steps, warmup, name, operands):
    """The fp16 single-term record with the split one under "split"
    (operands "both"), or one of them alone ("f16", "split": profiling runs)."""
    run = lambda f16, prof: bench_forward(m, d, torch, B, T, ids, steps, warmup, prof, f16=f16)
    if operands == "split":
        return run(False, f"profiles/{name}_split_kernels.md")
    out = run(True, f"profiles/{name}_kernels.md")
    if operands == "both":
        out["split"] = run(False, f"profiles/{name}_split_kernels.md")
    return out


def bench_prefill(m, d, steps, warmup, torch, operands="both"):
    """Depth-12 prefill, B=1, T=2048 uniform ids: logits + per-token CE."""
    from autoresearch_amd.weights import uniform_ids
    T = 2048
    return forward_pair(m, d, torch, 1, T, uniform_ids(2, T + 1, d.vocab), steps, warmup,
                        "prefill_d12_T2048", operands)


def bench_eval_b8(m, d, steps, warmup, torch, operands="both"):
    """bpb-style evaluation: B=8 independent rows of T=2048 Zipf(1.1) ids
    with the BOS id at position 0, summed NLL in nats per row."""
    from autoresearch_amd.weights import BOS_ID, zipf_ids
    B, T = 8, 2048
    rows = zipf_ids(31, B * (T + 1), d.vocab).reshape(B, T + 1)
    rows[:, 0] = BOS_ID
    return forward_pair(m, d, torch, B, T, rows, steps, warmup, "eval_d12_B8_T2048", operands)


def bench_decode(m, d, B, prompt_len, n_steps, reps, warmup, profile, prompts=None,
                 kv_bf16=False):
    """Greedy decode of B sequences: chunked prefill of prompt[:-1], then
    n_steps cached steps from the last prompt id, on the device loop
    (fg_decode_greedy), on an fp32 or a bf16 KV cache. tok/s from the wall
    clock over reps loops; the kernel roofline from an fg_timing pass over
    one loop."""
    from autoresearch_amd.weights import uniform_ids
    maxT = prompt_len + n_steps
    if prompts is None:
        prompts = uniform_ids(42 + B, B * prompt_len, d.vocab).reshape(B, prompt_len)
    kv = m.kv(B, maxT, bf16=kv_bf16)
    t0 = time.perf_counter()
    kv.step_multi(prompts[:, :-1], want_logits=False)
    m.sync()
    prefill_s = time.perf_counter() - t0
    L0 = prompt_len - 1

    def once():
        kv.len = L0
        return kv.decode_greedy(prompts[:, -1], n_steps)[0]

    for _ in range(warmup):
        once()
    t0 = time.perf_counter()
    for _ in range(reps):
        ids = once()
    dt = (time.perf_counter() - t0) / reps
    step_bytes = [decode_step_bytes(d, B, L0 + i) for i in range(n_steps)]
    mean_bytes = float(np.mean(step_bytes))
    out = {"B": B, "prompt": prompt_len, "steps": n_steps, "ms_per_step": dt / n_steps * 1e3,
           "tok_s": B * n_steps / dt, "prompt_prefill_s": prefill_s,
           "kv_cache": "bf16" if kv_bf16 else "fp32",
           "first_ids": ids[:8, 0].tolist(), "alg_bytes_per_step_mean": mean_bytes,
           "whole_step_achieved_gbs": mean_bytes / (dt / n_steps) / 1e9,
           "whole_step_frac": mean_bytes / (dt / n_steps) / 1e9 / HBM_PEAK_GBS,
           "fused_decode": m.fused_decode()[0] and B == 1}
    tm = timing_pass(m, once)
    out["kernel_ms_per_step"] = {k: v[1] / n_steps for k, v in tm.items()}
    kvl = kv_pos_bytes(d) // d.n_layer  # one layer's K and V of one position
    if tm["decode_fused"][0]:
        # one launch runs the whole loop: its algorithmic bytes are the steps'
        out["roofline"] = roofline(tm["decode_fused"], float(sum(step_bytes)), "hbm",
                                   "decode_fused", profile)
    else:
        # attention: per launch (one layer) n+1 cached positions read per
        # sequence; linears: weights once + activations, 2 N K + 4 M (K + N)
        att = float(sum(B * kvl * (L0 + i + 1) for i in range(n_steps)) * d.n_layer)
        lin = "gemm" if tm["gemm"][0] else "gemv"
        if B > 1:  # the KV reads bound the batched step; the linears beside them
            out["roofline"] = roofline(tm["attn_decode"], att, "hbm", "attn_decode", profile)
            out["roofline_linears"] = roofline(tm[lin], float(tm[lin][3]), "hbm", lin, profile)
        else:  # one sequence: the weight stream bounds the step
            out["roofline"] = roofline(tm[lin], float(tm[lin][3]), "hbm", lin, profile)
            out["roofline_attention"] = roofline(tm["attn_decode"], att, "hbm", "attn_decode",
                                                 profile)
    kv.close()
    return out


def bench_gqa20(steps, warmup, torch):
    """Depth-20 GQA model (10 query heads over 2 KV heads, d_model 1280):
    B=1 prefill of 2048 uniform ids (the cache fill of prompt[:-1] in one
    chunk, then the last id's step) followed by 256 greedy steps."""
    from autoresearch_amd import engine
    from autoresearch_amd.weights import GQA20, rope_tables, seeded_weights, uniform_ids
    d = GQA20
    P, n = 2048, 256
    log("bench: generating seeded depth-20 GQA weights")
    m = engine.Model(d, stacks=seeded_weights(d, SEED_GQA))
    c, s = rope_tables(P + n, d.head_dim)
    m.set_rope(c.reshape(-1), s.reshape(-1))
    prompt = uniform_ids(20, P, d.vocab)
    kv = m.kv(1, P + n)

    def prefill():
        kv.len = 0
        kv.step_multi(prompt[None, :-1], want_logits=False)

    for _ in range(warmup):
        prefill()
    m.sync()
    reps = max(3, min(steps, 10))
    t0 = time.perf_counter()
    for _ in range(reps):
        prefill()
    m.sync()
    pre_s = (time.perf_counter() - t0) / reps
    tm = timing_pass(m, prefill)
    pre = {"T": P - 1, "ms": pre_s * 1e3, "tok_s": (P - 1) / pre_s,
           "alg_gflop": prefill_flops(d, 1, P - 1) / 1e9,
           "whole_frac": prefill_flops(d, 1, P - 1) / pre_s / 1e12 / MFMA_BF16_PEAK_TFS,
           "kernel_ms": {k: v[1] for k, v in tm.items()},
           "roofline": roofline(tm["gemm"], tm["gemm"][2], "mfma", "gemm",
                                "profiles/gqa20_prefill2048_decode256_kernels.md")}
    if tm["attn_chunk"][0]:
        pre["roofline_attention"] = roofline(tm["attn_chunk"], tm["attn_chunk"][2], "mfma",
                                             "attn_chunk",
                                             "profiles/gqa20_prefill2048_decode256_kernels.md")
    dec = bench_decode(m, d, 1, P, n, reps=3, warmup=1,
                       profile="profiles/gqa20_prefill2048_decode256_kernels.md",
                       prompts=prompt[None, :])
    kv.close()
    m.close()
    return {"model": "gqa20 (L=20, D=1280, H=10, KH=2, hd=128, V=8192)", "prefill": pre,
            "decode": dec}


def bench_spec(m, d, reps, warmup, k=8, match=2, probe=8, min_acc=0.5):
    """Greedy speculative decoding (fg_decode_spec, prompt-lookup drafts) next
    to plain greedy decoding on the same prompt and weights: 256 ids after an
    88-id prompt that repeats a 24-id span (the context prompt lookup feeds
    on). Both streams must be equal; tok/s of each, and the loop's counters."""
    from autoresearch_amd.weights import uniform_ids
    base = uniform_ids(77, 24, d.vocab)
    prompt = np.concatenate([np.tile(base, 3), base[:16]]).astype(np.int32)
    n_gen = 256
    kv = m.kv(1, prompt.size + n_gen)
    kv.step_multi(prompt[:-1], want_logits=False)
    L0 = prompt.size - 1

    def timed(fn):
        for _ in range(warmup):
            kv.len = L0
            fn()
        t0 = time.perf_counter()
        for _ in range(reps):
            kv.len = L0
            out = fn()
        return out, (time.perf_counter() - t0) / reps

    # plain greedy as per-kernel steps (the arithmetic the verification pass
    # repeats row by row, so the streams must be equal), and the persistent
    # loop beside it
    m.set_fused_decode(False)
    try:
        g, t_g = timed(lambda: kv.decode_greedy(prompt[-1:], n_gen)[0][:, 0])
    finally:
        m.set_fused_decode(True)
    gf, t_f = timed(lambda: kv.decode_greedy(prompt[-1:], n_gen)[0][:, 0])
    (sp, st), t_s = timed(lambda: kv.decode_spec(prompt, n_gen, k=k, match=match, probe=probe,
                                                 min_acc=min_acc))
    kv.close()
    if not np.array_equal(g, sp):
        raise RuntimeError("speculative stream differs from the greedy stream")
    return {"prompt": int(prompt.size), "gen": n_gen, "k": k, "match": match,
            "greedy_tok_s": n_gen / t_g, "spec_tok_s": n_gen / t_s, "speedup": t_g / t_s,
            "persistent_greedy_tok_s": n_gen / t_f,
            "persistent_stream_equal": bool(np.array_equal(gf, g)),
            "stats": st, "streams_equal": True}


def bench_sample(m, d, reps, warmup, n_gen=256):
    """chat_text's plain loop with sample_next on the device (fg_decode_sample:
    temp 0.8, top-p 0.9, presence 0.2, frequency 0.1, repetition 1.1, no-repeat
    3-grams) after a 16-id prompt, beside plain greedy decoding; tok/s of
    each and the sampling kernel's share from an eager timing pass."""
    from autoresearch_amd.weights import uniform_ids
    cfg = dict(temp=0.8, topp=0.9, pres=0.2, freq=0.1, rep=1.1, nblock=3)
    prompt = uniform_ids(91, 16, d.vocab)
    kv = m.kv(1, prompt.size + n_gen)
    kv.step_multi(prompt[:-1], want_logits=False)
    L0 = prompt.size - 1

    def timed(fn):
        for _ in range(warmup):
            kv.len = L0
            fn()
        t0 = time.perf_counter()
        for _ in range(reps):
            kv.len = L0
            out = fn()
        return out, (time.perf_counter() - t0) / reps

    m.set_fused_decode(False)  # the per-kernel steps sampling is built on
    try:
        _, t_g = timed(lambda: kv.decode_greedy(prompt[-1:], n_gen))
    finally:
        m.set_fused_decode(True)
    (ids, _), t_s = timed(lambda: kv.decode_sample(prompt, n_gen, seed=12345, **cfg))
    m.timing(True)
    kv.len = L0
    kv.decode_sample(prompt, n_gen, seed=12345, **cfg)
    tm = m.timing_read()
    m.timing(False)
    kv.close()
    return {"prompt": int(prompt.size), "gen": n_gen, "cfg": cfg, "greedy_tok_s": n_gen / t_g,
            "sample_tok_s": n_gen / t_s, "first_ids": ids[:8].tolist(),
            "kernel_ms_per_step": {k: v[1] / n_gen for k, v in tm.items()}}


# --- PMC counters: HBM-side traffic of each record's dominant kernel, and
# the prefill kernels' MFMA use. Each reading comes from a child process run
# under `rocprofv3 --pmc` before this process touches the GPU.
CALIB_BYTES = 256 << 20           # plain copy of known size: reads and writes this much
# (probe mode, kernel-name fragments of the kind)
PMC_KINDS = {
    "prefill": ("prefill", ("k_gemm",)),
    "prefill_attn": ("prefill", ("k_attn_mfma",)),
    "decode_b1": ("decode_b1", ("k_fused_decode",)),
    "decode_b64": ("decode_b64", ("k_attn_dec",)),
}
PMC_B64_STEPS = 16                # batched-decode steps the probe runs
# the probe's prompt length: its 16 steps attend over 1272..1287 positions,
# 1279.5 on average, the mean of the timed 512 steps after 1023-id prompts
PMC_B64_PROMPT = 1272


def pmc_probe(workload: str = "prefill", f16: bool = True):
    """Child of a `rocprofv3 --pmc` run. prefill: one warm-up and one
    measured T=2048 forward (single-term fp16 operands, or split-bf16 ones
    with f16=False); decode_b1: two loops of the B=1 decode workload (16-id
    prompt, 32 steps); decode_b64: 64 sequences prefilled to
    PMC_B64_PROMPT - 1 positions, then PMC_B64_STEPS steps on the bf16 cache
    (the timed workload's mean context). Then a 256 MiB
    device copy whose reading calibrates the counter against known bytes.
    Every handle is closed and the device idle before the process exits."""
    import torch
    from autoresearch_amd import engine
    from autoresearch_amd.weights import D12, seeded_weights, rope_tables, uniform_ids
    d = D12
    m = engine.Model(d, stacks=seeded_weights(d, SEED))
    try:
        c, s = rope_tables(2048, d.head_dim)
        m.set_rope(c.reshape(-1), s.reshape(-1))
        dev = torch.device("cuda:0")
        if workload == "decode_b1":
            prompts = uniform_ids(43, 16, d.vocab).reshape(1, 16)
            kv = m.kv(1, 48)
            kv.step_multi(prompts[:, :-1], want_logits=False)
            for _ in range(2):
                kv.len = 15
                kv.decode_greedy(prompts[:, -1], 32)
            kv.close()
        elif workload == "decode_b64":
            B, P = 64, PMC_B64_PROMPT
            prompts = uniform_ids(42 + B, B * P, d.vocab).reshape(B, P)
            kv = m.kv(B, P + PMC_B64_STEPS, bf16=True)
            kv.step_multi(prompts[:, :-1], want_logits=False)
            kv.decode_greedy(prompts[:, -1], PMC_B64_STEPS)
            kv.close()
        else:
            T = 2048
            ids = uniform_ids(2, T + 1, d.vocab)
            d_ids = torch.from_numpy(ids[:T].copy()).to(dev)
            d_lg = torch.empty(T * d.vocab, dtype=torch.float32, device=dev)
            m.set_forward_f16(f16)  # on: the configuration the prefill line is quoted on
            for _ in range(2):
                m.forward_dev(d_ids.data_ptr(), 1, T, d_lg.data_ptr(), 0, 0, 0)
                m.sync()
        m.sync()
        a = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        b.copy_(a)
        torch.cuda.synchronize()
    finally:
        m.close()
        torch.cuda.synchronize()
    print("pmc probe done", flush=True)


def pmc_rows(mode: str, counters):
    """Per-dispatch rows (kernel, counter, value) of one `rocprofv3 --pmc`
    run of the probe, or None when the profiler is absent or gave nothing."""
    exe = shutil.which("rocprofv3")
    if exe is None:
        return None
    with tempfile.TemporaryDirectory(dir="/tmp") as td:
        cmd = ["timeout", "-s", "KILL", "240", exe, "--pmc", *counters, "--output-format",
               "csv", "-d", td, "-o", "run", "--", sys.executable, os.path.abspath(__file__),
               "--pmc-probe", mode]
        env = dict(os.environ, TMPDIR="/tmp")
        r = subprocess.run(cmd, cwd=ROOT, env=env, stdout=subprocess.PIPE,
                           stderr=subprocess.STDOUT, text=True)
        files = glob.glob(os.path.join(td, "**", "*counter_collection.csv"), recursive=True)
        if not files or "pmc probe done" not in r.stdout:
            log(f"bench: rocprofv3 --pmc {' '.join(counters)} ({mode}) gave no result "
                f"(rc {r.returncode})")
            return None
        return sorted(csv.DictReader(open(files[0])), key=lambda x: int(x["Dispatch_Id"]))


def kind_values(rows, counter, frags):
    """The counter's per-dispatch values, in dispatch order, of the kernels
    whose names hold one of frags."""
    return [float(x["Counter_Value"]) for x in rows
            if x["Counter_Name"] == counter and any(f in x["Kernel_Name"] for f in frags)]


def pmc_kind(key: str, counters, reduce_last):
    """Mean reading per launch of the kind (over the launches reduce_last
    picks from the kind's dispatches) for each counter, and the calibration
    copy's reading."""
    mode, frags = PMC_KINDS[key]
    rows = pmc_rows(mode, counters)
    if rows is None:
        return None
    out = {}
    for counter in counters:
        vals = kind_values(rows, counter, frags)
        sel = reduce_last(vals)
        if not sel:
            return None
        out[counter] = sum(sel) / len(sel)
        out["launches"] = len(sel)
        copy = [float(x["Counter_Value"]) for x in rows
                if x["Counter_Name"] == counter and "copy" in x["Kernel_Name"].lower()]
        if copy:
            out[counter + "_copy"] = copy[-1]
    return out


def _last_half(vals):
    return vals[len(vals) // 2:]


def pmc_traffic(key: str):
    """HBM-side bytes per launch of the kind: FETCH_SIZE and WRITE_SIZE (two
    runs, KiB per dispatch), each scaled by bytes / reading of the 256 MiB
    calibration copy. Prefill and B=1 decode ran their pass twice: the
    second pass's launches; the batched decode: every launch of its steps."""
    pick = (lambda v: v) if key == "decode_b64" else _last_half
    out = {}
    for counter, name in (("FETCH_SIZE", "read"), ("WRITE_SIZE", "write")):
        got = pmc_kind(key, [counter], pick)
        if got is None or counter + "_copy" not in got:
            return None
        factor = CALIB_BYTES / (got[counter + "_copy"] * 1024.0)
        out[name + "_bytes"] = got[counter] * 1024.0 * factor
        out[name + "_calibration"] = factor
        out["launches"] = got["launches"]
    out["bytes"] = out["read_bytes"] + out["write_bytes"]
    return out


# MfmaUtil is the profiler's derived metric: the MFMA busy cycles summed over
# the SIMDs / (the busiest XCC's GRBM_GUI_ACTIVE x the SIMD count), in %
MFMA_COUNTERS = ["MfmaUtil", "SQ_INSTS_VALU_MFMA_MOPS_F16"]


def pmc_mfma(key: str):
    """MFMA use of the kind over the second forward: the profiler's MfmaUtil
    per dispatch (as a fraction), and the executed fp16 MFMA flops per launch
    (SQ_INSTS_VALU_MFMA_MOPS_F16 x 512)."""
    got = pmc_kind(key, MFMA_COUNTERS, _last_half)
    if got is None:
        return None
    return {"launches": got["launches"], "mfma_util": got["MfmaUtil"] / 100.0,
            "mfma_f16_flop_per_launch": got["SQ_INSTS_VALU_MFMA_MOPS_F16"] * 512.0}


CPU_LOOP = ("naive loop order of the reference's non-BLAS path (fortran_linear / causal_attn: "
            "each output a sequential fp32 sum, OpenMP over outputs), not OpenBLAS sgemm_; "
            "weights transposed once before the timed region")


def cpu_facts() -> dict:
    """The host the CPU baseline runs on: model name, logical CPUs, the CPUs
    this process may use, and physical cores (lscpu's sockets x cores)."""
    out = {"logical_cpus": os.cpu_count(), "usable_cpus": len(os.sched_getaffinity(0))}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    out["model"] = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        r = subprocess.run(["lscpu"], stdout=subprocess.PIPE, stderr=subprocess.DEVNULL,
                           text=True, timeout=10)
        kv = dict(l.split(":", 1) for l in r.stdout.splitlines() if ":" in l)
        cps, sock = int(kv["Core(s) per socket"].strip()), int(kv["Socket(s)"].strip())
        out["physical_cores"] = cps * sock
    except Exception:
        pass
    return out


def cpu_baseline(d, w, budget_s: float = 12.0) -> dict:
    """The CPU oracle (a restatement of the reference loops) on this host's
    cores: T=2048 prefill forwards until the budget is spent. The transposed
    weight copies its linear loop uses are made once, by an untimed short
    forward, and kept (or_wt_cache)."""
    from oracle import oracle as O
    from autoresearch_amd.weights import uniform_ids, rope_tables
    T = 2048
    ids = uniform_ids(2, T, d.vocab)
    c, s = rope_tables(T, d.head_dim)
    O.lib().or_wt_cache(1)
    try:
        O.gpt_forward(ids[:8], c.reshape(-1), s.reshape(-1), w, d, 1, 8)
        n, t0 = 0, time.perf_counter()
        while True:
            O.gpt_forward(ids, c.reshape(-1), s.reshape(-1), w, d, 1, T)
            n += 1
            el = time.perf_counter() - t0
            if el >= budget_s or n >= 3:
                break
    finally:
        O.lib().or_wt_cache(0)
    return {"value": n * T / el, "unit": "tok/s", "cores": int(O.lib().or_num_threads()),
            "kind": "port",
            "sample": f"{n} x depth-12 prefill forward at B=1, T=2048 (same seeded weights and "
                      f"ids), {el:.1f} s wall; {CPU_LOOP}"}


def cpu_decode_baseline(d, w, c, s, budget_s: float = 6.0) -> dict:
    """The oracle's greedy loop of the B=1 decode workload: 15 prompt
    gpt_step calls, then 32 greedy gpt_step calls (only those timed)."""
    from oracle import oracle as O
    from autoresearch_amd.weights import uniform_ids
    prompt = uniform_ids(43, 16, d.vocab)
    O.lib().or_wt_cache(1)
    try:
        O.greedy_decode(prompt[:2], w, d, 1, c, s, maxT=48)  # makes the transposed copies
        kv = O.KVCache(d, 48)
        hd2 = d.head_dim // 2
        for t in range(15):
            O.gpt_step(prompt[t:t + 1], c[t * hd2:], s[t * hd2:], w, d, kv)
        reps, t0 = 0, time.perf_counter()
        while True:  # the 32 steps again from the same cache state until the budget is spent
            kv.len[0] = 15
            nxt, ids = int(prompt[15]), []
            for t in range(15, 47):
                lg = O.gpt_step(np.array([nxt], np.int32), c[t * hd2:], s[t * hd2:], w, d, kv)
                nxt = O.argmax(lg)
                ids.append(nxt)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s:
                break
    finally:
        O.lib().or_wt_cache(0)
    return {"value": 32 * reps / el, "unit": "tok/s", "cores": int(O.lib().or_num_threads()),
            "kind": "port", "sample": f"{reps} x 32 greedy gpt_step calls after a 15-step "
                                      f"prompt, B=1, depth-12, {el:.1f} s wall; {CPU_LOOP}",
            "first_ids": ids[:8]}


def cpu_child():
    """--cpu-child: the CPU baselines in a process of their own, so the
    oracle's OpenMP runtime starts with the settings the reference measured
    best (OMP_PROC_BIND=close, OMP_DYNAMIC=FALSE: set by the parent) and no
    GPU runtime beside it. Prints one JSON line."""
    from autoresearch_amd.weights import D12, seeded_weights, rope_tables
    d = D12
    w = seeded_weights(d, SEED)
    c, s = rope_tables(2304, d.head_dim)
    out = cpu_baseline(d, w)
    out["decode_b1"] = cpu_decode_baseline(d, w, c.reshape(-1), s.reshape(-1))
    print("CPU " + json.dumps(out), flush=True)


def run_cpu_baseline() -> dict:
    facts = cpu_facts()
    env = dict(os.environ, OMP_PROC_BIND="close", OMP_DYNAMIC="FALSE")
    if "OMP_NUM_THREADS" not in env:
        env["OMP_NUM_THREADS"] = str(facts.get("usable_cpus", os.cpu_count()))
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-child"], cwd=ROOT,
                       env=env, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                       timeout=600)
    line = [l for l in r.stdout.splitlines() if l.startswith("CPU ")]
    if r.returncode != 0 or not line:
        log("bench: CPU baseline child failed", r.stderr[-2000:])
        return None
    out = json.loads(line[-1][4:])
    out["host"] = {**facts, "OMP_NUM_THREADS": env["OMP_NUM_THREADS"],
                   "OMP_PROC_BIND": "close", "OMP_DYNAMIC": "FALSE"}
    return out


WORKLOADS = ("prefill", "decode_b1", "decode_b1_ctx1k", "eval_b8", "decode_b64",
             "decode_b64_fp32kv", "gqa20", "decode_spec", "decode_sample")

# what the final line keeps of a roofline record (the full records go to stderr)
ROOF_KEYS = ("bound", "kernel_kind", "avg_launch_us", "achieved", "peak", "unit", "frac",
             "traffic", "mfma_executed_frac", "mfma_util")
# (the workload records leave out peak and unit: the line's "peaks" holds
# them, per bound)
ROOF_KEYS_NESTED = tuple(k for k in ROOF_KEYS if k not in ("peak", "unit"))


def sig(v, n=5):
    """v to n significant digits (the line's figures; full ones on stderr)."""
    return float(f"{v:.{n}g}") if isinstance(v, float) and math.isfinite(v) else v


def brief_roof(r, keys=ROOF_KEYS_NESTED):
    if not r:
        return r
    return {k: sig(v) for k, v in r.items() if k in keys}


def brief(rec):
    """The figures of a workload record that the one-line summary keeps:
    throughput, step time, the rooflines (without per-launch detail), whole
    fractions; nested records likewise; per-row arrays and per-kernel
    breakdowns stay in the full record on stderr."""
    if not isinstance(rec, dict):
        return rec
    out = {}
    for k, v in rec.items():
        if k.startswith("roofline"):
            out[k] = brief_roof(v)
        elif isinstance(v, dict) and k in ("split", "prefill", "decode"):
            out[k] = brief(v)
        elif isinstance(v, (int, float, str, bool)) and k not in ("first_ids",):
            out[k] = sig(v)
    return out


def profiles_of(rec, prefix="", out=None):
    """record path -> the profiles/ summary each of its rooflines reproduces from."""
    out = {} if out is None else out
    for k, v in (rec or {}).items():
        if k.startswith("roofline") and isinstance(v, dict) and v.get("profile"):
            out.setdefault(v["profile"], []).append(prefix + k)
            if v.get("traffic_profile"):
                out.setdefault(v["traffic_profile"], []).append(prefix + k + ".traffic")
        elif isinstance(v, dict) and k in ("split", "prefill", "decode"):
            profiles_of(v, prefix + k + ".", out)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--skip", action="append", default=[], choices=WORKLOADS,
                    help="leave a workload out of the full run")
    ap.add_argument("--operands", choices=("both", "f16", "split"), default="both",
                    help="prefill / eval_b8: the fp16 single-term pass, the split one, or both")
    ap.add_argument("--only", choices=WORKLOADS,
                    help="run one workload and print its record (for profiling runs)")
    ap.add_argument("--no-pmc", action="store_true", help="skip the PMC counter runs")
    ap.add_argument("--detail", metavar="FILE", help="also write the full records to FILE")
    ap.add_argument("--pmc-probe", nargs="?", const="prefill",
                    choices=("prefill", "decode_b1", "decode_b64"), help=argparse.SUPPRESS)
    ap.add_argument("--cpu-child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.pmc_probe:
        pmc_probe(args.pmc_probe, f16=args.operands != "split")
        return
    if args.cpu_child:
        cpu_child()
        return
    if args.gpus != 1:
        print(f"bench.py: this engine runs on one GPU; --gpus {args.gpus} is not supported "
              "(data-parallel sharding is not built)", file=sys.stderr)
        sys.exit(2)

    # the counter runs go first, before this process touches the GPU
    pmc = {}
    if not args.only and not args.no_pmc:
        log("bench: PMC runs (FETCH_SIZE, WRITE_SIZE; MFMA busy cycles)")
        for key in ("prefill", "decode_b1", "decode_b64"):
            pmc[key] = pmc_traffic(key)
            log(f"bench: traffic {key}", json.dumps(pmc[key]))
        for key in ("prefill", "prefill_attn"):
            pmc["mfma_" + key] = pmc_mfma(key)
            log(f"bench: mfma {key}", json.dumps(pmc["mfma_" + key]))

    import torch
    from autoresearch_amd import engine
    from autoresearch_amd.weights import D12, seeded_weights, rope_tables

    d = D12
    log("bench: generating seeded depth-12 weights")
    w = seeded_weights(d, SEED)
    m = engine.Model(d, stacks=w)
    try:
        c, s = rope_tables(2304, d.head_dim)
        m.set_rope(c.reshape(-1), s.reshape(-1))
        runs = {
            "prefill": lambda: bench_prefill(m, d, args.steps, args.warmup, torch, args.operands),
            "decode_b1": lambda: bench_decode(m, d, 1, 16, 32, reps=max(args.steps, 5),
                                              warmup=args.warmup,
                                              profile="profiles/decode_d12_B1_fused.md"),
            # the B=1 loop at chat_text's context: a 1032-id prompt, 64 steps
            "decode_b1_ctx1k": lambda: bench_decode(
                m, d, 1, 1032, 64, reps=max(args.steps // 4, 3), warmup=1,
                profile="profiles/decode_d12_B1_ctx1k_fused.md"),
            "eval_b8": lambda: bench_eval_b8(m, d, max(3, args.steps // 4), 1, torch,
                                             args.operands),
            "decode_b64": lambda: bench_decode(m, d, 64, 1024, 512, reps=1, warmup=0,
                                               profile="profiles/decode_d12_B64_kernels.md",
                                               kv_bf16=True),
            "decode_b64_fp32kv": lambda: bench_decode(
                m, d, 64, 1024, 512, reps=1, warmup=0,
                profile="profiles/decode_d12_B64_fp32kv_kernels.md"),
            "gqa20": lambda: bench_gqa20(args.steps, 1, torch),
            "decode_spec": lambda: bench_spec(m, d, reps=3, warmup=1),
            "decode_sample": lambda: bench_sample(m, d, reps=3, warmup=1),
        }
        if args.only:
            print(json.dumps({"only": args.only, **runs[args.only]()}), flush=True)
            return
        rec = {}
        for name in WORKLOADS:
            if name in args.skip:
                rec[name] = None
                continue
            log(f"bench: {name}")
            rec[name] = runs[name]()
            log(f"bench: {name}", json.dumps(rec[name]))
    finally:
        m.close()
        torch.cuda.synchronize()

    cpu = None
    if not args.no_cpu:
        log("bench: CPU oracle baseline (child process)")
        cpu = run_cpu_baseline()
        log("bench: cpu", json.dumps(cpu))

    # counter readings into the records they belong to
    pre = rec["prefill"]
    attach = (("prefill", "roofline", "prefill", "gemm"),
              ("decode_b1", "roofline", "decode_b1", "decode_fused"),
              ("decode_b64", "roofline", "decode_b64", "attn_decode"))
    traffic_profiles = {"prefill": "profiles/prefill_d12_T2048_traffic.md",
                        "decode_b1": "profiles/decode_d12_B1_traffic.md",
                        "decode_b64": "profiles/decode_d12_B64_traffic.md"}
    for key, field, name, kind in attach:
        t = pmc.get(key)
        r = rec.get(name)
        if t and r and r.get(field, {}).get("kernel_kind") == kind:
            if key == "decode_b64":
                # the probed launches' own algorithmic bytes (PMC_B64_STEPS
                # steps after PMC_B64_PROMPT - 1 prefilled positions)
                kvl = kv_pos_bytes(d) // d.n_layer
                t["alg_bytes_per_launch"] = 64 * kvl * float(
                    np.mean([PMC_B64_PROMPT - 1 + i + 1 for i in range(PMC_B64_STEPS)]))
            r[field]["traffic"] = t["bytes"]
            r[field]["traffic_detail"] = t
            r[field]["traffic_profile"] = traffic_profiles[key]
    for key, field in (("mfma_prefill", "roofline"), ("mfma_prefill_attn", "roofline_attention")):
        mf = pmc.get(key)
        if mf and pre and pre.get(field):
            pre[field]["mfma_util"] = mf["mfma_util"]
            pre[field]["mfma_counters"] = mf
    if args.detail:
        with open(args.detail, "w") as f:
            json.dump({"records": rec, "pmc": pmc, "cpu_baseline": cpu}, f, indent=1)

    def roof_line(r, keys=ROOF_KEYS_NESTED):
        out = brief_roof(r, keys)
        if r and r.get("traffic_detail"):
            out["traffic"] = round(r["traffic_detail"]["bytes"])
        if r and r.get("mfma_counters"):
            out["mfma_util"] = sig(r["mfma_counters"]["mfma_util"])
        return out

    line = {
        "metric": METRIC, "value": pre["tok_s"], "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": pre["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded N(0,0.02) bf16-exact weights, uniform / Zipf ids)",
        "config": {"workload": "depth-12 prefill, B=1, T=2048: fp32 logits [2048,8192] + "
                               "per-token CE", "global_batch": 1, "seq_len": 2048,
                   "parallelism": "single GPU"},
        "roofline": roof_line(pre["roofline"], ROOF_KEYS),
        "peaks": {"hbm": [HBM_PEAK_GBS, "GB/s"], "mfma": [MFMA_BF16_PEAK_TFS, "TFLOP/s"]},
        "cpu_baseline": None if cpu is None else {
            k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample")},
    }
    if cpu is not None:
        line["cpu_baseline"]["host"] = cpu["host"]
        line["cpu_baseline"]["decode_b1"] = {k: cpu["decode_b1"][k] for k in ("value", "unit")}
    profs = {}
    for name in WORKLOADS:
        line[name] = brief(rec[name]) if rec[name] is not None else None
        if rec[name] is not None:
            for k, v in rec[name].items():
                if k.startswith("roofline") and isinstance(v, dict):
                    line[name][k] = roof_line(v)
            for path, keys in profiles_of(rec[name], name + ".").items():
                profs.setdefault(path, []).extend(keys)
    line["profiles"] = profs
    print(json.dumps(line, separators=(",", ":")), flush=True)


if __name__ == "__main__":
    main()
