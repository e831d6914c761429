#!/usr/bin/env python3
"""Benchmark of the MI355X engine for the fortran_gpt forward path.

One JSON line on stdout. `value` is the prefill throughput of the depth-12
model at B=1, T=2048 (logits [2048, 8192] plus per-token cross-entropy, ids
and targets already resident in HBM), one "step" being one full forward.
Beside it: the B=1 greedy decode (16-id prompt, 32 cached steps) and the
B=64 batched decode, each with its own roofline, and the CPU oracle timed on
this host's cores on a bounded sample.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-b64]
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
MFMA_BF16_PEAK_TFS = 2516.6    # 256 CU x 2.4 GHz x 4096 bf16 flop/clk, dense
SEED = 1234


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def roofline_from(timing: dict, kind: str, bound: str) -> dict:
    n, ms, fl, by = timing[kind]
    per_ms = ms / max(n, 1)
    if bound == "mfma":
        achieved = (fl / max(n, 1)) / (per_ms * 1e-3) / 1e12
        peak, unit = MFMA_BF16_PEAK_TFS, "TFLOP/s"
    else:
        achieved = (by / max(n, 1)) / (per_ms * 1e-3) / 1e9
        peak, unit = HBM_PEAK_GBS, "GB/s"
    return {"bound": bound, "kernel_kind": kind, "launches": n, "avg_launch_us": per_ms * 1e3,
            "achieved": achieved, "peak": peak, "unit": unit, "frac": achieved / peak,
            "traffic": None}


def dominant(timing: dict) -> str:
    return max(timing, key=lambda k: timing[k][1])


def bench_prefill(m, d, steps, warmup, torch):
    from autoresearch_amd.weights import uniform_ids
    T = 2048
    ids = uniform_ids(2, T + 1, d.vocab)
    dev = torch.device("cuda:0")
    d_ids = torch.from_numpy(ids[:T].copy()).to(dev)
    d_tgt = torch.from_numpy(ids[1:].copy()).to(dev)
    d_lg = torch.empty(T * d.vocab, dtype=torch.float32, device=dev)
    d_nll = torch.empty(T, dtype=torch.float32, device=dev)
    st = torch.cuda.Stream()  # a real stream handle: events and kernels share it
    run = lambda: m.forward_dev(d_ids.data_ptr(), 1, T, d_lg.data_ptr(), d_tgt.data_ptr(),
                                d_nll.data_ptr(), st.cuda_stream)
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(st):
        e0.record(st)
        for _ in range(steps):
            run()
        e1.record(st)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    bits = float(d_nll.double().mean().item() / math.log(2))
    # kernel timing pass: every launch bracketed by HIP events on this stream
    m.timing(True)
    for _ in range(min(steps, 5)):
        run()
    torch.cuda.synchronize()
    tm = m.timing_read()
    m.timing(False)
    kind = dominant(tm)
    roof = roofline_from(tm, kind, "mfma" if kind in ("gemm", "attn_chunk") else "hbm")
    return {"T": T, "ms_per_step": ms, "tok_s": T / (ms * 1e-3), "ce_bits_mean": bits,
            "kernel_ms_per_step": {k: v[1] / min(steps, 5) for k, v in tm.items()},
            "roofline": roof, "algorithmic_gflop": tm_total_flops(tm) / min(steps, 5) / 1e9}


def tm_total_flops(tm):
    return sum(v[2] for v in tm.values())


def bench_decode(m, d, B, prompt_len, n_steps, reps, warmup, with_roofline=True):
    from autoresearch_amd.weights import uniform_ids
    maxT = prompt_len + n_steps
    prompts = uniform_ids(42 + B, B * prompt_len, d.vocab).reshape(B, prompt_len)
    kv = m.kv(B, maxT)
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
    out = {"B": B, "prompt": prompt_len, "steps": n_steps, "ms_per_step": dt / n_steps * 1e3,
           "tok_s": B * n_steps / dt, "prompt_prefill_s": prefill_s,
           "first_ids": ids[:8, 0].tolist()}
    if with_roofline:
        m.timing(True)
        once()
        tm = m.timing_read()
        m.timing(False)
        kind = dominant(tm)
        out["roofline"] = roofline_from(tm, kind, "hbm")
        out["kernel_ms_per_step"] = {k: v[1] / n_steps for k, v in tm.items()}
        # whole-step algorithmic bytes: bf16 weights (all but the embedding
        # table) + one embedding row + KV read and append per sequence
        wbytes = 2 * (d.params - d.vocab * d.d_model) + 2 * d.d_model
        kvb = 4 * 2 * d.n_layer * d.n_kv_head * d.head_dim  # fp32 K and V per position
        mean_len = L0 + (n_steps + 1) / 2
        step_bytes = wbytes + B * kvb * (mean_len + 1)
        out["step_bytes_mean"] = step_bytes
        out["step_hbm_frac"] = step_bytes / (dt / n_steps) / 1e9 / HBM_PEAK_GBS
    kv.close()
    return out


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

    g, t_g = timed(lambda: kv.decode_greedy(prompt[-1:], n_gen)[0][:, 0])
    (sp, st), t_s = timed(lambda: kv.decode_spec(prompt, n_gen, k=k, match=match, probe=probe,
                                                 min_acc=min_acc))
    kv.close()
    if not np.array_equal(g, sp):
        raise RuntimeError("speculative stream differs from the greedy stream")
    return {"prompt": int(prompt.size), "gen": n_gen, "k": k, "match": match,
            "greedy_tok_s": n_gen / t_g, "spec_tok_s": n_gen / t_s, "speedup": t_g / t_s,
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

    _, t_g = timed(lambda: kv.decode_greedy(prompt[-1:], n_gen))
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


# --- HBM traffic of the dominant prefill kernel kind, from PMC counters ---
PMC_KIND = "gemm"                 # kernel kind the prefill roofline is quoted on
PMC_MATCH = ("k_gemm",)           # kernel-name fragments of that kind
CALIB_BYTES = 256 << 20           # plain copy of known size: reads and writes this much


def pmc_probe():
    """Child of a `rocprofv3 --pmc` run: one warm-up and one measured T=2048
    prefill, then a 256 MiB device copy whose counter reading calibrates the
    counter against known bytes."""
    import torch
    from autoresearch_amd import engine
    from autoresearch_amd.weights import D12, seeded_weights, rope_tables, uniform_ids
    d = D12
    m = engine.Model(d, stacks=seeded_weights(d, SEED))
    c, s = rope_tables(2048, d.head_dim)
    m.set_rope(c.reshape(-1), s.reshape(-1))
    T = 2048
    ids = uniform_ids(2, T + 1, d.vocab)
    dev = torch.device("cuda:0")
    d_ids = torch.from_numpy(ids[:T].copy()).to(dev)
    d_lg = torch.empty(T * d.vocab, dtype=torch.float32, device=dev)
    for _ in range(2):
        m.forward_dev(d_ids.data_ptr(), 1, T, d_lg.data_ptr(), 0, 0, 0)
        m.sync()
    a = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    print("pmc probe done", flush=True)


def pmc_counter(counter: str, launches_per_forward: int):
    """Mean `counter` (KiB per dispatch) over the dominant kind's launches of
    the probe's last forward, and the reading for the calibration copy."""
    exe = shutil.which("rocprofv3")
    if exe is None:
        return None
    with tempfile.TemporaryDirectory(dir="/tmp") as td:
        cmd = ["timeout", "-s", "KILL", "180", exe, "--pmc", counter, "--output-format", "csv",
               "-d", td, "-o", "run", "--", sys.executable, os.path.abspath(__file__),
               "--pmc-probe"]
        env = dict(os.environ, TMPDIR="/tmp")
        r = subprocess.run(cmd, cwd=ROOT, env=env, stdout=subprocess.PIPE,
                           stderr=subprocess.STDOUT, text=True)
        files = glob.glob(os.path.join(td, "**", "*counter_collection.csv"), recursive=True)
        if not files or "pmc probe done" not in r.stdout:
            log(f"bench: rocprofv3 --pmc {counter} gave no result (rc {r.returncode})")
            return None
        rows = sorted(csv.DictReader(open(files[0])), key=lambda x: int(x["Dispatch_Id"]))
    rows = [x for x in rows if x["Counter_Name"] == counter]
    kern = [float(x["Counter_Value"]) for x in rows
            if any(f in x["Kernel_Name"] for f in PMC_MATCH)][-launches_per_forward:]
    copy = [float(x["Counter_Value"]) for x in rows if "copy" in x["Kernel_Name"].lower()]
    if len(kern) < launches_per_forward or not copy:
        return None
    return sum(kern) / len(kern), copy[-1]


def pmc_traffic(launches_per_forward: int):
    """HBM bytes per launch of the dominant kind: FETCH_SIZE and WRITE_SIZE
    (two runs), each scaled by bytes / reading of the calibration copy."""
    out = {}
    for counter, key in (("FETCH_SIZE", "read"), ("WRITE_SIZE", "write")):
        got = pmc_counter(counter, launches_per_forward)
        if got is None:
            return None
        kib, calib_kib = got
        factor = CALIB_BYTES / (calib_kib * 1024.0)
        out[key + "_bytes"] = kib * 1024.0 * factor
        out[key + "_calibration"] = factor
    out["bytes"] = out["read_bytes"] + out["write_bytes"]
    return out


def cpu_baseline(d, w, budget_s: float = 12.0) -> dict:
    """The CPU oracle (a restatement of the reference loops) on this host's
    cores: T=2048 prefill forwards until the budget is spent."""
    from oracle import oracle as O
    from autoresearch_amd.weights import uniform_ids, rope_tables
    T = 2048
    ids = uniform_ids(2, T, d.vocab)
    c, s = rope_tables(T, d.head_dim)
    n, t0 = 0, time.perf_counter()
    while True:
        O.gpt_forward(ids, c.reshape(-1), s.reshape(-1), w, d, 1, T)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 3:
            break
    return {"value": n * T / el, "unit": "tok/s", "cores": int(O.lib().or_num_threads()),
            "kind": "port",
            "sample": f"{n} x depth-12 prefill forward at B=1, T=2048 (same seeded weights and "
                      f"ids), {el:.1f} s wall, default causal_attn order"}


def cpu_decode_baseline(d, w, c, s) -> dict:
    from oracle import oracle as O
    from autoresearch_amd.weights import uniform_ids
    prompt = uniform_ids(43, 16, d.vocab)
    t0 = time.perf_counter()
    ids, _ = O.greedy_decode(prompt, w, d, 32, c, s, maxT=48)
    el = time.perf_counter() - t0
    return {"value": 32 / el, "unit": "tok/s", "cores": int(O.lib().or_num_threads()),
            "kind": "port", "sample": "15 prompt gpt_step + 32 greedy gpt_step, B=1, depth-12",
            "first_ids": ids[:8].tolist()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-b64", action="store_true")
    ap.add_argument("--only", choices=("prefill", "decode_b1", "decode_b64", "decode_spec",
                                       "decode_sample"),
                    help="run one workload and print its record (for profiling runs)")
    ap.add_argument("--no-pmc", action="store_true", help="skip the PMC traffic runs")
    ap.add_argument("--pmc-probe", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.pmc_probe:
        pmc_probe()
        return
    if args.gpus != 1:
        print(f"bench.py: this engine runs on one GPU; --gpus {args.gpus} is not supported "
              "(data-parallel sharding is not built)", file=sys.stderr)
        sys.exit(2)

    # the counter runs go first, before this process touches the GPU
    traffic = None
    if not args.only and not args.no_pmc:
        log("bench: PMC traffic runs (FETCH_SIZE, WRITE_SIZE)")
        from autoresearch_amd.weights import D12 as _d
        traffic = pmc_traffic(4 * _d.n_layer + 1)
        log("bench: traffic", json.dumps(traffic))

    import torch
    from autoresearch_amd import engine
    from autoresearch_amd.weights import D12, seeded_weights, rope_tables

    d = D12
    log("bench: generating seeded depth-12 weights")
    w = seeded_weights(d, SEED)
    m = engine.Model(d, stacks=w)
    c, s = rope_tables(2304, d.head_dim)
    m.set_rope(c.reshape(-1), s.reshape(-1))

    if args.only:
        rec = {"prefill": lambda: bench_prefill(m, d, args.steps, args.warmup, torch),
               "decode_b1": lambda: bench_decode(m, d, 1, 16, 32, reps=max(args.steps, 5),
                                                 warmup=args.warmup),
               "decode_b64": lambda: bench_decode(m, d, 64, 1024, 512, reps=1, warmup=0),
               "decode_spec": lambda: bench_spec(m, d, reps=3, warmup=1),
               "decode_sample": lambda: bench_sample(m, d, reps=3, warmup=1)}[args.only]()
        print(json.dumps({"only": args.only, **rec}), flush=True)
        return

    log("bench: prefill B=1 T=2048")
    pre = bench_prefill(m, d, args.steps, args.warmup, torch)
    log("bench: prefill", json.dumps(pre))
    log("bench: decode B=1")
    dec1 = bench_decode(m, d, 1, 16, 32, reps=max(args.steps, 5), warmup=args.warmup)
    log("bench: decode B=1", json.dumps(dec1))
    dec64 = None
    if not args.no_b64:
        log("bench: decode B=64")
        dec64 = bench_decode(m, d, 64, 1024, 512, reps=1, warmup=0)
        log("bench: decode B=64", json.dumps(dec64))
    log("bench: speculative decode B=1")
    spec = bench_spec(m, d, reps=3, warmup=1)
    log("bench: decode spec", json.dumps(spec))
    log("bench: sampled decode B=1")
    samp = bench_sample(m, d, reps=3, warmup=1)
    log("bench: decode sample", json.dumps(samp))
    cpu = None
    if not args.no_cpu:
        log("bench: CPU oracle baseline")
        cpu = cpu_baseline(d, w)
        cpu["decode_b1"] = cpu_decode_baseline(d, w, c.reshape(-1), s.reshape(-1))
        log("bench: cpu", json.dumps(cpu))

    if traffic is not None and pre["roofline"]["kernel_kind"] == PMC_KIND:
        pre["roofline"]["traffic"] = traffic["bytes"]
        pre["roofline"]["traffic_detail"] = traffic
    line = {
        "metric": METRIC, "value": pre["tok_s"], "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": pre["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) bf16-exact weights, uniform ids)",
        "config": {"workload": "depth-12 prefill, B=1, T=2048: fp32 logits [2048,8192] + "
                               "per-token CE", "global_batch": 1, "seq_len": 2048,
                   "parallelism": "single GPU"},
        "roofline": pre["roofline"],
        "cpu_baseline": cpu,
        "prefill": pre,
        "decode_b1": dec1,
        "decode_b64": dec64,
        "decode_spec": spec,
        "decode_sample": samp,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
