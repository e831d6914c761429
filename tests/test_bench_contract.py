"""The parts of bench.py's output contract that run without a GPU: it refuses
more than one GPU, and the roofline figure is algorithmic units per launch
over the mean launch time, against MI355X's published peaks."""
import os
import subprocess
import sys

import pytest

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_roofline_arithmetic():
    # kind -> (launches, total ms, algorithmic flops, algorithmic bytes)
    tm = {"gemm": (49, 1.40, 49 * 7.6e9, 49 * 15.0e6), "attn_chunk": (24, 0.50, 0.0, 0.0)}
    assert bench.dominant(tm) == "gemm"
    launch_s = 1.40e-3 / 49
    r = bench.roofline(tm["gemm"], tm["gemm"][2], "mfma", "gemm", "profiles/x.md")
    assert r["unit"] == "TFLOP/s" and r["peak"] == 2516.6
    assert r["achieved"] == pytest.approx(7.6e9 / launch_s / 1e12)
    assert r["frac"] == pytest.approx(r["achieved"] / 2516.6)
    assert r["avg_launch_us"] == pytest.approx(launch_s * 1e6)
    assert r["alg_flop_per_launch"] == pytest.approx(7.6e9)
    # the linears multiply hi and lo activation planes: twice the MFMA work
    assert r["mfma_executed_frac"] == pytest.approx(2 * r["frac"])
    assert r["profile"] == "profiles/x.md"
    h = bench.roofline(tm["gemm"], tm["gemm"][3], "hbm", "gemm", "profiles/x.md")
    assert h["unit"] == "GB/s" and h["peak"] == 8000.0
    assert h["achieved"] == pytest.approx(15.0e6 / launch_s / 1e9)


def test_decode_units_closed_form():
    """Per-unit decode bytes: bf16 weights but the embedding table once per
    step, one embedding row and (n+1 read + 1 written) bf16 KV positions per
    sequence: 182.45 MB + 36 864 B x (n + 2) at depth 12, mean 183.65 MB over
    the 16-id prompt + 32 steps workload and 3.20 GB over B=64 x 512 steps
    after 1024-id prompts; the depth-20 GQA model's mean is 747.1 MB."""
    from autoresearch_amd.weights import D12, GQA20
    assert bench.kv_pos_bytes(D12) == 36864 and bench.kv_pos_bytes(GQA20) == 20480
    w12 = 2 * (D12.params - D12.vocab * D12.d_model)
    assert w12 == pytest.approx(182.45e6, rel=1e-4)
    assert bench.decode_step_bytes(D12, 1, 15) == w12 + 2 * 768 + 36864 * 17
    m1 = sum(bench.decode_step_bytes(D12, 1, 15 + i) for i in range(32)) / 32
    assert m1 == pytest.approx(183.65e6, rel=1e-4)
    m64 = sum(bench.decode_step_bytes(D12, 64, 1023 + i) for i in range(512)) / 512
    assert m64 == pytest.approx(3.20e9, rel=2e-3)
    mg = sum(bench.decode_step_bytes(GQA20, 1, 2047 + i) for i in range(256)) / 256
    assert mg == pytest.approx(747.1e6, rel=1e-4)
    assert bench.prefill_flops(D12, 1, 2048) == pytest.approx(451.009314816e9, rel=1e-12)
    assert bench.prefill_flops(D12, 8, 2048) == pytest.approx(8 * 451.009314816e9, rel=1e-12)


def test_prefill_flop_count_closed_form():
    """The depth-12 T=2048 prefill's algorithmic flops, counted per matrix
    product of gpt_forward (src/lib/fortran_gpt.f90:54-199): QKV, proj, fc,
    proj2 per layer, causal attention (q.k and p.v over t+1 keys per query)
    and lm_head. The engine's per-launch figures sum to 451.009 GFLOP."""
    from autoresearch_amd.weights import D12 as d
    T, D, hd, H, KH, V, L = 2048, d.d_model, d.head_dim, d.n_head, d.n_kv_head, d.vocab, d.n_layer
    per_layer = 2 * T * D * (H + 2 * KH) * hd + 2 * T * (H * hd) * D + 2 * (2 * T * D * 4 * D)
    attn = 4 * hd * H * (T * (T + 1) // 2)
    total = L * (per_layer + attn) + 2 * T * D * V
    assert total == pytest.approx(451.009314816e9, rel=1e-12)
