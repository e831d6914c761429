"""The Fortran host layer: the iso_c_binding module, the drop-in
gpt_forward / gpt_step / gpt_step_multi, the ids-in/ids-out harness
(autoresearch_amd/fgpt_run) and the drop-in check program
(tests/fortran/dropin_checks), checked against the CPU oracle."""
import os
import subprocess

import numpy as np
import pytest

from autoresearch_amd.weights import (D12, Dims, seeded_weights, uniform_ids, write_npy_dir,
                                      write_safetensors, zipf_ids, BOS_ID)
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "autoresearch_amd", "fgpt_run")
CHECKS = os.path.join(ROOT, "tests", "fortran", "dropin_checks")
SMALL = Dims(n_layer=2, d_model=128, n_head=2, n_kv_head=1, head_dim=64, vocab=512)


def dims_args(d):
    return [str(x) for x in (d.n_layer, d.d_model, d.n_head, d.n_kv_head, d.head_dim, d.vocab)]


def run(args, timeout=300):
    return subprocess.run([EXE, *args], capture_output=True, text=True, timeout=timeout)


def run_checks(args, timeout=300):
    return subprocess.run([CHECKS, *args], capture_output=True, text=True, timeout=timeout)


def test_harness_built_and_fails_loudly_without_device():
    import torch
    assert os.path.exists(EXE), "build() must compile the Fortran harness"
    assert os.path.exists(CHECKS), "build() must compile the drop-in check program"
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    r = run_checks(["selftest"], timeout=60)
    assert r.returncode != 0
    assert "no HIP device" in r.stderr or "gfx950" in r.stderr


def test_harness_usage_error():
    r = run(["nonsense"], timeout=30)
    assert r.returncode == 2 and "usage" in r.stderr
    r = run_checks(["nonsense"], timeout=30)
    assert r.returncode == 2 and "usage" in r.stderr


@pytest.mark.gpu
def test_fortran_selftest_steps_equal_forward():
    r = run_checks(["selftest"], timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and "selftest: ok" in r.stdout


@pytest.mark.gpu
def test_fortran_posfrac_attn_blas(tmp_path):
    """eval_bpb --attn blas through the drop-in: gpt_forward with attn_blas
    and pos_frac / pos_n, called twice into the same accumulators and then
    once without attn_blas (which leaves them alone). pos_n must count one
    addition per (call, layer, row); pos_frac must equal the reference's
    accumulation (src/lib/fortran_attn.f90:291-296, fp32, (layer, row)
    order) of the CPU oracle's positive-score counts on the same inputs,
    within the counts whose score sits within rounding of zero."""
    d = SMALL
    w = seeded_weights(d, 61)
    write_npy_dir(str(tmp_path / "w"), d, w, ctx=160)
    B, T, ncall = 2, 96, 2
    rows = uniform_ids(62, B * T, d.vocab)
    np.savetxt(tmp_path / "rows.txt", rows[None, :], fmt="%d")
    r = run_checks(["posfrac", str(tmp_path / "w"), *dims_args(d), str(tmp_path / "rows.txt"),
                    str(B), str(T), str(ncall), str(tmp_path / "pf.txt")])
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    got = np.loadtxt(tmp_path / "pf.txt").reshape(d.n_head, 2)
    c, s = O.rope_tables(T, d.head_dim)
    _, npos, namb = O.gpt_forward_pos(rows, c, s, w, d, B, T)
    assert np.array_equal(got[:, 1], np.full(d.n_head, ncall * d.n_layer * B))
    den = np.float32(T * (T + 1) // 2)
    pf = np.zeros(d.n_head, np.float32)
    lo = np.zeros(d.n_head, np.float32)
    hi = np.zeros(d.n_head, np.float32)
    for _ in range(ncall):
        for ll in range(d.n_layer):
            for aa in range(B):
                for hh in range(d.n_head):
                    n, a = npos[ll, aa, hh], namb[ll, aa, hh]
                    pf[hh] = np.float32(pf[hh] + np.float32(n) / den)
                    lo[hh] = np.float32(lo[hh] + np.float32(n - a) / den)
                    hi[hh] = np.float32(hi[hh] + np.float32(n + a) / den)
    print("pos_frac", got[:, 0], "oracle", pf, "ambiguous scores", int(namb.sum()))
    assert np.all(got[:, 0] >= lo * (1 - 1e-6)) and np.all(got[:, 0] <= hi * (1 + 1e-6))
    if namb.sum() == 0:
        assert np.array_equal(got[:, 0].astype(np.float32), pf)


def oracle_greedy(d, w, prompt, ngen):
    c, s = O.rope_tables(prompt.size + ngen, d.head_dim)
    return O.greedy_decode(prompt, w, d, ngen, c, s, maxT=prompt.size + ngen)[0]


@pytest.mark.gpu
@pytest.mark.parametrize("loop,pchunk", [("host", 64), ("device", 4)])
def test_fortran_greedy_small(tmp_path, loop, pchunk):
    d = SMALL
    w = seeded_weights(d, 21)
    write_npy_dir(str(tmp_path / "w"), d, w, ctx=64)
    prompt = uniform_ids(31, 11, d.vocab)
    np.savetxt(tmp_path / "ids.txt", prompt, fmt="%d")
    r = run(["greedy", str(tmp_path / "w"), *dims_args(d), str(tmp_path / "ids.txt"), "20",
             str(tmp_path / "out.txt"), str(pchunk), loop])
    print(r.stdout, r.stderr)
    assert r.returncode == 0
    got = np.loadtxt(tmp_path / "out.txt", dtype=np.int32)
    assert np.array_equal(got, oracle_greedy(d, w, prompt, 20))


@pytest.mark.gpu
def test_fortran_greedy_from_safetensors(tmp_path):
    """A checkpoint directory holding only model.safetensors (the trainer's
    default output) drives the same greedy run as the .npy export."""
    d = SMALL
    w = seeded_weights(d, 21)
    write_safetensors(str(tmp_path / "w"), d, w, ctx=64)
    prompt = uniform_ids(31, 11, d.vocab)
    np.savetxt(tmp_path / "ids.txt", prompt, fmt="%d")
    r = run(["greedy", str(tmp_path / "w"), *dims_args(d), str(tmp_path / "ids.txt"), "20",
             str(tmp_path / "out.txt"), "64", "device"])
    print(r.stdout, r.stderr)
    assert r.returncode == 0
    got = np.loadtxt(tmp_path / "out.txt", dtype=np.int32)
    assert np.array_equal(got, oracle_greedy(d, w, prompt, 20))
    # declared arch that disagrees with the dims stops the program
    write_safetensors(str(tmp_path / "bad"), d, w, ctx=64, metadata={"arch.n_layer": 3})
    r = run(["greedy", str(tmp_path / "bad"), *dims_args(d), str(tmp_path / "ids.txt"), "2",
             str(tmp_path / "o2.txt")])
    assert r.returncode != 0 and "architecture mismatch" in r.stderr


@pytest.mark.gpu
def test_fortran_greedy_depth12(tmp_path):
    """The B=1 decode workload through the Fortran drop-in: 16 prompt ids,
    32 greedy steps, host argmax per step as chat_text does."""
    d = D12
    w = seeded_weights(d, 1234)
    write_npy_dir(str(tmp_path / "w"), d, w)
    prompt = uniform_ids(42, 16, d.vocab)
    np.savetxt(tmp_path / "ids.txt", prompt, fmt="%d")
    ref = oracle_greedy(d, w, prompt, 32)
    for loop in ("host", "device"):
        r = run(["greedy", str(tmp_path / "w"), *dims_args(d), str(tmp_path / "ids.txt"), "32",
                 str(tmp_path / f"out_{loop}.txt"), "64", loop])
        print(r.stderr)
        assert r.returncode == 0
        got = np.loadtxt(tmp_path / f"out_{loop}.txt", dtype=np.int32)
        assert np.array_equal(got, ref), loop


@pytest.mark.gpu
def test_fortran_eval_rows(tmp_path):
    d = SMALL
    w = seeded_weights(d, 22)
    write_npy_dir(str(tmp_path / "w"), d, w, ctx=128)
    B, T = 3, 96
    rows = zipf_ids(5, B * (T + 1), d.vocab).reshape(B, T + 1)
    rows[:, 0] = BOS_ID % d.vocab
    np.savetxt(tmp_path / "rows.txt", rows.reshape(-1), fmt="%d")
    r = run(["eval", str(tmp_path / "w"), *dims_args(d), str(tmp_path / "rows.txt"), str(B),
             str(T), str(tmp_path / "nll.txt")])
    print(r.stderr)
    assert r.returncode == 0
    got = np.loadtxt(tmp_path / "nll.txt")
    c, s = O.rope_tables(T, d.head_dim)
    for b in range(B):
        lg = O.gpt_forward(rows[b, :T], c, s, w, d, 1, T)
        ref = float(O.nll(lg.reshape(T, -1), rows[b, 1:], d.vocab).astype(np.float64).sum())
        assert abs(got[b] - ref) < 2 * 2e-3 * np.abs(lg).max() * T
        assert abs(got[b] - ref) < 1e-3 * T


@pytest.mark.gpu
def test_fortran_eval_rows_f16(tmp_path):
    """fgpt_forward_f16(.true.): the same rows through single-term fp16
    gpt_forward passes (288 rows), within the contract's bar."""
    d = SMALL
    w = seeded_weights(d, 22)
    write_npy_dir(str(tmp_path / "w"), d, w, ctx=128)
    B, T = 3, 96
    rows = zipf_ids(5, B * (T + 1), d.vocab).reshape(B, T + 1)
    rows[:, 0] = BOS_ID % d.vocab
    np.savetxt(tmp_path / "rows.txt", rows.reshape(-1), fmt="%d")
    args = ["eval", str(tmp_path / "w"), *dims_args(d), str(tmp_path / "rows.txt"), str(B), str(T)]
    r = run(args + [str(tmp_path / "nll16.txt"), "f16"])
    print(r.stderr)
    assert r.returncode == 0
    r32 = run(args + [str(tmp_path / "nll.txt")])
    assert r32.returncode == 0
    got, split = np.loadtxt(tmp_path / "nll16.txt"), np.loadtxt(tmp_path / "nll.txt")
    c, s = O.rope_tables(T, d.head_dim)
    for b in range(B):
        lg = O.gpt_forward(rows[b, :T], c, s, w, d, 1, T)
        ref = float(O.nll(lg.reshape(T, -1), rows[b, 1:], d.vocab).astype(np.float64).sum())
        assert abs(got[b] - ref) < 2 * 2e-3 * np.abs(lg).max() * T
        assert abs(got[b] - ref) < 1e-3 * T
    assert not np.array_equal(got, split)  # the option reached the engine


@pytest.mark.gpu
def test_fortran_arch_mismatch_stops(tmp_path):
    d = SMALL
    w = seeded_weights(d, 23)
    write_npy_dir(str(tmp_path / "w"), d, w, ctx=64)
    np.savetxt(tmp_path / "ids.txt", [1, 2, 3], fmt="%d")
    wrong = dims_args(d)
    wrong[3] = "2"  # n_kv_head 2 vs arch.txt n_kv = 1
    r = run(["greedy", str(tmp_path / "w"), *wrong, str(tmp_path / "ids.txt"), "2",
             str(tmp_path / "o.txt")])
    assert r.returncode != 0 and "arch.txt" in r.stdout + r.stderr


@pytest.mark.gpu
def test_fortran_bpb_rows_npy(tmp_path):
    """eval_bpb + bpb_agg through the harness: a Fortran-order (N, T+1) int32
    rows .npy, a token byte-length table, the summary line of bpb_agg and the
    per-position NLL lines of eval_bpb, against the oracle weighted on the
    host (scripts/eval_driver.py:174-190)."""
    d = SMALL
    w = seeded_weights(d, 29)
    write_safetensors(str(tmp_path / "w"), d, w, ctx=64)
    N, T = 3, 40
    rows = zipf_ids(3, N * (T + 1), d.vocab).reshape(N, T + 1)
    rows[:, 0] = 7
    np.save(tmp_path / "rows.npy", np.asfortranarray(rows))
    tb = uniform_ids(8, d.vocab, 4)      # 0..3 bytes per token
    np.savetxt(tmp_path / "tb.txt", tb, fmt="%d")
    r = run(["bpb", str(tmp_path / "w"), *dims_args(d), str(tmp_path / "rows.npy"),
             str(tmp_path / "tb.txt"), "2", str(tmp_path / "nll.txt")])
    print(r.stdout, r.stderr)
    assert r.returncode == 0
    c, s = O.rope_tables(T, d.head_dim)
    nats, nbytes, maxlg = 0.0, 0, 0.0
    lines = open(tmp_path / "nll.txt").read().split("\n")
    for b in range(N):
        lg = O.gpt_forward(rows[b, :T], c, s, w, d, 1, T).reshape(T, d.vocab)
        nl = O.nll(lg, rows[b, 1:], d.vocab).astype(np.float64)
        got = np.array(lines[b].split(), dtype=np.float64)
        assert got.size == T and np.abs(got - nl).max() < 2 * 2e-3 * np.abs(lg).max()
        keep = tb[rows[b, 1:]] > 0
        nats += nl[keep].sum()
        nbytes += int(tb[rows[b, 1:]][keep].sum())
        maxlg = max(maxlg, float(np.abs(lg).max()))
    summary = [x for x in r.stdout.split("\n") if x.startswith("rows=")][0]
    kv = dict(p.split("=") for p in summary.split())
    assert int(kv["rows"]) == N and int(kv["bytes"]) == nbytes
    bpb = nats / nbytes / np.log(2)
    assert abs(float(kv["bpb"]) - bpb) < 1e-4 * bpb + 1e-5


def test_fortran_spectest_reference_kats(tmp_path):
    """accept_prefix / lookup_draft through the drop-in names on the
    reference's known answers (host functions: no device needed). The KAT
    program (tests/fortran/spectest_kats.f90) is compiled here against the
    built drop-in modules."""
    from autoresearch_amd import build as B
    fmod = os.path.join(B.BUILD, "fmod")
    objs = [os.path.join(B.BUILD, s.replace(".f90", ".o")) for s in B.F_SOURCES]
    assert all(os.path.exists(o) for o in objs), "build() must compile the Fortran modules"
    exe = str(tmp_path / "spectest_kats")
    c = subprocess.run([B.FLANG, "-O1", "-I", fmod, os.path.join(ROOT, "tests", "fortran",
                        "spectest_kats.f90"), *objs, "-L", B.PKG, "-lfgpt",
                        f"-Wl,-rpath,{B.PKG}", "-o", exe], capture_output=True, text=True,
                       timeout=120)
    assert c.returncode == 0, c.stdout + c.stderr
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and "spectest: 12 of 12 checks passed" in r.stdout


@pytest.mark.gpu
def test_fortran_specbench_trunc_drafter(tmp_path):
    """src/app/spec_bench.f90's truncated-drafter run through the drop-in:
    target and drafter (first 1 of 2 layers of the same arrays) on two
    caller caches, prefill of both, a plain greedy run, then draft-and-verify
    rounds with cache_len rolled back on both caches. The plain stream must
    be the oracle's greedy ids and the speculative stream must equal it."""
    d = SMALL
    w = seeded_weights(d, 31)
    write_npy_dir(str(tmp_path / "w"), d, w, ctx=160)
    ids = uniform_ids(47, 40, d.vocab)
    np.savetxt(tmp_path / "rows.txt", ids[None, :], fmt="%d")
    npre, ngen = 33, 48
    r = run_checks(["specbench", str(tmp_path / "w"), *dims_args(d), str(tmp_path / "rows.txt"),
             str(npre), str(ngen), str(tmp_path / "o.txt"), "4", "1"])
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "EQUIVALENCE ok" in r.stdout and "passes=" in r.stdout
    got = np.loadtxt(tmp_path / "o.txt", dtype=np.int32).reshape(-1)
    assert np.array_equal(got, oracle_greedy(d, w, ids[:npre], ngen))


@pytest.mark.gpu
def test_fortran_specbench_depth12(tmp_path):
    """The same run at the depth-12 shape with spec_bench's defaults (K=8,
    3 drafter layers), 64 prompt ids and 32 generated."""
    d = D12
    w = seeded_weights(d, 1234)
    write_npy_dir(str(tmp_path / "w"), d, w)
    ids = uniform_ids(48, 70, d.vocab)
    np.savetxt(tmp_path / "rows.txt", ids[None, :], fmt="%d")
    r = run_checks(["specbench", str(tmp_path / "w"), *dims_args(d), str(tmp_path / "rows.txt"), "64",
             "32", str(tmp_path / "o.txt")])
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "EQUIVALENCE ok" in r.stdout
    got = np.loadtxt(tmp_path / "o.txt", dtype=np.int32).reshape(-1)
    assert np.array_equal(got, oracle_greedy(d, w, ids[:64], 32))


@pytest.mark.gpu
def test_fortran_spec_equals_greedy(tmp_path):
    """chat_text --spec semantics through the harness: the speculative stream
    equals the plain greedy stream (printed EQUIVALENCE line) and the oracle's
    greedy ids."""
    d = SMALL
    w = seeded_weights(d, 23)
    write_npy_dir(str(tmp_path / "w"), d, w, ctx=160)
    base = uniform_ids(41, 10, d.vocab)
    prompt = np.concatenate([base, base, base[:4]]).astype(np.int32)
    np.savetxt(tmp_path / "p.txt", prompt[None, :], fmt="%d")
    ngen = 60
    r = run(["spec", str(tmp_path / "w"), *dims_args(d), str(tmp_path / "p.txt"), str(ngen),
             str(tmp_path / "o.txt"), "6", "2", "4", "0.5"])
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    assert "EQUIVALENCE ok" in r.stdout
    assert "passes=" in r.stdout
    got = np.loadtxt(tmp_path / "o.txt", dtype=np.int32).reshape(-1)
    assert np.array_equal(got, oracle_greedy(d, w, prompt, ngen))


@pytest.mark.gpu
def test_fortran_sample_host_loop_equals_device_loop(tmp_path):
    """chat_text's plain loop with sample_next: stepping through the drop-in
    gpt_step + sample_next gives the same ids and generator state as one
    fg_decode_sample call; temp 0 gives the oracle's greedy ids."""
    d = SMALL
    w = seeded_weights(d, 29)
    write_npy_dir(str(tmp_path / "w"), d, w, ctx=96)
    prompt = uniform_ids(43, 9, d.vocab)
    np.savetxt(tmp_path / "p.txt", prompt, fmt="%d")
    ngen = 40
    outs = {}
    for loop in ("host", "device"):
        r = run(["sample", str(tmp_path / "w"), *dims_args(d), str(tmp_path / "p.txt"), str(ngen),
                 str(tmp_path / f"o_{loop}.txt"), "0.9", "0.92", "777", "0.3", "0.1", "1.15", "12",
                 "0.5", "3", "0", loop])
        print(r.stdout, r.stderr)
        assert r.returncode == 0, r.stderr
        outs[loop] = (np.loadtxt(tmp_path / f"o_{loop}.txt", dtype=np.int32),
                      r.stdout.strip().splitlines()[-1])
    assert np.array_equal(outs["host"][0], outs["device"][0])
    assert outs["host"][1] == outs["device"][1]  # rng_state=...
    r = run(["sample", str(tmp_path / "w"), *dims_args(d), str(tmp_path / "p.txt"), str(ngen),
             str(tmp_path / "g.txt"), "0", "1", "1", "0", "0", "1", "0", "0", "0", "0", "device"])
    assert r.returncode == 0, r.stderr
    got = np.loadtxt(tmp_path / "g.txt", dtype=np.int32)
    assert np.array_equal(got, oracle_greedy(d, w, prompt, ngen))
