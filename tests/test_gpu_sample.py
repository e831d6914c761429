"""Token sampling on the GPU (fg_sample, fg_decode_sample) through the C ABI.

The device sampler against the oracle (oracle/sample.py, pinned in
tests/test_sample_host.py): the reference's known answers, then random
rows and histories over every option. The generator state must match
exactly; the drawn id must match unless the oracle's draw lies within
rounding of a cumulative boundary (the device sums and sorts in another
order: tree sums, ties in id order), which the test measures and reports.
The loop (chat_text's plain decode with sample_next) is checked against
stepping the engine one position at a time with the oracle choosing ids.
"""
import numpy as np
import pytest

from autoresearch_amd import engine
from autoresearch_amd.weights import Dims, rope_tables, seeded_weights, uniform_ids
from oracle import sample as S

pytestmark = pytest.mark.gpu

SMALL = Dims(n_layer=2, d_model=128, n_head=2, n_kv_head=1, head_dim=64, vocab=512)


@pytest.fixture(scope="module")
def m():
    mm = engine.Model(SMALL, stacks=seeded_weights(SMALL, 5))
    yield mm
    mm.close()


def dev(m, lg, gen=(), st=12345, **cfg):
    return m.sample(lg, gen, st, **cfg)


def test_kats_on_device(m):
    lg4 = np.array([-1.0, 2.0, 0.5, -0.5], np.float32)
    assert dev(m, lg4, st=1, temp=0.0)[0] == 1
    st, hits = 42, [0] * 4
    for _ in range(400):
        i, st = dev(m, lg4, st=st, temp=1.0)
        hits[i] += 1
    assert hits[1] > 200 and sum(h > 0 for h in hits) > 1
    lg5 = np.array([0, 1, 2, 3, 4], np.float32)
    assert dev(m, lg5, [3, 4, 4], 9, temp=0.0, nblock=2)[0] == 3
    assert dev(m, lg5, [3, 4, 4], 9, temp=0.0)[0] == 4
    st = 3
    for _ in range(50):
        i, st = dev(m, lg5, st=st, temp=1.0, topp=0.0)
        assert i == 4
    lgv = np.ones(8192, np.float32)
    lgv[5000] = 100.0
    assert dev(m, lgv, [1], 42, temp=0.0)[0] == 5000
    tok = dev(m, lgv, [1], 42, temp=0.0, byte_space=True)[0]
    assert tok < 128 or 256 <= tok < 512
    # temp <= 0 makes no draw: the state is left as it was
    assert dev(m, lg5, st=77, temp=0.0)[1] == 77


CFGS = [
    dict(temp=0.0),
    dict(temp=0.0, pres=0.7, freq=0.3, rep=1.3, nblock=3),
    dict(temp=1.0),
    dict(temp=0.7, topp=0.9),
    dict(temp=1.4, topp=0.5, pres=0.5, freq=0.2),
    dict(temp=0.9, topp=0.95, pres=0.4, freq=0.1, pwin=16, plen=0.8, rep=1.2, nblock=2),
    dict(temp=1e-8, topp=1.0),
    dict(temp=1.0, byte_space=True),
]


def margin(detail, u):
    c = np.asarray(detail["cums"], np.float64)
    return float(np.min(np.abs(c - u))) / max(detail["total"], 1e-30)


# 512 / 1500 / 3000 / 8192 entries: the sort's 1, 2, 4 and 8 keys per thread
@pytest.mark.parametrize("V", [512, 1500, 3000, 8192])
@pytest.mark.parametrize("ci", range(len(CFGS)))
def test_device_matches_oracle(m, V, ci):
    cfg = CFGS[ci]
    rng = np.random.default_rng(V + ci)
    near, mism = 0, 0
    for trial in range(12):
        lg = rng.normal(0, 2.0, V).astype(np.float32)
        ngen = int(rng.integers(0, 40))
        gen = rng.integers(0, min(V, 64), ngen).astype(np.int32)  # repeats likely
        st0 = int(rng.integers(-2**62, 2**62))
        got, st = dev(m, lg, gen, st0, **cfg)
        want, wst, det = S.sample_next(
            lg, cfg.get("temp", 0.0), cfg.get("topp", 1.0), cfg.get("pres", 0.0),
            cfg.get("freq", 0.0), cfg.get("rep", 1.0), cfg.get("pwin", 0), cfg.get("plen", 0.0),
            gen, ngen, cfg.get("nblock", 0), st0, byte_space=cfg.get("byte_space", False))
        assert st == wst  # the same number of draws, the same generator
        if got != want:
            mism += 1
            assert det is not None, "argmax differs"
            mg = margin(det, det["u"])
            assert mg < 1e-5, f"trial {trial}: {got} vs {want}, draw margin {mg}"
            near += 1
    print(f"V={V} cfg={cfg}: {mism} near-boundary differences of 12", flush=True)


def test_decode_sample_loop(m):
    d = SMALL
    prompt = uniform_ids(8, 12, d.vocab)
    n_gen = 48
    ntot = prompt.size + n_gen
    c, s = rope_tables(ntot, d.head_dim)
    m.set_rope(c.reshape(-1), s.reshape(-1))

    def fresh():
        kv = m.kv(1, ntot)
        kv.step_multi(prompt[:-1], want_logits=False)
        return kv

    # temp 0, no penalties: the greedy stream
    kv = fresh()
    g, _ = kv.decode_greedy(prompt[-1:], n_gen)
    kv.close()
    kv = fresh()
    out, st = kv.decode_sample(prompt, n_gen, seed=5, temp=0.0)
    assert kv.len == ntot - 1
    kv.close()
    assert np.array_equal(out, g[:, 0]) and st == 5
    # a drawn stream with penalties: engine steps + oracle choice per position
    cfg = dict(temp=0.9, topp=0.9, pres=0.3, freq=0.2, rep=1.1, nblock=3)
    kv = fresh()
    out, st_dev = kv.decode_sample(prompt, n_gen, seed=2024, **cfg)
    kv.close()
    kv = fresh()
    ids, st = [int(prompt[-1])], 2024
    gen = []
    for t in range(n_gen):
        lg, _ = kv.step(np.array([ids[-1]], np.int32))
        want, st, det = S.sample_next(lg[0], cfg["temp"], cfg["topp"], cfg["pres"], cfg["freq"],
                                      cfg["rep"], 0, 0.0, gen, len(gen), cfg["nblock"], st)
        if want != out[t]:
            mg = margin(det, det["u"])
            assert mg < 1e-5, f"step {t}: {out[t]} vs {want}, margin {mg}"
            print(f"near-boundary divergence at step {t}; stream compared up to it", flush=True)
            break
        gen.append(want)
        ids.append(want)
    else:
        assert st == st_dev
    kv.close()


SMALL_MHA = Dims(n_layer=2, d_model=256, n_head=2, n_kv_head=2, head_dim=128, vocab=1024)
# the grouped-KV persistent kernel's small build: 4 heads over 2 KV heads
SMALL_GQA2 = Dims(n_layer=2, d_model=512, n_head=4, n_kv_head=2, head_dim=128, vocab=1024)


@pytest.mark.parametrize("d", [SMALL_MHA, SMALL_GQA2], ids=["mha", "gqa"])
def test_decode_sample_loop_persistent(d):
    """On a shape a persistent B=1 kernel serves (one KV head per query
    head, or two shared KV heads), each sampled step's forward is one
    persistent launch (the timing records one per id) and the draw a kernel
    of its own. temp 0 gives decode_greedy's stream bit for bit (the same
    kernel); with penalties, the stream against stepping the engine one
    position at a time with the oracle choosing ids (the per-step logits
    come from the single-row kernels there, ~1e-6 apart), up to a
    near-boundary draw."""
    m = engine.Model(d, stacks=seeded_weights(d, 7))
    assert m.fused_decode()[0], m.fused_decode()[1]
    prompt = uniform_ids(18, 12, d.vocab)
    n_gen = 40
    ntot = prompt.size + n_gen
    c, s = rope_tables(ntot, d.head_dim)
    m.set_rope(c.reshape(-1), s.reshape(-1))

    def fresh():
        kv = m.kv(1, ntot)
        kv.step_multi(prompt[:-1], want_logits=False)
        return kv

    kv = fresh()
    g, _ = kv.decode_greedy(prompt[-1:], n_gen)
    kv.close()
    kv = fresh()
    m.timing(True)
    out, st = kv.decode_sample(prompt, n_gen, seed=3, temp=0.0)
    tm = m.timing_read()
    m.timing(False)
    kv.close()
    assert tm["decode_fused"][0] == n_gen, tm
    assert np.array_equal(out, g[:, 0]) and st == 3
    cfg = dict(temp=0.8, topp=0.9, pres=0.2, freq=0.1, rep=1.2, nblock=3)
    kv = fresh()
    out, st_dev = kv.decode_sample(prompt, n_gen, seed=77, **cfg)
    kv.close()
    m.set_fused_decode(False)  # (single steps on the per-kernel path)
    kv = fresh()
    ids, st = [int(prompt[-1])], 77
    gen = []
    for t in range(n_gen):
        lg, _ = kv.step(np.array([ids[-1]], np.int32))
        want, st, det = S.sample_next(lg[0], cfg["temp"], cfg["topp"], cfg["pres"], cfg["freq"],
                                      cfg["rep"], 0, 0.0, gen, len(gen), cfg["nblock"], st)
        if want != out[t]:
            mg = margin(det, det["u"])
            assert mg < 1e-5, f"step {t}: {out[t]} vs {want}, margin {mg}"
            print(f"near-boundary divergence at step {t}; stream compared up to it", flush=True)
            break
        gen.append(want)
        ids.append(want)
    else:
        assert st == st_dev
    kv.close()
    m.close()


def test_sample_errors(m):
    with pytest.raises(engine.FgptError):
        m.sample(np.zeros(8193, np.float32))
    kv = m.kv(2, 32)
    with pytest.raises(engine.FgptError, match="B=1"):
        kv.decode_sample(np.array([1, 2], np.int32), 4)
    kv.close()
