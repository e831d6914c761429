"""fg_step_dev_noalloc (a cached step that allocates nothing: its scratch is
the library's own per-GPU device array) against fg_step, through the C ABI,
on twin caches filled by the same prefill: the same kernels on the same
inputs, so logits, next ids and the cache rows written must be identical.
Two calls in a row, the second with fewer sequences, one whose attention
spans several chunks (merged in the launch, with the arrival counters at
the array's start), then the refusals: sizes beyond the array, and a call
on a second stream while the first stream's call may still be running.
"""
import ctypes as C

import numpy as np
import pytest

from autoresearch_amd import engine
from autoresearch_amd.weights import D12, Dims, rope_tables, seeded_weights, uniform_ids

from .devbuf import DevBuf

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def d12():
    m = engine.Model(D12, stacks=seeded_weights(D12, 1234))
    c, s = rope_tables(320, D12.head_dim)
    m.set_rope(c.reshape(-1), s.reshape(-1))
    yield D12, m
    m.close()


def noalloc_vs_step(d, m, B, P, seed, n_steps=3):
    prompts = uniform_ids(seed, B * P, d.vocab).reshape(B, P)
    ka, kb = m.kv(B, P + n_steps), m.kv(B, P + n_steps)
    for kv in (ka, kb):
        kv.step_multi(prompts[:, :-1], want_logits=False)
    ids = prompts[:, -1].astype(np.int32)
    d_ids = DevBuf(ids)
    d_lg = DevBuf(np.zeros(B * d.vocab, np.float32))
    d_nx = DevBuf(np.zeros(B, np.int32))
    for _ in range(n_steps):
        lg_a, nx_a = ka.step(ids)
        kb.step_dev_noalloc(d_ids.ptr, d_lg.ptr, d_nx.ptr)
        m.sync()
        lg_b = d_lg.get().reshape(B, d.vocab)
        nx_b = d_nx.get()
        assert np.array_equal(nx_a, nx_b)
        assert np.array_equal(lg_a, lg_b)
        ids = nx_a.astype(np.int32)
        d_ids.put(ids)
    for b_ in (d_ids, d_lg, d_nx):
        b_.free()
    assert ka.len == kb.len == P - 1 + n_steps
    (k_a, v_a), (k_b, v_b) = ka.read(), kb.read()
    assert np.array_equal(k_a, k_b) and np.array_equal(v_a, v_b)
    ka.close()
    kb.close()


def test_noalloc_step_equals_step_then_smaller(d12):
    d, m = d12
    noalloc_vs_step(d, m, B=4, P=9, seed=3)
    noalloc_vs_step(d, m, B=2, P=5, seed=4)
    # 300 cached positions: five 64-position chunks per head, merged by the
    # last chunk workgroup to arrive; then a short one again (counters left
    # zero by the previous launches)
    noalloc_vs_step(d, m, B=2, P=300, seed=5)
    noalloc_vs_step(d, m, B=1, P=7, seed=6)


def test_noalloc_second_stream_refused_while_busy(d12):
    """A call on stream B while stream A's call may still run fails with
    FG_EBUSY and leaves the cache alone; once A has finished, B may call."""
    d, m = d12
    P = 9
    kv = m.kv(1, P + 2)
    kv.step_multi(uniform_ids(7, P, d.vocab)[None, :-1], want_logits=False)
    d_ids = DevBuf(np.array([5], np.int32))
    d_lg = DevBuf(np.zeros(d.vocab, np.float32))
    hip = DevBuf.hip
    sa, sb, big = C.c_void_p(), C.c_void_p(), C.c_void_p()
    assert hip.hipStreamCreateWithFlags(C.byref(sa), 1) == 0
    assert hip.hipStreamCreateWithFlags(C.byref(sb), 1) == 0
    nbig = 8 << 30
    assert hip.hipMalloc(C.byref(big), C.c_size_t(nbig)) == 0
    try:
        # ~1.5 ms of fill ahead of A's step keeps it queued while B calls
        assert hip.hipMemsetAsync(big, 0, C.c_size_t(nbig), sa) == 0
        kv.step_dev_noalloc(d_ids.ptr, d_lg.ptr, stream=sa.value)
        with pytest.raises(engine.FgptError, match="another stream"):
            kv.step_dev_noalloc(d_ids.ptr, d_lg.ptr, stream=sb.value)
        assert kv.len == P
        assert hip.hipStreamSynchronize(sa) == 0
        kv.step_dev_noalloc(d_ids.ptr, d_lg.ptr, stream=sb.value)
        assert hip.hipStreamSynchronize(sb) == 0
        assert kv.len == P + 1
    finally:
        hip.hipStreamSynchronize(sa)
        hip.hipStreamSynchronize(sb)
        hip.hipFree(big)
        hip.hipStreamDestroy(sa)
        hip.hipStreamDestroy(sb)
        kv.close()
        d_ids.free()
        d_lg.free()


def test_noalloc_refusals(d12):
    d, m = d12
    d_ids = DevBuf(np.zeros(8, np.int32))
    d_lg = DevBuf(np.zeros(8 * d.vocab, np.float32))
    kv = m.kv(8, 16)  # 8 sequences take the GEMM path
    with pytest.raises(engine.FgptError, match="single-row path"):
        kv.step_dev_noalloc(d_ids.ptr, d_lg.ptr)
    kv.close()
    # 4 sequences x 8 heads x 16000 positions of attention partials exceed
    # the 4 MiB array
    dw = Dims(n_layer=1, d_model=1024, n_head=8, n_kv_head=8, head_dim=128, vocab=256)
    mw = engine.Model(dw, stacks=seeded_weights(dw, 1))
    c, s = rope_tables(4, dw.head_dim)
    mw.set_rope(c.reshape(-1), s.reshape(-1))
    kv = mw.kv(4, 16000)
    d_lw = DevBuf(np.zeros(4 * dw.vocab, np.float32))
    with pytest.raises(engine.FgptError, match="scratch"):
        kv.step_dev_noalloc(d_ids.ptr, d_lw.ptr)
    assert kv.len == 0
    kv.close()
    mw.close()
    for b_ in (d_ids, d_lg, d_lw):
        b_.free()
