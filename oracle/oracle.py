"""ctypes wrapper of oracle/liboracle.so, the CPU restatement of the reference path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, which check the engine's results against it or
time it. The product library never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

_f = C.POINTER(C.c_float)
_i = C.POINTER(C.c_int32)


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return os.path.join(_HERE, "liboracle.so")


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = C.CDLL(path)
        i32, i64, f32 = C.c_int32, C.c_int64, C.c_float
        sig = {
            "or_frand_fill": (None, [_i, _f, i32, f32]),
            "or_rope_tables": (None, [_f, _f, i32, i32]),
            "or_wte_lookup": (None, [_i, _f, _f, i32, i32, i32]),
            "or_rmsnorm0": (None, [_f, _f, i64, i32, f32]),
            "or_linear": (None, [_f, _f, _f, i64, i32, i32]),
            "or_rope": (None, [_f, _f, _f, _f, i32, i32, i32, i32]),
            "or_causal_attn": (None, [_f, _f, _f, _f, i32, i32, i32, i32, i32]),
            "or_attn_step": (None, [_f, _f, _f, _f, i32, i32, i32, i32, i32]),
            "or_attn_chunk": (None, [_f, _f, _f, _f, i32, i32, i32, i32, i32, i32]),
            "or_relu2": (None, [_f, i64]),
            "or_attn_pos_count": (None, [_f, _f, i32, i32, i32, i32, i32, f32, _i, _i]),
            "or_gpt_forward_pos": (None, [_i, _f, _f] + [_f] * 8 + [_f] + [i32] * 8 + [f32, f32, _i, _i]),
            "or_gpt_forward": (None, [_i, _f, _f] + [_f] * 8 + [_f] + [i32] * 8 + [f32]),
            "or_gpt_step": (i32, [_i, _f, _f] + [_f] * 8 + [_f, _f, _i, i32, _f] + [i32] * 7 + [f32]),
            "or_gpt_step_multi": (i32, [_i, _f, _f] + [_f] * 8 + [_f, _f, _i, i32, _f] + [i32] * 8 + [f32]),
            "or_nll": (None, [_f, _i, _f, i64, i32]),
            "or_argmax": (i32, [_f, i32]),
            "or_num_threads": (i32, []),
            "or_wt_cache": (None, [i32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_f)


def ip(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_i)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


# ----------------------------------------------------------------- kernels

def frand(seed: int, n: int, scale: float = 1.0):
    s = np.array([seed], dtype=np.int32)
    x = np.empty(n, dtype=np.float32)
    lib().or_frand_fill(ip(s), fp(x), n, scale)
    return x, int(s[0])


def rope_tables(T: int, hd: int):
    c = np.empty(T * (hd // 2), dtype=np.float32)
    s = np.empty_like(c)
    lib().or_rope_tables(fp(c), fp(s), T, hd)
    return c, s


def rmsnorm0(x, C_: int, eps: float = 1e-5):
    x = f32(x)
    y = np.empty_like(x)
    lib().or_rmsnorm0(fp(x), fp(y), x.size // C_, C_, eps)
    return y


def linear(x, w, IF: int, OF: int):
    x, w = f32(x), f32(w)
    BT = x.size // IF
    y = np.empty(BT * OF, dtype=np.float32)
    lib().or_linear(fp(x), fp(w), fp(y), BT, IF, OF)
    return y


def rope(x, cosb, sinb, B, T, H, D):
    x, cosb, sinb = f32(x), f32(cosb), f32(sinb)
    y = np.empty_like(x)
    lib().or_rope(fp(x), fp(cosb), fp(sinb), fp(y), B, T, H, D)
    return y


def causal_attn(q, k, v, B, T, H, KH, D):
    q, k, v = f32(q), f32(k), f32(v)
    y = np.empty_like(q)
    lib().or_causal_attn(fp(q), fp(k), fp(v), fp(y), B, T, H, KH, D)
    return y


def attn_step(q, K, V, B, H, KH, D, TC):
    q, K, V = f32(q), f32(K), f32(V)
    y = np.empty_like(q)
    lib().or_attn_step(fp(q), fp(K), fp(V), fp(y), B, H, KH, D, TC)
    return y


def attn_chunk(q, K, V, B, H, KH, D, TC_PREV, TB):
    q, K, V = f32(q), f32(K), f32(V)
    y = np.empty_like(q)
    lib().or_attn_chunk(fp(q), fp(K), fp(V), fp(y), B, H, KH, D, TC_PREV, TB)
    return y


def relu2(x):
    x = f32(x).copy()
    lib().or_relu2(fp(x), x.size)
    return x


def nll(logits, targets, V: int):
    logits, targets = f32(logits), i32(targets)
    out = np.empty(targets.size, dtype=np.float32)
    lib().or_nll(fp(logits), ip(targets), fp(out), targets.size, V)
    return out


def argmax(logits) -> int:
    logits = f32(logits)
    return int(lib().or_argmax(fp(logits), logits.size))


def _w(w: dict):
    return [fp(f32(w[n])) for n in ("wte", "c_q", "c_k", "c_v", "c_proj", "c_fc", "c_proj2", "lm_head")]


def _dims(d):
    return [d.vocab, d.d_model, d.n_head, d.n_kv_head, d.head_dim, d.n_layer]


def gpt_forward(ids, cosb, sinb, w: dict, d, B: int, T: int) -> np.ndarray:
    ids, cosb, sinb = i32(ids), f32(cosb), f32(sinb)
    assert ids.size == B * T
    out = np.empty(B * T * d.vocab, dtype=np.float32)
    ws = {n: f32(w[n]) for n in w}
    lib().or_gpt_forward(ip(ids), fp(cosb), fp(sinb), *_w(ws), fp(out), B, T, *_dims(d), d.eps)
    return out.reshape(B, T, d.vocab)


def attn_pos_count(q, k, B: int, T: int, H: int, KH: int, D: int, rel_tol: float = 1e-4):
    """attn_sgemm's positive-score count per (b, h) (npos) and how many of
    the scores sit within rel_tol of zero relative to sum |q_d k_d| (namb)."""
    npos = np.zeros(B * H, np.int32)
    namb = np.zeros(B * H, np.int32)
    lib().or_attn_pos_count(fp(f32(q)), fp(f32(k)), B, T, H, KH, D, rel_tol, ip(npos), ip(namb))
    return npos.reshape(B, H), namb.reshape(B, H)


def gpt_forward_pos(ids, cosb, sinb, w: dict, d, B: int, T: int, rel_tol: float = 1e-4):
    """gpt_forward's logits with each layer's positive-score counts
    (npos, namb: [L, B, H])."""
    ids, cosb, sinb = i32(ids), f32(cosb), f32(sinb)
    out = np.empty(B * T * d.vocab, dtype=np.float32)
    npos = np.zeros(d.n_layer * B * d.n_head, np.int32)
    namb = np.zeros_like(npos)
    ws = {n: f32(w[n]) for n in w}
    lib().or_gpt_forward_pos(ip(ids), fp(cosb), fp(sinb), *_w(ws), fp(out), B, T, *_dims(d),
                             d.eps, rel_tol, ip(npos), ip(namb))
    sh = (d.n_layer, B, d.n_head)
    return out.reshape(B, T, d.vocab), npos.reshape(sh), namb.reshape(sh)


class KVCache:
    """Host fp32 cache in the reference layout, L x maxT x (KVH*hd) per tensor."""

    def __init__(self, d, maxT: int):
        n = d.n_layer * maxT * d.n_kv_head * d.head_dim
        self.k = np.zeros(n, dtype=np.float32)
        self.v = np.zeros(n, dtype=np.float32)
        self.maxT = maxT
        self.len = np.zeros(1, dtype=np.int32)


def gpt_step(ids1, cos1, sin1, w: dict, d, kv: KVCache) -> np.ndarray:
    ids1, cos1, sin1 = i32(ids1), f32(cos1), f32(sin1)
    out = np.empty(d.vocab, dtype=np.float32)
    ws = {n: f32(w[n]) for n in w}
    rc = lib().or_gpt_step(ip(ids1), fp(cos1), fp(sin1), *_w(ws), fp(kv.k), fp(kv.v),
                           ip(kv.len), kv.maxT, fp(out), 1, *_dims(d), d.eps)
    if rc != 0:
        raise RuntimeError("gpt_step: cache full (raise maxT)")
    return out


def gpt_step_multi(ids, cosb, sinb, w: dict, d, kv: KVCache) -> np.ndarray:
    ids, cosb, sinb = i32(ids), f32(cosb), f32(sinb)
    TB = ids.size
    out = np.empty(max(TB, 1) * d.vocab, dtype=np.float32)
    ws = {n: f32(w[n]) for n in w}
    rc = lib().or_gpt_step_multi(ip(ids), fp(cosb), fp(sinb), *_w(ws), fp(kv.k), fp(kv.v),
                                 ip(kv.len), kv.maxT, fp(out), 1, *_dims(d), TB, d.eps)
    if rc == 1:
        raise ValueError("gpt_step_multi: TB must be >= 1")
    if rc == 2:
        raise RuntimeError("gpt_step_multi: cache full (raise maxT)")
    return out.reshape(TB, d.vocab)


def greedy_decode(prompt, w: dict, d, n_gen: int, cosb, sinb, maxT: int,
                  prefill_multi: bool = False):
    """The ids-in/ids-out loop of src/app/chat_text.f90:257-278,423-462 with
    plain argmax: prompt[:-1] through gpt_step (or, with prefill_multi, one
    gpt_step_multi call, as a chunked prefill does), then n_gen steps each fed
    the previous id. Returns (generated ids, per-step logits)."""
    prompt = i32(prompt)
    hd2 = d.head_dim // 2
    kv = KVCache(d, maxT)
    cosb, sinb = f32(cosb).reshape(-1), f32(sinb).reshape(-1)
    if prefill_multi and prompt.size > 1:
        gpt_step_multi(prompt[:-1], cosb, sinb, w, d, kv)
    else:
        for t in range(prompt.size - 1):
            gpt_step(prompt[t:t + 1], cosb[t * hd2:], sinb[t * hd2:], w, d, kv)
    ids = list(prompt)
    logits = []
    for step in range(n_gen):
        tc = prompt.size - 1 + step
        lg = gpt_step(np.array([ids[tc]], np.int32), cosb[tc * hd2:], sinb[tc * hd2:], w, d, kv)
        logits.append(lg)
        ids.append(argmax(lg))
    return np.array(ids[prompt.size:], dtype=np.int32), np.stack(logits)
