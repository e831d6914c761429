"""An independent float64 numpy formulation of the fortran_gpt forward.

Written as whole-tensor algebra (matrix products, complex rotation for RoPE,
a masked softmax), not as the reference's loops, so that it checks the C
oracle rather than restating it. Used only by the CPU tests.
"""
import numpy as np


def rmsnorm(x, eps):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def rope(x, cosb, sinb):
    """x (..., T, H, D) rotated by exp(-i*angle) on (x[:D/2], x[D/2:]) pairs."""
    d2 = x.shape[-1] // 2
    z = x[..., :d2] + 1j * x[..., d2:]
    rot = (cosb - 1j * sinb)[:, None, :]          # (T, 1, D/2)
    zr = z * rot
    return np.concatenate([zr.real, zr.imag], axis=-1)


def attention(q, k, v, causal_offset=0):
    """q (Tq,H,D), k/v (Tk,KH,D); query i sees keys 0..causal_offset+i."""
    Tq, H, D = q.shape
    Tk, KH, _ = k.shape
    rep = H // KH
    kk = np.repeat(k, rep, axis=1)
    vv = np.repeat(v, rep, axis=1)
    s = np.einsum("qhd,khd->hqk", q, kk) / np.sqrt(D)
    mask = np.arange(Tk)[None, :] > (causal_offset + np.arange(Tq))[:, None]
    s = np.where(mask[None], -np.inf, s)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("hqk,khd->qhd", p, vv)


def forward(ids, cosb, sinb, w, d, B, T):
    """Logits (B, T, V) in float64. w holds the reference's stacked buffers."""
    D, H, KH, hd, L, V = d.d_model, d.n_head, d.n_kv_head, d.head_dim, d.n_layer, d.vocab
    f = {n: np.asarray(w[n], dtype=np.float64) for n in w}
    cos = np.asarray(cosb, np.float64).reshape(-1, hd // 2)[:T]
    sin = np.asarray(sinb, np.float64).reshape(-1, hd // 2)[:T]
    wte = f["wte"].reshape(V, D)
    x = rmsnorm(wte[np.asarray(ids).reshape(B, T)], d.eps)
    for l in range(L):
        Wq = f["c_q"].reshape(L, H * hd, D)[l]
        Wk = f["c_k"].reshape(L, KH * hd, D)[l]
        Wv = f["c_v"].reshape(L, KH * hd, D)[l]
        Wp = f["c_proj"].reshape(L, D, H * hd)[l]
        Wf = f["c_fc"].reshape(L, 4 * D, D)[l]
        W2 = f["c_proj2"].reshape(L, D, 4 * D)[l]
        xn = rmsnorm(x, d.eps)
        out = np.empty((B, T, H * hd))
        for b in range(B):
            q = rope((xn[b] @ Wq.T).reshape(T, H, hd), cos, sin)
            k = rope((xn[b] @ Wk.T).reshape(T, KH, hd), cos, sin)
            v = (xn[b] @ Wv.T).reshape(T, KH, hd)
            out[b] = attention(q, k, v).reshape(T, H * hd)
        x = x + out @ Wp.T
        h = np.maximum(rmsnorm(x, d.eps) @ Wf.T, 0.0) ** 2
        x = x + h @ W2.T
    return rmsnorm(x, d.eps) @ f["lm_head"].reshape(V, D).T


def nll(logits, targets):
    lg = np.asarray(logits, np.float64)
    m = lg.max(axis=-1, keepdims=True)
    lse = (m + np.log(np.exp(lg - m).sum(axis=-1, keepdims=True)))[..., 0]
    return lse - np.take_along_axis(lg, np.asarray(targets)[..., None], axis=-1)[..., 0]


def pos_counts(ids, cosb, sinb, w, d, B, T):
    """Per layer, row and head ([L, B, H]): how many causal scores
    q.k/sqrt(hd) are > 0 in float64 (attn_sgemm's statistic), and the
    smallest |q.k| / sum|q_d k_d| among them (how close any sign is to
    rounding)."""
    D, H, KH, hd, L, V = d.d_model, d.n_head, d.n_kv_head, d.head_dim, d.n_layer, d.vocab
    f = {n: np.asarray(w[n], dtype=np.float64) for n in w}
    cos = np.asarray(cosb, np.float64).reshape(-1, hd // 2)[:T]
    sin = np.asarray(sinb, np.float64).reshape(-1, hd // 2)[:T]
    x = rmsnorm(f["wte"].reshape(V, D)[np.asarray(ids).reshape(B, T)], d.eps)
    cnt = np.zeros((L, B, H), np.int64)
    closest = np.inf
    causal = np.tril(np.ones((T, T), bool))
    for l in range(L):
        Wq = f["c_q"].reshape(L, H * hd, D)[l]
        Wk = f["c_k"].reshape(L, KH * hd, D)[l]
        Wv = f["c_v"].reshape(L, KH * hd, D)[l]
        Wp = f["c_proj"].reshape(L, D, H * hd)[l]
        Wf = f["c_fc"].reshape(L, 4 * D, D)[l]
        W2 = f["c_proj2"].reshape(L, D, 4 * D)[l]
        xn = rmsnorm(x, d.eps)
        out = np.empty((B, T, H * hd))
        for b in range(B):
            q = rope((xn[b] @ Wq.T).reshape(T, H, hd), cos, sin)
            k = rope((xn[b] @ Wk.T).reshape(T, KH, hd), cos, sin)
            v = (xn[b] @ Wv.T).reshape(T, KH, hd)
            kk = np.repeat(k, H // KH, axis=1)
            s = np.einsum("qhd,khd->hqk", q, kk)
            mag = np.einsum("qhd,khd->hqk", np.abs(q), np.abs(kk))
            cnt[l, b] = ((s > 0) & causal[None]).sum(axis=(1, 2))
            closest = min(closest, float((np.abs(s) / mag)[:, causal].min()))
            out[b] = attention(q, k, v).reshape(T, H * hd)
        x = x + out @ Wp.T
        h = np.maximum(rmsnorm(x, d.eps) @ Wf.T, 0.0) ** 2
        x = x + h @ W2.T
    return cnt, closest
