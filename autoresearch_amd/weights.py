"""Model dims, seeded synthetic weights and ids, and the `.npy` weight layout.

The on-disk layout is the reference loader's: one 1-D ``<f4`` C-order
``.npy`` per tensor (``scripts/export_weights.py:22-24,151-166``), named as
``src/lib/load_weights.f90:7-9`` lists them, per-layer tensors stacked by
``load_gpt_weights`` (``src/lib/load_weights.f90:853-873``), plus the
``arch.txt`` sidecar of ``src/lib/fortran_arch.f90:100-116``.

Synthetic weights are i.i.d. N(0, std) from a counter-based splitmix64
stream (one stream per tensor) through Box-Muller, rounded to bf16 with
round-to-nearest-even and stored widened to fp32, so the fp32 CPU oracle and
the bf16 engine hold bit-identical values (csrc/seedgen.c).
"""
from __future__ import annotations

import dataclasses
import os
import struct

import numpy as np


@dataclasses.dataclass(frozen=True)
class Dims:
    n_layer: int
    d_model: int
    n_head: int
    n_kv_head: int
    head_dim: int
    vocab: int
    eps: float = 1e-5

    @property
    def d_ff(self) -> int:  # hard-wired 4*d_model, src/lib/fortran_gpt.f90:105
        return 4 * self.d_model

    @property
    def params(self) -> int:
        d, L = self.d_model, self.n_layer
        per = (self.n_head * self.head_dim * d + 2 * self.n_kv_head * self.head_dim * d
               + d * self.n_head * self.head_dim + 2 * self.d_ff * d)
        return 2 * self.vocab * d + L * per


D12 = Dims(n_layer=12, d_model=768, n_head=6, n_kv_head=6, head_dim=128, vocab=8192)
GQA20 = Dims(n_layer=20, d_model=1280, n_head=10, n_kv_head=2, head_dim=128, vocab=8192)
BOS_ID = 8188  # ARCH_BOS, src/lib/fortran_arch.f90:60

STACK_NAMES = ("wte", "c_q", "c_k", "c_v", "c_proj", "c_fc", "c_proj2", "lm_head")

_SEED_LIB = None


def _seedlib():
    """autoresearch_amd/libfgpt_seed.so (built from csrc/seedgen.c)."""
    global _SEED_LIB
    if _SEED_LIB is None:
        import ctypes as C
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libfgpt_seed.so")
        if not os.path.exists(path):
            from . import build
            build.build_seedgen()
        L = C.CDLL(path)
        L.sg_normal_bf16.argtypes = [C.c_uint64, C.c_uint64, C.c_int64, C.c_double, C.c_void_p]
        L.sg_normal_bf16.restype = None
        L.sg_uniform.argtypes = [C.c_uint64, C.c_uint64, C.c_int64, C.c_void_p]
        L.sg_uniform.restype = None
        _SEED_LIB = L
    return _SEED_LIB


def uniform01(seed: int, stream: int, n: int) -> np.ndarray:
    """n doubles in (0, 1] from the splitmix64 stream (seed, stream)."""
    out = np.empty(n, dtype=np.float64)
    _seedlib().sg_uniform(seed, stream, n, out.ctypes.data)
    return out


def normal_bf16(seed: int, stream: int, n: int, std: float) -> np.ndarray:
    """n N(0, std^2) values by Box-Muller, rounded to bf16, as fp32."""
    out = np.empty(n, dtype=np.float32)
    _seedlib().sg_normal_bf16(seed, stream, n, std, out.ctypes.data)
    return out


def round_bf16(a: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bf16 (ties to even), returned widened back to fp32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    r = ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)) << np.uint64(16)
    out = (r & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.float32)
    nan = np.isnan(a)
    if nan.any():
        out = out.copy()
        out[nan] = np.float32("nan")
    return out


def is_bf16_exact(a: np.ndarray) -> bool:
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    return bool(np.all((u & np.uint32(0xFFFF)) == 0))


def stack_sizes(d: Dims) -> dict:
    hd = d.head_dim
    return {
        "wte": d.vocab * d.d_model,
        "c_q": d.n_layer * d.n_head * hd * d.d_model,
        "c_k": d.n_layer * d.n_kv_head * hd * d.d_model,
        "c_v": d.n_layer * d.n_kv_head * hd * d.d_model,
        "c_proj": d.n_layer * d.d_model * d.n_head * hd,
        "c_fc": d.n_layer * d.d_ff * d.d_model,
        "c_proj2": d.n_layer * d.d_model * d.d_ff,
        "lm_head": d.vocab * d.d_model,
    }


def seeded_weights(d: Dims, seed: int, std: float = 0.02) -> dict:
    """The eight stacked fp32 buffers of load_gpt_weights, bf16-exact values."""
    out = {}
    for i, (name, n) in enumerate(stack_sizes(d).items()):
        out[name] = normal_bf16(seed, i + 1, n, std)
    return out


def uniform_ids(seed: int, n: int, vocab: int, stream: int = 101) -> np.ndarray:
    u = uniform01(seed, stream, n)
    return np.minimum((u * vocab).astype(np.int64), vocab - 1).astype(np.int32)


def zipf_ids(seed: int, n: int, vocab: int, s: float = 1.1, stream: int = 202) -> np.ndarray:
    """Ids with P(rank r) proportional to r^-s over ranks 1..vocab, id = rank-1."""
    w = np.arange(1, vocab + 1, dtype=np.float64) ** (-s)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    u = uniform01(seed, stream, n)
    return np.minimum(np.searchsorted(cdf, u, side="left"), vocab - 1).astype(np.int32)


def rope_tables(T: int, hd: int) -> tuple:
    """Host fp32 RoPE tables (T, hd/2) as src/app/chat_text.f90:225-235 builds them."""
    j = np.arange(hd // 2, dtype=np.float32)
    theta = np.power(np.float32(10000.0), (np.float32(-2.0) * j) / np.float32(hd)).astype(np.float32)
    i = np.arange(T, dtype=np.float32)[:, None]
    ang = (i * theta[None, :]).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


# ---------------------------------------------------------------- .npy files

def _npy_header_1d_f4(n: int) -> bytes:
    h = "{'descr': '<f4', 'fortran_order': False, 'shape': (%d,), }" % n
    pad = 64 - (10 + len(h) + 1) % 64
    h = h + " " * pad + "\n"
    return b"\x93NUMPY\x01\x00" + struct.pack("<H", len(h)) + h.encode("latin1")


def write_npy_f4(path: str, a: np.ndarray) -> None:
    a = np.ascontiguousarray(a, dtype="<f4").reshape(-1)
    with open(path, "wb") as f:
        f.write(_npy_header_1d_f4(a.size))
        f.write(a.tobytes())


def layer_file_names(d: Dims) -> list:
    """(stack name, layer or None, file name) in the order the loader reads them."""
    out = [("wte", None, "transformer_wte_weight.npy"), ("lm_head", None, "lm_head_weight.npy")]
    for L in range(d.n_layer):
        p = f"transformer_h_{L}_"
        out += [("c_q", L, p + "attn_c_q_weight.npy"), ("c_k", L, p + "attn_c_k_weight.npy"),
                ("c_v", L, p + "attn_c_v_weight.npy"), ("c_proj", L, p + "attn_c_proj_weight.npy"),
                ("c_fc", L, p + "mlp_c_fc_weight.npy"), ("c_proj2", L, p + "mlp_c_proj_weight.npy")]
    return out


def write_npy_dir(path: str, d: Dims, w: dict, ctx: int = 2048, bos: int = BOS_ID) -> None:
    os.makedirs(path, exist_ok=True)
    sizes = stack_sizes(d)
    for name, L, fname in layer_file_names(d):
        a = w[name]
        if L is None:
            part = a
        else:
            per = sizes[name] // d.n_layer
            part = a[L * per:(L + 1) * per]
        write_npy_f4(os.path.join(path, fname), part)
    with open(os.path.join(path, "arch.txt"), "w") as f:
        f.write(f"d_model = {d.d_model}\nn_head = {d.n_head}\nn_kv = {d.n_kv_head}\n"
                f"n_layer = {d.n_layer}\nvocab = {d.vocab}\nctx = {ctx}\nbos = {bos}\n"
                f"head_dim = {d.head_dim}\n")


# ---------------------------------------------------------------- safetensors
def arch_canonical_of(d_model, n_head, n_kv, head_dim, n_layer, vocab, ctx, bos) -> str:
    """The canonical arch string checkpoints carry as arch.canonical
    (src/lib/fortran_arch.f90:200-210): fixed key order, no spaces."""
    return ('{"schema":"fortran_gpt/arch/1"' + f',"d_model":{d_model},"n_head":{n_head}'
            f',"n_kv":{n_kv},"head_dim":{head_dim},"n_layer":{n_layer},"vocab":{vocab}'
            f',"ctx":{ctx},"bos":{bos}' + "}")


def arch_id_of(s: str) -> str:
    """arch.id: 16 hex digits of a 64-bit rotate-left-17 / xor-shift-29 digest
    of the canonical string's bytes from seed 0x0123456789abcdef
    (src/lib/fortran_arch.f90:217-236)."""
    acc, mask = 0x0123456789ABCDEF, (1 << 64) - 1
    for b in s.encode():
        acc ^= b
        acc = ((acc << 17) | (acc >> 47)) & mask
        acc ^= acc >> 29
    return f"{acc:016x}"


def safetensors_tensors(d: Dims, w: dict) -> dict:
    """Canonical names and 2-D shapes of a checkpoint (load_weights.f90:469-489)."""
    D, qd, kd, ff = d.d_model, d.n_head * d.head_dim, d.n_kv_head * d.head_dim, d.d_ff
    out = {"wte": w["wte"].reshape(d.vocab, D), "lm": w["lm_head"].reshape(d.vocab, D)}
    per = {"q": ("c_q", qd, D), "k": ("c_k", kd, D), "v": ("c_v", kd, D),
           "p": ("c_proj", D, qd), "fc": ("c_fc", ff, D), "p2": ("c_proj2", D, ff)}
    for L in range(d.n_layer):
        for short, (name, r, c) in per.items():
            out[f"l{L}.{short}"] = w[name][L * r * c:(L + 1) * r * c].reshape(r, c)
    return {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in out.items()}


def write_safetensors(path: str, d: Dims, w: dict, ctx: int = 2048, bos: int = BOS_ID,
                      metadata: dict | None = None) -> str:
    """model.safetensors in `path` with the arch.* metadata a trained
    checkpoint carries (fields, arch.canonical, arch.id); `metadata` entries
    override or add keys (None values remove them)."""
    from safetensors.numpy import save_file
    os.makedirs(path, exist_ok=True)
    meta = {"arch.d_model": d.d_model, "arch.n_head": d.n_head, "arch.n_kv": d.n_kv_head,
            "arch.head_dim": d.head_dim, "arch.n_layer": d.n_layer, "arch.vocab": d.vocab,
            "arch.ctx": ctx, "arch.bos": bos}
    canon = arch_canonical_of(d.d_model, d.n_head, d.n_kv_head, d.head_dim, d.n_layer, d.vocab,
                              ctx, bos)
    meta = {k: str(v) for k, v in meta.items()}
    meta["arch.canonical"] = canon
    meta["arch.id"] = arch_id_of(canon)
    for k, v in (metadata or {}).items():
        if v is None:
            meta.pop(k, None)
        else:
            meta[k] = str(v)
    out = os.path.join(path, "model.safetensors")
    save_file(safetensors_tensors(d, w), out, metadata=meta)
    return out
