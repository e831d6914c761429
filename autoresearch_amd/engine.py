"""Python host side of the gfx950 engine: ctypes over include/fgpt.h.

Mirrors the reference's model API (14NGiestas/autoresearch):
  gpt_forward     src/lib/fortran_gpt.f90:54-199
  gpt_step        src/lib/fortran_kv.f90:26-149
  gpt_step_multi  src/lib/fortran_kv.f90:160-289
  load_gpt_weights src/lib/load_weights.f90:830-874
with the same argument meaning and the same loud failures (cache full,
missing weights, arch mismatch) raised as exceptions. There is no CPU path:
without libfgpt.so or a gfx950 device every call raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from .weights import Dims, STACK_NAMES

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libfgpt.so")

FG_ERRORS = {
    -1: "FG_EARG", -2: "FG_EDIMS", -3: "FG_EWEIGHT", -4: "FG_EHIP", -5: "FG_EFULL",
    -6: "FG_EROPE", -7: "FG_ENODEV", -8: "FG_EBUSY", -9: "FG_EARCH", -10: "FG_ERANGE",
}

# every symbol include/fgpt.h declares
EXPORTS = (
    "fg_version", "fg_last_error", "fg_model_create", "fg_weights_read", "fg_model_load",
    "fg_model_destroy",
    "fg_set_rope", "fg_forward", "fg_forward_pos", "fg_forward_dev", "fg_kv_create", "fg_kv_create_ex", "fg_kv_destroy",
    "fg_kv_len", "fg_kv_set_len", "fg_kv_read", "fg_step", "fg_step_multi",
    "fg_decode_greedy", "fg_sync", "fg_model_bytes", "fg_timing", "fg_timing_read",
    "fg_eval_bpb", "fg_rows_npy", "fg_decode_spec", "fg_spec_accept", "fg_spec_draft",
    "fg_sample", "fg_decode_sample", "fg_set_option", "fg_get_option", "fg_step_dev_noalloc",
)

KERNEL_KINDS = {0: "gemm", 1: "gemv", 2: "attn_chunk", 3: "attn_decode", 4: "other",
                5: "decode_fused"}
FG_OPT_FUSED_DECODE = 1
FG_OPT_FORWARD_F16 = 2


FG_KV_BF16 = 1  # fg_kv_create_ex flag: bf16 K/V cache


class FgptError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{FG_ERRORS.get(code, code)}: {msg}")
        self.code = code


class CacheFull(FgptError):
    pass


class _FgDims(C.Structure):
    _fields_ = [("n_layer", C.c_int32), ("d_model", C.c_int32), ("n_head", C.c_int32),
                ("n_kv_head", C.c_int32), ("head_dim", C.c_int32), ("vocab_size", C.c_int32),
                ("eps", C.c_float)]


class _SpecCfg(C.Structure):
    _fields_ = [("k", C.c_int32), ("match", C.c_int32), ("probe", C.c_int32),
                ("min_acc", C.c_float)]


class _SpecStats(C.Structure):
    _fields_ = [("passes", C.c_int64), ("accepted", C.c_int64), ("proposed", C.c_int64),
                ("plain", C.c_int64), ("pauses", C.c_int64)]


class _SampleCfg(C.Structure):
    _fields_ = [("temp", C.c_float), ("topp", C.c_float), ("pres", C.c_float),
                ("freq", C.c_float), ("rep", C.c_float), ("plen", C.c_float),
                ("pwin", C.c_int32), ("nblock", C.c_int32), ("byte_space", C.c_int32)]


def sample_cfg(temp=0.0, topp=1.0, pres=0.0, freq=0.0, rep=1.0, plen=0.0, pwin=0, nblock=0,
               byte_space=False) -> _SampleCfg:
    """chat_text's sampling options (defaults as its command line has them)."""
    return _SampleCfg(temp, topp, pres, freq, rep, plen, pwin, nblock, 1 if byte_space else 0)


_f = C.POINTER(C.c_float)
_i = C.POINTER(C.c_int32)
_vp = C.c_void_p
_LIB = None


def load_library(path: str = LIB_PATH):
    """Load libfgpt.so (fails loudly when it has not been built)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is missing: build it with autoresearch_amd/build.py")
    L = C.CDLL(path)
    i32, i64 = C.c_int32, C.c_int64
    sig = {
        "fg_version": (i32, []),
        "fg_last_error": (i32, [C.c_char_p, i32]),
        "fg_model_create": (i32, [C.POINTER(_FgDims)] + [_f] * 8 + [C.POINTER(_vp)]),
        "fg_weights_read": (i32, [C.POINTER(_FgDims), C.c_char_p] + [_f] * 8),
        "fg_model_load": (i32, [C.POINTER(_FgDims), C.c_char_p, C.POINTER(_vp)]),
        "fg_model_destroy": (i32, [_vp]),
        "fg_set_rope": (i32, [_vp, i32, i32, _f, _f]),
        "fg_forward": (i32, [_vp, _i, i32, i32, _f, _i, _f]),
        "fg_forward_pos": (i32, [_vp, _i, i32, i32, _f, _i, _f, _i]),
        "fg_forward_dev": (i32, [_vp, _vp, i32, i32, _vp, _vp, _vp, _vp]),
        "fg_kv_create": (i32, [_vp, i32, i32, C.POINTER(_vp)]),
        "fg_kv_create_ex": (i32, [_vp, i32, i32, i32, C.POINTER(_vp)]),
        "fg_kv_destroy": (i32, [_vp]),
        "fg_kv_len": (i32, [_vp, _i]),
        "fg_kv_set_len": (i32, [_vp, i32]),
        "fg_kv_read": (i32, [_vp, _f, _f]),
        "fg_step": (i32, [_vp, _vp, _i, _f, _i]),
        "fg_step_multi": (i32, [_vp, _vp, _i, i32, _f, _i]),
        "fg_decode_greedy": (i32, [_vp, _vp, _i, i32, _i, _f]),
        "fg_sync": (i32, [_vp]),
        "fg_model_bytes": (i32, [_vp, C.POINTER(i64), C.POINTER(i64)]),
        "fg_timing": (i32, [_vp, i32]),
        "fg_eval_bpb": (i32, [_vp, _i, i32, i32, i32, _i, i32, _f, C.POINTER(C.c_double),
                              C.POINTER(i64), C.POINTER(C.c_double), C.POINTER(i64)]),
        "fg_rows_npy": (i32, [C.c_char_p, _i, _i, _i]),
        "fg_decode_spec": (i32, [_vp, _vp, _i, i32, i32, C.POINTER(_SpecCfg),
                                 C.POINTER(_SpecStats)]),
        "fg_spec_accept": (i32, [_i, _i, i32, _i, _i]),
        "fg_spec_draft": (i32, [_i, i32, i32, i32, _i, _i]),
        "fg_sample": (i32, [_vp, _f, i32, _i, i32, C.POINTER(_SampleCfg), C.POINTER(i64), _i]),
        "fg_decode_sample": (i32, [_vp, _vp, _i, i32, i32, C.POINTER(_SampleCfg),
                                   C.POINTER(i64)]),
        "fg_set_option": (i32, [_vp, i32, i32]),
        "fg_step_dev_noalloc": (i32, [_vp, _vp, _vp, _vp, _vp, _vp]),
        "fg_get_option": (i32, [_vp, i32, _i, C.c_char_p, i32]),
        "fg_timing_read": (i32, [_vp, i32, C.POINTER(i64), C.POINTER(C.c_double),
                                 C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = L
    return L


def _check(rc: int):
    if rc != 0:
        buf = C.create_string_buffer(512)
        _LIB.fg_last_error(buf, 512)
        msg = buf.value.decode(errors="replace")
        raise (CacheFull if rc == -5 else FgptError)(rc, msg)


def _fp(a):
    return None if a is None else a.ctypes.data_as(_f)


def _ip(a):
    return None if a is None else a.ctypes.data_as(_i)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def _cdims(d: Dims) -> _FgDims:
    return _FgDims(d.n_layer, d.d_model, d.n_head, d.n_kv_head, d.head_dim, d.vocab, d.eps)


class Model:
    """One resident model: bf16 weight arena, workspace and RoPE tables in HBM."""

    def __init__(self, d: Dims, stacks: dict | None = None, weights_dir: str | None = None):
        L = load_library()
        self.d = d
        self._h = _vp()
        cd = _cdims(d)
        if weights_dir is not None:
            _check(L.fg_model_load(C.byref(cd), weights_dir.encode(), C.byref(self._h)))
        else:
            bufs = [_f32(stacks[n]) for n in STACK_NAMES]
            _check(L.fg_model_create(C.byref(cd), *[_fp(b) for b in bufs], C.byref(self._h)))

    def close(self):
        if self._h:
            _LIB.fg_model_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    def set_rope(self, cos_buf, sin_buf, pos0: int = 0):
        c, s = _f32(cos_buf).reshape(-1), _f32(sin_buf).reshape(-1)
        n = c.size // (self.d.head_dim // 2)
        _check(_LIB.fg_set_rope(self._h, pos0, n, _fp(c), _fp(s)))

    def forward(self, ids, B: int, T: int, targets=None, want_logits: bool = True):
        ids = _i32(ids).reshape(-1)
        if ids.size != B * T:
            raise ValueError("ids must hold B*T values")
        lg = np.empty(B * T * self.d.vocab, np.float32) if want_logits else None
        tg = _i32(targets).reshape(-1) if targets is not None else None
        nll = np.empty(B * T, np.float32) if tg is not None else None
        _check(_LIB.fg_forward(self._h, _ip(ids), B, T, _fp(lg), _ip(tg), _fp(nll)))
        lg = lg.reshape(B, T, self.d.vocab) if lg is not None else None
        return lg, (nll.reshape(B, T) if nll is not None else None)

    def forward_pos(self, ids, B: int, T: int, want_logits: bool = True):
        """fg_forward_pos: the forward's logits and attn_sgemm's positive-score
        counts per layer, row and head ([L, B, H] int32)."""
        ids = _i32(ids).reshape(-1)
        if ids.size != B * T:
            raise ValueError("ids must hold B*T values")
        lg = np.empty(B * T * self.d.vocab, np.float32) if want_logits else None
        npos = np.zeros(self.d.n_layer * B * self.d.n_head, np.int32)
        _check(_LIB.fg_forward_pos(self._h, _ip(ids), B, T, _fp(lg), None, None, _ip(npos)))
        lg = lg.reshape(B, T, self.d.vocab) if lg is not None else None
        return lg, npos.reshape(self.d.n_layer, B, self.d.n_head)

    @staticmethod
    def pos_frac_accumulate(npos, T: int, pos_frac=None, pos_n=None):
        """The reference's accumulation of the counts into pos_frac / pos_n
        (src/lib/fortran_attn.f90:291-296): per (layer, row) in that order,
        pos_frac[h] += npos / (T(T+1)/2) in fp32, pos_n[h] += 1."""
        L, B, H = npos.shape
        pf = np.zeros(H, np.float32) if pos_frac is None else pos_frac
        pn = np.zeros(H, np.int32) if pos_n is None else pos_n
        den = np.float32(T * (T + 1) // 2)
        for ll in range(L):
            for aa in range(B):
                for bb in range(H):
                    pf[bb] = np.float32(pf[bb] + np.float32(npos[ll, aa, bb]) / den)
                    pn[bb] += 1
        return pf, pn

    def forward_dev(self, d_ids: int, B: int, T: int, d_logits: int = 0, d_targets: int = 0,
                    d_nll: int = 0, stream: int = 0):
        """Enqueue a forward on device pointers (ints), no host synchronisation."""
        _check(_LIB.fg_forward_dev(self._h, d_ids, B, T, d_logits or None, d_targets or None,
                                   d_nll or None, stream or None))

    def sync(self):
        _check(_LIB.fg_sync(self._h))

    def bytes(self):
        w, k = C.c_int64(), C.c_int64()
        _check(_LIB.fg_model_bytes(self._h, C.byref(w), C.byref(k)))
        return w.value, k.value

    def timing(self, enable: bool):
        _check(_LIB.fg_timing(self._h, 1 if enable else 0))

    def set_fused_decode(self, enable: bool):
        """FG_OPT_FUSED_DECODE: the persistent B=1 greedy loop (1) or the
        captured per-kernel steps (0)."""
        _check(_LIB.fg_set_option(self._h, FG_OPT_FUSED_DECODE, 1 if enable else 0))

    def fused_decode(self):
        """(active, reason when not): whether fg_decode_greedy runs B=1
        loops as one persistent launch."""
        v = C.c_int32()
        buf = C.create_string_buffer(256)
        _check(_LIB.fg_get_option(self._h, FG_OPT_FUSED_DECODE, C.byref(v), buf, 256))
        return bool(v.value), buf.value.decode(errors="replace")

    def set_forward_f16(self, enable: bool):
        """FG_OPT_FORWARD_F16: forward / eval passes of more than 128 token
        rows as single-term fp16 MFMA work (1) or in the split bf16 format
        (0, the default). Enabling it makes the fp16 weight copy."""
        _check(_LIB.fg_set_option(self._h, FG_OPT_FORWARD_F16, 1 if enable else 0))

    def forward_f16(self) -> bool:
        v = C.c_int32()
        _check(_LIB.fg_get_option(self._h, FG_OPT_FORWARD_F16, C.byref(v), None, 0))
        return bool(v.value)

    def eval_bpb(self, rows, token_bytes, batch: int = 8, want_nll: bool = False) -> dict:
        """fg_eval_bpb over rows (N, T+1): per-row and total byte-weighted nats
        and bytes, bpb = nats / bytes / ln 2 (and the per-position NLL)."""
        rows = _i32(rows)
        n, w = rows.shape
        T = w - 1
        tb = _i32(token_bytes)
        nll = np.empty(n * T, np.float32) if want_nll else None
        rn = np.empty(n, np.float64)
        rb = np.empty(n, np.int64)
        tn, tbt = C.c_double(), C.c_int64()
        _check(_LIB.fg_eval_bpb(self._h, _ip(rows), n, T, batch, _ip(tb), tb.size, _fp(nll),
                                rn.ctypes.data_as(C.POINTER(C.c_double)),
                                rb.ctypes.data_as(C.POINTER(C.c_int64)), C.byref(tn),
                                C.byref(tbt)))
        out = {"row_nats": rn, "row_bytes": rb, "nats": tn.value, "bytes": tbt.value,
               "bpb": tn.value / tbt.value / np.log(2) if tbt.value else float("nan")}
        if want_nll:
            out["nll"] = nll.reshape(n, T)
        return out

    def timing_read(self) -> dict:
        """{kind: (launches, ms, flops, bytes)} of the launches recorded so far."""
        out = {}
        for k, name in KERNEL_KINDS.items():
            n, ms, fl, by = C.c_int64(), C.c_double(), C.c_double(), C.c_double()
            _check(_LIB.fg_timing_read(self._h, k, C.byref(n), C.byref(ms), C.byref(fl), C.byref(by)))
            out[name] = (n.value, ms.value, fl.value, by.value)
        return out

    def sample(self, logits, gen=(), state: int = 12345, **cfg):
        """fg_sample (sample_next) on one row of logits: (id, new state)."""
        lg = _f32(logits).reshape(-1)
        g = _i32(np.asarray(gen, dtype=np.int32)).reshape(-1)
        st = C.c_int64(state)
        out = C.c_int32()
        c = sample_cfg(**cfg)
        _check(_LIB.fg_sample(self._h, _fp(lg), lg.size, _ip(g) if g.size else None, g.size,
                              C.byref(c), C.byref(st), C.byref(out)))
        return out.value, st.value

    def kv(self, B: int, maxT: int, bf16: bool = False) -> "KV":
        return KV(self, B, maxT, bf16)


class KV:
    """A KV cache of B sequences x maxT positions resident in HBM."""

    def __init__(self, m: Model, B: int, maxT: int, bf16: bool = False):
        """bf16: K and V held as bf16 (FG_KV_BF16), half the cache bytes."""
        self.m, self.B, self.maxT, self.bf16 = m, B, maxT, bf16
        self._h = _vp()
        _check(_LIB.fg_kv_create_ex(m.handle, B, maxT, FG_KV_BF16 if bf16 else 0,
                                    C.byref(self._h)))

    def close(self):
        if self._h:
            _LIB.fg_kv_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def len(self) -> int:
        v = C.c_int32()
        _check(_LIB.fg_kv_len(self._h, C.byref(v)))
        return v.value

    @len.setter
    def len(self, v: int):
        _check(_LIB.fg_kv_set_len(self._h, v))

    def read(self):
        d = self.m.d
        n = d.n_layer * self.B * self.maxT * d.n_kv_head * d.head_dim
        k, v = np.empty(n, np.float32), np.empty(n, np.float32)
        _check(_LIB.fg_kv_read(self._h, _fp(k), _fp(v)))
        return k, v

    def step(self, ids, want_logits: bool = True):
        ids = _i32(ids).reshape(-1)
        lg = np.empty(self.B * self.m.d.vocab, np.float32) if want_logits else None
        nxt = np.empty(self.B, np.int32)
        _check(_LIB.fg_step(self.m.handle, self._h, _ip(ids), _fp(lg), _ip(nxt)))
        return (lg.reshape(self.B, -1) if lg is not None else None), nxt

    def step_dev_noalloc(self, d_ids: int, d_logits: int, d_next: int = 0, stream: int = 0):
        """fg_step_dev_noalloc on device pointers (ints): one cached step whose
        scratch is the library's own device array (no allocation)."""
        _check(_LIB.fg_step_dev_noalloc(self.m.handle, self._h, d_ids, d_logits, d_next or None,
                                        stream or None))

    def step_multi(self, ids, want_logits: bool = True):
        ids = _i32(ids).reshape(self.B, -1)
        TB = ids.shape[1]
        lg = np.empty(self.B * TB * self.m.d.vocab, np.float32) if want_logits else None
        nxt = np.empty(self.B, np.int32)
        _check(_LIB.fg_step_multi(self.m.handle, self._h, _ip(ids), TB, _fp(lg), _ip(nxt)))
        return (lg.reshape(self.B, TB, -1) if lg is not None else None), nxt

    def decode_greedy(self, ids, n_steps: int, want_logits: bool = False):
        ids = _i32(ids).reshape(-1)
        out = np.empty(n_steps * self.B, np.int32)
        lg = np.empty(n_steps * self.B * self.m.d.vocab, np.float32) if want_logits else None
        _check(_LIB.fg_decode_greedy(self.m.handle, self._h, _ip(ids), n_steps, _ip(out), _fp(lg)))
        out = out.reshape(n_steps, self.B)
        return out, (lg.reshape(n_steps, self.B, -1) if lg is not None else None)


    def decode_spec(self, prompt, n_gen: int, k: int = 8, match: int = 2, probe: int = 8,
                    min_acc: float = 0.5):
        """fg_decode_spec: greedy speculative continuation of `prompt`, whose
        first len-1 ids must already be cached (B = 1). Returns the n_gen
        generated ids and the loop's counters."""
        prompt = _i32(prompt).reshape(-1)
        ids = np.zeros(prompt.size + n_gen, np.int32)
        ids[:prompt.size] = prompt
        cfg = _SpecCfg(k, match, probe, min_acc)
        st = _SpecStats()
        _check(_LIB.fg_decode_spec(self.m.handle, self._h, _ip(ids), prompt.size, ids.size,
                                   C.byref(cfg), C.byref(st)))
        stats = {f: getattr(st, f) for f, _ in _SpecStats._fields_}
        return ids[prompt.size:], stats

    def decode_sample(self, prompt, n_gen: int, seed: int = 12345, **cfg):
        """fg_decode_sample: chat_text's plain loop with sample_next after
        `prompt` (its first len-1 ids already cached, B = 1). Returns the
        n_gen ids and the generator state after them."""
        return _decode_sample(self, prompt, n_gen, seed, cfg)


def _decode_sample(kv, prompt, n_gen, seed, cfg):
    prompt = _i32(prompt).reshape(-1)
    ids = np.zeros(prompt.size + n_gen, np.int32)
    ids[:prompt.size] = prompt
    st = C.c_int64(seed)
    c = sample_cfg(**cfg)
    _check(_LIB.fg_decode_sample(kv.m.handle, kv._h, _ip(ids), prompt.size, ids.size,
                                 C.byref(c), C.byref(st)))
    return ids[prompt.size:], st.value


def spec_accept(draft, targmax):
    """fg_spec_accept (accept_prefix): (n_accept, correction)."""
    load_library()
    d, t = _i32(draft).reshape(-1), _i32(targmax).reshape(-1)
    if t.size < d.size + 1:
        raise ValueError("targmax needs k+1 ids")
    na, corr = C.c_int32(), C.c_int32()
    _check(_LIB.fg_spec_accept(_ip(d) if d.size else None, _ip(t), d.size, C.byref(na),
                               C.byref(corr)))
    return na.value, corr.value


def spec_draft(ids, p: int, m: int, k: int):
    """fg_spec_draft (lookup_draft) over ids[0:p]: the proposed ids."""
    load_library()
    ids = _i32(ids).reshape(-1)
    if p > ids.size:
        raise ValueError("p exceeds the ids given")
    d = np.zeros(max(k, 1), np.int32)
    n = C.c_int32()
    _check(_LIB.fg_spec_draft(_ip(ids) if ids.size else None, p, m, k, _ip(d), C.byref(n)))
    return d[:n.value].tolist()


# ------------------------------------------------------- reference-shaped API

def rows_npy(path: str) -> np.ndarray:
    """fg_rows_npy: eval_bpb's (N, T+1) int32 rows file, C or Fortran order."""
    load_library()
    n, w = C.c_int32(), C.c_int32()
    _check(_LIB.fg_rows_npy(path.encode(), C.byref(n), C.byref(w), None))
    out = np.empty((n.value, w.value), np.int32)
    _check(_LIB.fg_rows_npy(path.encode(), C.byref(n), C.byref(w), _ip(out)))
    return out


def weights_read(wdir: str, d: Dims) -> dict:
    """fg_weights_read: the eight fp32 stacks of a checkpoint directory
    (model.safetensors when present, else the .npy files), host only."""
    load_library()
    D, qd, kd, ff, V, L = d.d_model, d.n_head * d.head_dim, d.n_kv_head * d.head_dim, \
        d.d_ff, d.vocab, d.n_layer
    out = {"wte": np.empty(V * D, np.float32), "c_q": np.empty(L * qd * D, np.float32),
           "c_k": np.empty(L * kd * D, np.float32), "c_v": np.empty(L * kd * D, np.float32),
           "c_proj": np.empty(L * D * qd, np.float32), "c_fc": np.empty(L * ff * D, np.float32),
           "c_proj2": np.empty(L * D * ff, np.float32), "lm_head": np.empty(V * D, np.float32)}
    dims = _cdims(d)
    _check(_LIB.fg_weights_read(C.byref(dims), wdir.encode(), *[_fp(out[k]) for k in STACK_NAMES]))
    return out


def load_gpt_weights(wdir: str, d: Dims) -> Model:
    """load_gpt_weights + require_arch (src/lib/load_weights.f90:830-874,
    src/lib/fortran_arch.f90:238-246), uploading straight to HBM."""
    return Model(d, weights_dir=wdir)


def greedy_generate(m: Model, prompt, n_gen: int, cos_buf, sin_buf, pchunk: int = 64):
    """The ids-in/ids-out loop of src/app/chat_text.f90:257-278,423-462 with
    plain argmax: prompt[:-1] through chunked cached passes (gpt_step_multi,
    pchunk tokens each), then n_gen device-side greedy steps fed from
    prompt[-1]. Returns the generated ids."""
    prompt = _i32(prompt).reshape(-1)
    ntot = prompt.size + n_gen
    m.set_rope(np.asarray(cos_buf).reshape(-1)[: ntot * m.d.head_dim // 2],
               np.asarray(sin_buf).reshape(-1)[: ntot * m.d.head_dim // 2])
    kv = m.kv(1, ntot)
    npre = prompt.size - 1
    s = 0
    while s < npre:
        tb = min(pchunk, npre - s)
        kv.step_multi(prompt[s:s + tb], want_logits=False)
        s += tb
    out, _ = kv.decode_greedy(prompt[-1:], n_gen)
    kv.close()
    return out[:, 0]
