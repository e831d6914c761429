"""Phase timings of the persistent B=1 decode loop (kern_fused.hip).

With FGPT_FUSED_TRACE=<file> set, fg_decode_greedy's persistent launch
appends one record per call to <file>: a header of four int32 (workgroups,
pseudo-layers L+1, slots per layer 32 with the kernel's kind in bits 16 and
up, steps) and then, for one step (the second of the call when it has two or
more), per workgroup and layer, 32 uint64 device-clock stamps (100 MHz,
s_memrealtime; 0 = not taken). Stamp k of a layer marks, for the kernel with
one KV head per query head (kern_fused.hip, kind 0):

    0  layer start (after the barrier that opens the layer)
    1  the workgroup's q/k/v values published (head XCDs)
    2  the head's q/k/v gathered (barrier B1)
    3  attention done (barrier B2)
    4  c_proj partials published
    5  residual columns published after summing the heads' partials
    6  the residual gathered (barrier B3)
    7  relu2(fc) rows published
    8  the hidden block gathered (barrier B4)
    9  c_proj2 partials published
   10  residual columns published after summing the blocks' partials
   11  the residual gathered: layer end
   14, 15  the loader wave's wait for its weight DMA (before / after)
   24, 25  shader clock counter at layer start / end (clock estimate)

and for the grouped-KV kernel (kern_fused_gqa.hip, kind 1):

    0  layer start            1  q/k/v pairs published
    2  the group's q/k/v gathered (B1)       3  attention records (B2)
    4  the workgroup's partial published    5  the XCD's partials gathered (B3)
    6  the XCD's merged partial published   7  the group's partials gathered (B4)
    8  attention output in LDS (B4b)        9  c_proj partials published
   10  residual columns published          11  the residual gathered (B5)
   12  relu2(fc) rows published            13  the hidden block gathered (B6)
   16  c_proj2 partials published          17  residual columns published
   18  the residual gathered: layer end

For the lm_head pseudo-layer: 1 logits + candidates, 2 the argmax exchanged,
3 barrier B6 (kind 0; kind 1: 0 rows landed, 1 logits + candidates, 2 the
argmax exchanged, 3 the barrier after it).

    python -m autoresearch_amd.trace FILE [--json]
"""
from __future__ import annotations

import json
import sys

import numpy as np

PHASES = {1: "qkv published", 2: "qkv gathered", 3: "attention done", 4: "c_proj published",
          5: "residual published", 6: "residual gathered", 7: "fc published",
          8: "hidden gathered", 9: "c_proj2 published", 10: "residual published",
          11: "residual gathered (end)"}
PHASES_GQA = {1: "qkv published", 2: "qkv gathered", 3: "attention records", 4: "wg partial published",
              5: "xcd partials gathered", 6: "xcd partial published", 7: "group gathered",
              8: "attention output", 9: "c_proj published", 10: "residual published",
              11: "residual gathered", 12: "fc published", 13: "hidden gathered",
              16: "c_proj2 published", 17: "residual published", 18: "residual gathered (end)"}
TICK_US = 0.01  # 100 MHz


def read(path: str) -> list:
    """Every record of the file: (kind, array [workgroups, L+1, 32] of int64
    stamps)."""
    raw = open(path, "rb").read()
    off, out = 0, []
    while off + 16 <= len(raw):
        nwg, nl, nk, ns = (int(v) for v in np.frombuffer(raw[off:off + 16], np.int32))
        kind, nk = nk >> 16, nk & 0xFFFF
        off += 16
        n = nwg * nl * nk
        out.append((kind, np.frombuffer(raw[off:off + 8 * n], np.uint64).reshape(nwg, nl, nk)
                    .astype(np.int64)))
        off += 8 * n
    return out


def summary(t: np.ndarray, kind: int = 0) -> dict:
    """Per-phase times (us, relative to each workgroup's layer start; mean
    and max over workgroups and layers 1..L-2), layer durations, lm_head
    phases, the loader's DMA waits and the shader clock estimate."""
    L = t.shape[1] - 1
    layers = range(1, L - 1) if L > 2 else range(L)
    start = t[:, :, 0]
    out = {"workgroups": int(t.shape[0]), "layers": L, "phases": {}}
    end = 18 if kind == 1 else 11
    for k, name in (PHASES_GQA if kind == 1 else PHASES).items():
        rel = []
        for l in layers:
            v = t[:, l, k]
            ok = v > 0
            rel.append((v[ok] - start[ok, l]) * TICK_US)
        r = np.concatenate(rel) if rel else np.zeros(0)
        if r.size:
            out["phases"][f"{k:2d} {name}"] = {"mean_us": float(r.mean()), "max_us": float(r.max()),
                                              "n": int(r.size)}
    t0 = start[:, 0][start[:, 0] > 0].min()
    ls = [float((start[:, l].max() - t0) * TICK_US) for l in range(L + 1)]
    out["layer_start_us"] = ls
    out["layer_us_mean"] = float(np.diff(ls[:L]).mean()) if L > 1 else None
    lm = {}
    for k in (1, 2, 3):
        v = t[:, L, k]
        ok = v > 0
        if ok.any():
            lm[k] = float(((v[ok] - start[ok, L]) * TICK_US).mean())
    out["lm_head_us"] = lm
    lw = (t[:, :L, 15] - t[:, :L, 14]) * TICK_US
    out["loader_dma_wait_us"] = {"mean": float(lw.mean()), "max": float(lw.max())}
    dr = (t[:, :L, end] - t[:, :L, 0]).astype(np.float64)
    dm = (t[:, :L, 25] - t[:, :L, 24]).astype(np.float64)
    ok = (dr > 0) & (dm > 0)
    if ok.any():
        mhz = dm[ok] / dr[ok] * 100.0
        out["shader_clock_mhz"] = {"mean": float(mhz.mean()), "min": float(mhz.min()),
                                   "max": float(mhz.max())}
    return out


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    if not argv:
        print(__doc__)
        return 2
    recs = read(argv[0])
    if not recs:
        print("no records")
        return 1
    s = summary(recs[-1][1], recs[-1][0])
    if "--json" in argv:
        print(json.dumps(s))
        return 0
    print(f"{s['workgroups']} workgroups, {s['layers']} layers; layer time {s['layer_us_mean']:.2f} us")
    for name, v in s["phases"].items():
        print(f"  {name:28s} mean {v['mean_us']:6.2f} us  max {v['max_us']:6.2f} us")
    print("  lm_head pseudo-layer:", {k: round(v, 2) for k, v in s["lm_head_us"].items()})
    print("  loader DMA wait:", {k: round(v, 2) for k, v in s["loader_dma_wait_us"].items()})
    if "shader_clock_mhz" in s:
        print("  shader clock (MHz):", {k: round(v) for k, v in s["shader_clock_mhz"].items()})
    return 0


if __name__ == "__main__":
    sys.exit(main())
