"""The reader of the persistent decode loop's phase trace (FGPT_FUSED_TRACE)
on a synthetic record: header, stamps per workgroup and layer, and the
per-phase times it derives."""
import numpy as np

from autoresearch_amd import trace


def test_trace_roundtrip(tmp_path):
    nwg, L = 4, 3
    t = np.zeros((nwg, L + 1, 32), np.uint64)
    for w in range(nwg):
        for l in range(L + 1):
            base = 1000 + l * 900 + w  # 9 us a layer
            t[w, l, 0] = base
            for k in range(1, 12):
                t[w, l, k] = base + 50 * k  # 0.5 us per phase
            t[w, l, 14], t[w, l, 15] = base, base + 20
            t[w, l, 24], t[w, l, 25] = 0, 2200 * 550 // 100  # cycles over the layer
    p = tmp_path / "tr.bin"
    with open(p, "wb") as f:
        for _ in range(2):  # two calls appended
            f.write(np.array([nwg, L + 1, 32, 5], np.int32).tobytes())
            f.write(t.tobytes())
    recs = trace.read(str(p))
    assert len(recs) == 2 and recs[1][0] == 0 and recs[1][1].shape == (nwg, L + 1, 32)
    s = trace.summary(recs[-1][1], recs[-1][0])
    assert s["workgroups"] == nwg and s["layers"] == L
    assert abs(s["phases"][" 3 attention done"]["mean_us"] - 1.5) < 1e-9
    assert abs(s["phases"][f"11 {trace.PHASES[11]}"]["max_us"] - 5.5) < 1e-9
    assert abs(s["layer_us_mean"] - 9.0) < 1e-9
    assert abs(s["loader_dma_wait_us"]["mean"] - 0.2) < 1e-9
    assert abs(s["shader_clock_mhz"]["mean"] - 2200) < 1


def test_trace_grouped_kv_kind(tmp_path):
    """The grouped-KV kernel's records carry kind 1 in the header's third
    word; its layer ends at stamp 18."""
    nwg, L = 2, 2
    t = np.zeros((nwg, L + 1, 32), np.uint64)
    for w in range(nwg):
        for l in range(L + 1):
            base = 5000 + l * 2000 + w  # 20 us a layer
            t[w, l, 0] = base
            for k in list(range(1, 14)) + [16, 17, 18]:
                t[w, l, k] = base + 100 * k  # 1 us per stamp index
            t[w, l, 24], t[w, l, 25] = 0, 2400 * 1800 // 100
    p = tmp_path / "tg.bin"
    with open(p, "wb") as f:
        f.write(np.array([nwg, L + 1, 32 | (1 << 16), 5], np.int32).tobytes())
        f.write(t.tobytes())
    (kind, arr), = trace.read(str(p))
    assert kind == 1 and arr.shape == (nwg, L + 1, 32)
    s = trace.summary(arr, kind)
    assert abs(s["phases"][f"18 {trace.PHASES_GQA[18]}"]["mean_us"] - 18.0) < 1e-9
    assert abs(s["phases"][" 7 group gathered"]["max_us"] - 7.0) < 1e-9
    assert abs(s["shader_clock_mhz"]["mean"] - 2400) < 1
