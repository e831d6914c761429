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
    assert len(recs) == 2 and recs[1].shape == (nwg, L + 1, 32)
    s = trace.summary(recs[-1])
    assert s["workgroups"] == nwg and s["layers"] == L
    assert abs(s["phases"][" 3 attention done"]["mean_us"] - 1.5) < 1e-9
    assert abs(s["phases"][f"11 {trace.PHASES[11]}"]["max_us"] - 5.5) < 1e-9
    assert abs(s["layer_us_mean"] - 9.0) < 1e-9
    assert abs(s["loader_dma_wait_us"]["mean"] - 0.2) < 1e-9
    assert abs(s["shader_clock_mhz"]["mean"] - 2200) < 1
