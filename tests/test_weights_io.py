"""fg_weights_read: the checkpoint formats load_gpt_weights accepts
(src/lib/load_weights.f90:830-874), read on the host, no device needed.

Mirrors the reference's own checks: the same model written as .npy files and
as model.safetensors reads back to the same bytes (test_st_ckpt.f90, part 1);
a directory holding only model.safetensors loads (part 3); declared arch.*
metadata that disagrees with the dims, or with itself (arch.canonical,
arch.id), stops the load (load_weights.f90:533-590, :799-821).
"""
import os
import struct

import numpy as np
import pytest

from autoresearch_amd import engine
from autoresearch_amd.weights import (Dims, STACK_NAMES, arch_canonical_of, arch_id_of,
                                      seeded_weights, write_npy_dir, write_safetensors)

SMALL = Dims(n_layer=2, d_model=128, n_head=2, n_kv_head=1, head_dim=64, vocab=512)


@pytest.fixture(scope="module")
def w():
    return seeded_weights(SMALL, 3)


def same(a, b):
    return all(np.array_equal(a[k], b[k]) for k in STACK_NAMES)


def test_npy_and_safetensors_read_back_the_same_bytes(tmp_path, w):
    write_npy_dir(str(tmp_path / "npy"), SMALL, w)
    write_safetensors(str(tmp_path / "st"), SMALL, w)
    a = engine.weights_read(str(tmp_path / "npy"), SMALL)
    b = engine.weights_read(str(tmp_path / "st"), SMALL)
    assert same(a, w) and same(b, w)


def test_safetensors_wins_when_both_are_present(tmp_path, w):
    other = seeded_weights(SMALL, 4)
    write_npy_dir(str(tmp_path), SMALL, other)
    write_safetensors(str(tmp_path), SMALL, w)
    assert same(engine.weights_read(str(tmp_path), SMALL), w)


def test_metadata_may_be_absent(tmp_path, w):
    keys = ["arch.d_model", "arch.n_head", "arch.n_kv", "arch.head_dim", "arch.n_layer",
            "arch.vocab", "arch.ctx", "arch.bos", "arch.canonical", "arch.id"]
    write_safetensors(str(tmp_path), SMALL, w, metadata={k: None for k in keys})
    assert same(engine.weights_read(str(tmp_path), SMALL), w)


@pytest.mark.parametrize("key,val", [("arch.d_model", 256), ("arch.n_kv", 2),
                                     ("arch.n_layer", 3), ("arch.vocab", 1024)])
def test_declared_arch_mismatch_stops(tmp_path, w, key, val):
    write_safetensors(str(tmp_path), SMALL, w, metadata={key: val})
    with pytest.raises(engine.FgptError) as e:
        engine.weights_read(str(tmp_path), SMALL)
    assert e.value.code == -9 and "architecture mismatch" in str(e.value) and key in str(e.value)


def test_non_integer_metadata_stops(tmp_path, w):
    write_safetensors(str(tmp_path), SMALL, w, metadata={"arch.n_head": "two"})
    with pytest.raises(engine.FgptError) as e:
        engine.weights_read(str(tmp_path), SMALL)
    assert e.value.code == -9 and "not an integer" in str(e.value)


def test_inconsistent_canonical_or_id_stops(tmp_path, w):
    write_safetensors(str(tmp_path / "c"), SMALL, w, metadata={"arch.canonical": "{}"})
    with pytest.raises(engine.FgptError) as e:
        engine.weights_read(str(tmp_path / "c"), SMALL)
    assert "arch.canonical" in str(e.value)
    write_safetensors(str(tmp_path / "i"), SMALL, w, metadata={"arch.id": "0" * 16})
    with pytest.raises(engine.FgptError) as e:
        engine.weights_read(str(tmp_path / "i"), SMALL)
    assert "arch.id" in str(e.value)
    # a ctx that differs from the one the canonical string was built with is
    # caught by the cross-check even though ctx is not compared with the dims
    write_safetensors(str(tmp_path / "x"), SMALL, w, metadata={"arch.ctx": 4096})
    with pytest.raises(engine.FgptError):
        engine.weights_read(str(tmp_path / "x"), SMALL)


def test_arch_id_properties():
    """What test_arch_id.f90 asks of the digest: 16 hex digits, deterministic,
    and distinct for distinct configurations (the known ones included)."""
    base = arch_canonical_of(768, 6, 6, 128, 12, 8192, 2048, 8188)
    assert len(arch_id_of(base)) == 16 and int(arch_id_of(base), 16) >= 0
    assert arch_id_of(base) == arch_id_of(base)
    fields = [768, 6, 6, 128, 12, 8192, 2048, 8188]
    ids = {arch_id_of(base)}
    for i in range(8):
        f = list(fields)
        f[i] += 1
        ids.add(arch_id_of(arch_canonical_of(*f)))
    ids.add(arch_id_of(arch_canonical_of(1280, 10, 2, 128, 20, 8192, 2304, 8188)))
    assert len(ids) == 10
    # the empty string leaves the seed untouched
    assert arch_id_of("") == "0123456789abcdef"


def test_arch_id_golden_vectors(tmp_path):
    """arch.canonical and arch.id against the reference's own Python twin of
    fortran_arch (scripts/arch.py:33-63; vectors written by
    tests/golden/make_arch_vectors.py): the host digest in weights.py, and
    the engine's C++ one, which accepts a checkpoint carrying the golden id
    and refuses the same checkpoint with one digit of the id changed."""
    import json
    g = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "arch_id_vectors.json")))
    for v in g["vectors"]:
        assert arch_canonical_of(*v["fields"]) == v["canonical"]
        assert arch_id_of(v["canonical"]) == v["id"]
    v = next(x for x in g["vectors"] if x["fields"][:6] == [128, 2, 1, 64, 2, 512])
    w = seeded_weights(SMALL, 3)
    ctx, bos = v["fields"][6], v["fields"][7]
    write_safetensors(str(tmp_path / "ok"), SMALL, w, ctx=ctx, bos=bos,
                      metadata={"arch.canonical": v["canonical"], "arch.id": v["id"]})
    got = engine.weights_read(str(tmp_path / "ok"), SMALL)
    assert np.array_equal(got["wte"], w["wte"])
    bad = v["id"][:-1] + ("0" if v["id"][-1] != "0" else "1")
    write_safetensors(str(tmp_path / "bad"), SMALL, w, ctx=ctx, bos=bos,
                      metadata={"arch.canonical": v["canonical"], "arch.id": bad})
    with pytest.raises(engine.FgptError, match="arch"):
        engine.weights_read(str(tmp_path / "bad"), SMALL)


def _raw_st(path, header: dict, payload: bytes):
    import json
    h = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + payload)


@pytest.mark.parametrize("case", ["dtype", "shape", "missing", "truncated", "garbage"])
def test_malformed_safetensors_stop(tmp_path, w, case):
    p = str(tmp_path / "model.safetensors")
    if case == "garbage":
        with open(p, "wb") as f:
            f.write(b"\x05\x00\x00\x00\x00\x00\x00\x00{oops")
    else:
        write_safetensors(str(tmp_path), SMALL, w)
        import json
        raw = open(p, "rb").read()
        n = struct.unpack("<Q", raw[:8])[0]
        hdr = json.loads(raw[8:8 + n])
        data = raw[8 + n:]
        if case == "dtype":
            hdr["wte"]["dtype"] = "F16"
        elif case == "shape":
            hdr["l1.fc"]["shape"] = [1, 1]
        elif case == "missing":
            del hdr["l0.v"]
        elif case == "truncated":
            data = data[:len(data) // 2]
        _raw_st(p, hdr, data)
    with pytest.raises(engine.FgptError) as e:
        engine.weights_read(str(tmp_path), SMALL)
    assert e.value.code == -3


@pytest.mark.parametrize("order", ["C", "F"])
def test_rows_npy_either_order(tmp_path, order):
    """eval_bpb's rows file: (N, T+1) int32; numpy writes a Fortran-order
    array with fortran_order True (what the reference's exporter produces)."""
    rows = np.arange(5 * 9, dtype=np.int32).reshape(5, 9) * 7 % 8192
    p = str(tmp_path / "rows.npy")
    np.save(p, np.asfortranarray(rows) if order == "F" else rows)
    assert np.array_equal(engine.rows_npy(p), rows)


def test_rows_npy_rejects_bad_files(tmp_path):
    p = str(tmp_path / "r.npy")
    np.save(p, np.zeros((3, 4), np.int64))
    with pytest.raises(engine.FgptError, match="int32"):
        engine.rows_npy(p)
    np.save(p, np.zeros(5, np.int32))
    with pytest.raises(engine.FgptError, match="2-D"):
        engine.rows_npy(p)
    with pytest.raises(engine.FgptError, match="missing"):
        engine.rows_npy(str(tmp_path / "nope.npy"))
