"""CPU checks of the C ABI: the library loads, exports exactly what
include/fgpt.h declares, and fails loudly (no CPU fallback) without a GPU."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

from autoresearch_amd import engine
from autoresearch_amd.weights import Dims, seeded_weights

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fgpt.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(fg_[a-z_]+)\s*\(", text)))


def test_header_matches_wrapper_list():
    assert declared() == sorted(engine.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = engine.load_library()
    for name in declared():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", engine.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = sorted(set(re.findall(r" T (fg_[a-z_]+)$", out, re.M)))
    assert exported == declared()


def test_version_and_error_buffer():
    lib = engine.load_library()
    assert lib.fg_version() == 101
    buf = C.create_string_buffer(8)
    lib.fg_last_error(buf, 8)


def test_no_device_fails_loudly():
    """Without a visible gfx950 the product path raises; nothing runs on the CPU."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    d = Dims(n_layer=1, d_model=128, n_head=2, n_kv_head=1, head_dim=64, vocab=256)
    w = seeded_weights(d, 3)
    with pytest.raises(engine.FgptError) as e:
        engine.Model(d, stacks=w)
    assert e.value.code in (-7, -4)


def test_bad_dims_rejected_before_device():
    d = Dims(n_layer=1, d_model=96, n_head=3, n_kv_head=1, head_dim=32, vocab=256)
    w = seeded_weights(d, 3)
    with pytest.raises(engine.FgptError) as e:
        engine.Model(d, stacks=w)
    assert e.value.code == -2
