#!/usr/bin/env python3
"""Write arch_id_vectors.json: canonical strings and arch.id digests from the
reference's own Python twin of fortran_arch (scripts/arch.py:33-63), for a
set of architectures (the depth-12 and depth-20 GQA models, the test dims,
and values that reach every digit count). Run in the build container, where
the reference is at /root/reference; the vectors are committed and the tests
read only them.

    python tests/golden/make_arch_vectors.py
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REF_SCRIPTS = "/root/reference/scripts"

ARCHS = [
    # d_model, n_head, n_kv, head_dim, n_layer, vocab, ctx, bos
    (768, 6, 6, 128, 12, 8192, 2048, 8188),
    (1280, 10, 2, 128, 20, 8192, 2048, 8188),
    (128, 2, 1, 64, 2, 512, 64, 8188),
    (256, 2, 2, 128, 2, 1024, 160, 8188),
    (96, 6, 2, 16, 12, 8192, 1024, 8188),
    (1, 1, 1, 1, 1, 1, 1, 0),
    (4096, 32, 8, 128, 48, 131072, 131072, 131071),
]


def main():
    sys.path.insert(0, REF_SCRIPTS)
    import arch  # the reference's module, imported only here
    out = []
    for a in ARCHS:
        canon = arch.canonical_of(*a)
        out.append({"fields": list(a), "canonical": canon, "id": arch.arch_id_of(canon)})
    with open(os.path.join(HERE, "arch_id_vectors.json"), "w") as f:
        json.dump({"source": "scripts/arch.py:33-63 (canonical_of, arch_id_of)",
                   "vectors": out}, f, indent=1)
    print(f"wrote {len(out)} vectors")


if __name__ == "__main__":
    main()
