"""Write the golden vectors of the reference's make_paged_kv (kernels.py:265-286).

make_paged_kv is a seeded generator: its bytes follow from the order of its torch.Generator
calls (randperm for the block table, then randn for K and V, then the per-row INT8
quantisation).  No closed form or invariant fixes that order, so the drop-in restatement in
kernels.py is tied to the reference by the reference's own outputs.  This script imports
the reference module from its source file (on the CPU, in the build container only, since the
reference does not travel to the GPU box) and stores its outputs for a few small cases in
make_paged_kv.npz.  tests/test_golden.py compares the drop-in's outputs with them.

Usage: python tests/golden/make_golden.py [path/to/reference/kernels.py]
"""
from __future__ import annotations

import importlib.util
import os
import sys

sys.dont_write_bytecode = True  # importing the reference must leave no __pycache__ in its tree

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "make_paged_kv.npz")

# (B, ctx_len, H_KV, D, PAGE, seed): ragged, page-aligned and single-token contexts,
# several head counts, head dims and page sizes.
CASES = [
    (3, [37, 16, 50], 2, 16, 16, 5),
    (2, [33, 17], 8, 64, 16, 11),
    (1, [1], 1, 64, 32, 0),
    (4, [64, 3, 48, 20], 2, 32, 16, 123),
]


def load_reference(path: str):
    spec = importlib.util.spec_from_file_location("reference_kernels", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main() -> int:
    path = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/kernels.py"
    ref = load_reference(path)
    arrays = {}
    for i, (B, ctx, H_KV, D, PAGE, seed) in enumerate(CASES):
        kc, vc, ks, vs, bt, cl = ref.make_paged_kv(B, ctx, H_KV, D, PAGE=PAGE, device="cpu", seed=seed)
        arrays[f"c{i}_kc"] = kc.numpy()
        arrays[f"c{i}_vc"] = vc.numpy()
        arrays[f"c{i}_ks_bits"] = ks.numpy().view(np.uint16)   # fp16 scales, stored bit for bit
        arrays[f"c{i}_vs_bits"] = vs.numpy().view(np.uint16)
        arrays[f"c{i}_bt"] = bt.numpy()
        arrays[f"c{i}_cl"] = cl.numpy()
        arrays[f"c{i}_args"] = np.array([B, H_KV, D, PAGE, seed] + list(ctx), dtype=np.int64)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(CASES)} cases)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
