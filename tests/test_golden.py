"""The drop-in's make_paged_kv against the reference's own outputs (tests/golden/make_paged_kv.npz).

The fixture was written by tests/golden/make_golden.py from the reference's make_paged_kv
(kernels.py:265-286) on the CPU.  Equal bytes mean the drop-in makes the same generator calls
in the same order and quantises K/V the same way, so a seed gives both the same cache.
"""
import os

import numpy as np
import pytest

import kernels as K
from oracle import oracle as O

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "make_paged_kv.npz")


@pytest.mark.parametrize("case", range(4))
def test_make_paged_kv_matches_reference_bytes(case):
    z = np.load(FIXTURE)
    args = z[f"c{case}_args"].tolist()
    B, H_KV, D, PAGE, seed = args[:5]
    ctx = args[5:]
    kc, vc, ks, vs, bt, cl = (t.numpy() for t in K.make_paged_kv(B, ctx, H_KV, D, PAGE=PAGE, device="cpu", seed=seed))
    assert np.array_equal(bt, z[f"c{case}_bt"]) and np.array_equal(cl, z[f"c{case}_cl"])
    assert np.array_equal(kc, z[f"c{case}_kc"]) and np.array_equal(vc, z[f"c{case}_vc"])
    assert np.array_equal(ks.view(np.uint16), z[f"c{case}_ks_bits"])
    assert np.array_equal(vs.view(np.uint16), z[f"c{case}_vs_bits"])


def test_golden_cache_quantisation_follows_the_oracle():
    # Each (page, slot, head) row of the reference's cache is an INT8 row with scale
    # max(amax, 1e-8) / 127: re-quantising the dequantised row reproduces it.
    z = np.load(FIXTURE)
    kc, ks = z["c1_kc"], z["c1_ks_bits"].view(np.float16)
    assert np.abs(kc).max(axis=-1).min() == 127          # every row reaches the full range
    deq = kc.astype(np.float32) * ks.astype(np.float32)[..., None]
    q, _ = O.quantize_rows_int8(deq)
    assert np.array_equal(q, kc)
