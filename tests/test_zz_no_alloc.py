"""The allocation-free W8A8 entry point, specq_w8a8_packed_noalloc, through the C ABI.

Its outputs must be bit-identical to those of specq_w8a8_packed, which takes a workspace,
and to the CPU oracle.  This holds on two calls in a row, the second with a smaller input, in
split-K, forced-split and unsplit configurations.  A call that needs more scratch than the static
array holds is refused (ENOSPC) before anything is launched, and its output is left untouched.
"""
import numpy as np
import pytest
import torch

import kernels as K
from gpu_util import assert_bitexact_fp16, note
from oracle import oracle as O
from specq import _lib, gen
from specq import workspace as _ws

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _stream():
    return torch.cuda.current_stream().cuda_stream


def call_noalloc(a, sa, wp, sw, out, M, N, Kd, block_m=0, split_k=0):
    return _lib.lib().specq_w8a8_packed_noalloc(
        a.data_ptr(), a.stride(0), wp.data.data_ptr(), sa.data_ptr(), sw.data_ptr(), out.data_ptr(), out.stride(0),
        M, N, Kd, 0, None, block_m, 0, 4, split_k, _stream())


def call_workspace(a, sa, wp, sw, out, M, N, Kd, block_m=0, split_k=0):
    L = _lib.lib()
    need = L.specq_w8a8_packed_workspace_size(M, N, Kd, block_m, 0, 4, split_k)
    ptr, nbytes = _ws.shared(DEV).ensure(need)
    return L.specq_w8a8_packed(
        a.data_ptr(), a.stride(0), wp.data.data_ptr(), sa.data_ptr(), sw.data_ptr(), out.data_ptr(), out.stride(0),
        M, N, Kd, 0, None, block_m, 0, 4, split_k, ptr, nbytes, _stream())


@pytest.mark.parametrize("N,Kd,Ms,split_k", [
    (4096, 14336, (72, 20), 0),    # down: the automatic tile splits K
    (1024, 4096, (100, 9), 4),     # k/v with a forced 4-way split
    (4096, 4096, (8, 3), 0),       # decode-sized q/o: no split, no scratch
    (1000, 528, (300, 17), 2),     # ragged N, K ending inside a 64-byte step
])
def test_noalloc_matches_workspace_entry(N, Kd, Ms, split_k):
    a, w, sa, sw = gen.w8a8_inputs(max(Ms), N, Kd, seed=N + Kd)
    ref = O.w8a8(a.numpy(), sa.numpy(), w.numpy(), sw.numpy())
    a, w, sa, sw = (t.to(DEV) for t in (a, w, sa, sw))
    wp = K.pack_weight_int8(w)
    for M in Ms:  # two calls in a row, the second smaller
        note(f"noalloc N={N} K={Kd} M={M} split_k={split_k}")
        cfg = K.KernelInfo(0, 1, M, N, Kd, 0, 0, 4, split_k).config
        o1 = torch.full((M, N), 7.0, dtype=torch.float16, device=DEV)
        o2 = torch.full((M, N), 7.0, dtype=torch.float16, device=DEV)
        assert call_workspace(a, sa, wp, sw, o1, M, N, Kd, split_k=split_k) == 0
        rc = call_noalloc(a, sa, wp, sw, o2, M, N, Kd, split_k=split_k)
        assert rc == 0, _lib.lib().specq_last_error().decode()
        torch.cuda.synchronize()
        assert torch.equal(o1, o2), f"noalloc differs from the workspace entry point at M={M} (split_k={cfg['split_k']})"
        assert_bitexact_fp16(o2, ref[:M], f"noalloc N={N} K={Kd} M={M}")
    if N == 4096 and Kd == 14336:
        assert K.KernelInfo(0, 1, 72, N, Kd, 0, 0, 4, 0).config["split_k"] > 1  # the scratch was used


def test_noalloc_back_to_back_without_sync():
    # Calls queued on one stream reuse the same counters and partial tiles in stream order.
    N, Kd = 4096, 14336
    a, w, sa, sw = (t.to(DEV) for t in gen.w8a8_inputs(80, N, Kd, seed=5))
    wp = K.pack_weight_int8(w)
    note("noalloc back to back")
    outs = []
    for M in (80, 33, 80, 1, 64):
        o = torch.empty((M, N), dtype=torch.float16, device=DEV)
        assert call_noalloc(a, sa, wp, sw, o, M, N, Kd, split_k=4) == 0
        outs.append((M, o))
    torch.cuda.synchronize()
    for M, o in outs:
        e = torch.empty((M, N), dtype=torch.float16, device=DEV)
        assert call_workspace(a, sa, wp, sw, e, M, N, Kd, split_k=4) == 0
        torch.cuda.synchronize()
        assert torch.equal(o, e), f"back-to-back noalloc call M={M} differs"


def test_noalloc_refuses_calls_beyond_the_scratch():
    N, Kd, M = 14336, 4096, 300
    a, w, sa, sw = (t.to(DEV) for t in gen.w8a8_inputs(M, N, Kd, seed=6))
    wp = K.pack_weight_int8(w)
    need = _lib.lib().specq_w8a8_packed_workspace_size(M, N, Kd, 16, 0, 4, 4)
    assert need > 32 * 1024 * 1024
    out = torch.full((M, N), 7.0, dtype=torch.float16, device=DEV)
    note("noalloc ENOSPC")
    rc = call_noalloc(a, sa, wp, sw, out, M, N, Kd, block_m=16, split_k=4)
    torch.cuda.synchronize()
    assert rc == -28 and "static scratch" in _lib.lib().specq_last_error().decode()
    assert bool((out == 7.0).all())


def test_noalloc_plan_mode_automatic_tiles():
    # A plan-mode call with automatic tiles (the launch that runs, per 16 rows of the active M,
    # its own tiling): the static scratch serves every step's split-K tiling, rows >= M untouched.
    N, Kd, M_MAX = 4096, 14336, 288
    a, w, sa, sw = (t.to(DEV) for t in gen.w8a8_inputs(M_MAX, N, Kd, seed=6))
    wp = K.pack_weight_int8(w)
    ref, _ = K.w8a8_matmul(a, sa, wp, sw, BLOCK_M=None)
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    L = _lib.lib()
    for M in (72, 8, 288, 144, 1, 200):
        note(f"noalloc plan M={M}")
        plan[0] = M
        o = torch.full((M_MAX, N), 7.0, dtype=torch.float16, device=DEV)
        rc = L.specq_w8a8_packed_noalloc(a.data_ptr(), a.stride(0), wp.data.data_ptr(), sa.data_ptr(), sw.data_ptr(),
                                         o.data_ptr(), o.stride(0), M_MAX, N, Kd, M_MAX, plan.data_ptr(), 0, 0, 4, 0,
                                         _stream())
        assert rc == 0, L.specq_last_error().decode()
        torch.cuda.synchronize()
        assert torch.equal(o[:M], ref[:M]), f"noalloc plan mode differs from eager at M={M}"
        assert bool((o[M:] == 7.0).all()), f"noalloc plan mode wrote rows >= M at M={M}"
