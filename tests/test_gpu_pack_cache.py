"""The transparent packing of row-major W8A8 weights (kernels._WeightPackCache) on the GPU.

A drop-in caller passes the reference's row-major int8 w_q (bench_graphs.py:55-64,
correctness.py:36).  With the cache on, w8a8_matmul and w8a8_matmul_grouped pack each such
weight once and run the packed-fragment kernels: the outputs must be bit-identical to the
row-major kernels and to the oracle; an in-place update of the weight must repack it; a miss
inside graph capture must run the row-major kernel without allocating; the byte budget must hold.
"""
import pytest
import torch

import kernels as K
from gpu_util import assert_bitexact_fp16, note
from oracle import oracle as O
from specq import gen

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture
def cache_on():
    K.clear_weight_pack_cache()
    K.set_weight_pack_cache(True, budget_bytes=64 << 30)
    yield K._pack_cache
    K.set_weight_pack_cache(False)


def test_rowmajor_weight_packed_once_bit_identical(cache_on):
    a, w, sa, sw = gen.w8a8_inputs(72, 4096, 4096, seed=21)
    ref = O.w8a8(a.numpy(), sa.numpy(), w.numpy(), sw.numpy())
    a, w, sa, sw = (t.to(DEV) for t in (a, w, sa, sw))
    note("pack cache: row-major weight, two calls")
    o1, ck1 = K.w8a8_matmul(a, sa, w, sw, BLOCK_M=None)
    o2, ck2 = K.w8a8_matmul(a, sa, w, sw, BLOCK_M=None)
    torch.cuda.synchronize()
    assert len(cache_on._d) == 1 and cache_on.bytes == K.pack_weight_int8(w).data.numel()
    assert ck1.name == ck2.name
    assert_bitexact_fp16(o1, ref, "cached call 1")
    assert torch.equal(o1, o2)
    K.set_weight_pack_cache(False)
    o3, _ = K.w8a8_matmul(a, sa, w, sw, BLOCK_M=None)  # the row-major kernels
    torch.cuda.synchronize()
    assert torch.equal(o1, o3)


def test_inplace_update_repacks(cache_on):
    a, w, sa, sw = gen.w8a8_inputs(20, 1024, 512, seed=22)
    a, w, sa, sw = (t.to(DEV) for t in (a, w, sa, sw))
    note("pack cache: in-place weight update")
    K.w8a8_matmul(a, sa, w, sw, BLOCK_M=None)
    w.neg_()  # int8 [-127, 127] stays in range
    view = w[:512]
    w2 = w.cpu()
    out, _ = K.w8a8_matmul(a, sa, w, sw, BLOCK_M=None)
    outv, _ = K.w8a8_matmul(a, sa, view, sw[:512], BLOCK_M=None)
    torch.cuda.synchronize()
    ref = O.w8a8(a.cpu().numpy(), sa.cpu().numpy(), w2.numpy(), sw.cpu().numpy())
    assert_bitexact_fp16(out, ref, "after the in-place update")
    assert_bitexact_fp16(outv, ref[:, :512], "a view of the updated weight")


def test_grouped_rowmajor_members_use_cache(cache_on):
    mem = [gen.w8a8_weights(N, 4096, seed=30 + i) for i, N in enumerate((4096, 1024, 1024))]
    a, sa = gen.w8a8_acts(72, 4096, seed=33)
    a, sa = a.to(DEV), sa.to(DEV)
    mem = [(w.to(DEV), sw.to(DEV)) for w, sw in mem]
    note("pack cache: grouped launch over row-major members")
    outs, _ = K.w8a8_matmul_grouped(a, sa, mem, BLOCK_M=None)
    torch.cuda.synchronize()
    assert len(cache_on._d) == 3
    for (w, sw), o in zip(mem, outs):
        ref = O.w8a8(a.cpu().numpy(), sa.cpu().numpy(), w.cpu().numpy(), sw.cpu().numpy())
        assert_bitexact_fp16(o, ref, "grouped member through the cache")


def test_miss_during_capture_runs_rowmajor_kernel(cache_on):
    a, w, sa, sw = gen.w8a8_inputs(72, 4096, 14336, seed=24)
    ref = O.w8a8(a.numpy(), sa.numpy(), w.numpy(), sw.numpy())
    a, w, sa, sw = (t.to(DEV) for t in (a, w, sa, sw))
    out = torch.empty((72, 4096), dtype=torch.float16, device=DEV)
    K.set_weight_pack_cache(False)  # warm-up (sizes the workspace) without packing
    K.w8a8_matmul(a, sa, w, sw, out=out, BLOCK_M=None)
    K.set_weight_pack_cache(True)
    torch.cuda.synchronize()
    note("pack cache: miss inside graph capture")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            K.w8a8_matmul(a, sa, w, sw, out=out, BLOCK_M=None)
    torch.cuda.current_stream().wait_stream(s)
    assert len(cache_on._d) == 0, "a miss during capture must not pack"
    for rep in range(3):
        out.fill_(7.0)
        g.replay()
        torch.cuda.synchronize()
        assert_bitexact_fp16(out, ref, f"replay {rep}")


def test_budget_evicts_least_recently_used(cache_on):
    ws = [gen.w8a8_weights(1024, 1024, seed=40 + i)[0].to(DEV) for i in range(4)]
    a, sa = gen.w8a8_acts(8, 1024, seed=44)
    a, sa = a.to(DEV), sa.to(DEV)
    sw = torch.full((1024,), 0.01, device=DEV)
    per = K.pack_weight_int8(ws[0]).data.numel()
    K.set_weight_pack_cache(True, budget_bytes=2 * per)
    note("pack cache: budget")
    for w in ws:
        K.w8a8_matmul(a, sa, w, sw, BLOCK_M=None)
    torch.cuda.synchronize()
    assert cache_on.bytes <= 2 * per and len(cache_on._d) == 2
    keys = list(cache_on._d)
    assert keys[-1] == K._WeightPackCache._key(ws[3]) and keys[0] == K._WeightPackCache._key(ws[2])
