"""Grouped W8A8 launches (w8a8_matmul_grouped / specq_w8a8_grouped) on the GPU.

GEMMs that share one activation -- q, k and v; gate and up -- run as one launch over separate
weight tensors and outputs.  Every output must be bit-identical to the one-GEMM call of the same
weight (and so to the CPU oracle): on row-major, packed INT8 and packed INT4 (W4A8) weights,
at the automatic tile and at forced BLOCK_M / split_k, with ragged widths whose last channel
block is partial, and in plan mode, where rows >= M stay untouched.
"""
import pytest
import torch

import kernels as K
from gpu_util import assert_bitexact_fp16, note
from oracle import oracle as O
from specq import gen

pytestmark = pytest.mark.gpu
DEV = "cuda"
GROUPS = {"qkv": [(4096, 4096), (1024, 4096), (1024, 4096)], "gate_up": [(14336, 4096), (14336, 4096)],
          "ragged": [(1000, 528), (24, 528), (520, 528), (8, 528)]}


def members(name, layout, seed):
    """[(weight as the launch takes it, channel scale, source weight)] of one group."""
    out = []
    for i, (N, Kd) in enumerate(GROUPS[name]):
        w, sw = gen.w8a8_weights(N, Kd, seed=seed + i, device=DEV)
        if layout == 0:
            out.append((w, sw, w))
        elif layout == 1:
            out.append((K.pack_weight_int8(w), sw, w))
        else:  # W4A8: INT4 nibbles in the reference uint8 packing
            qu = (w.to(torch.int16) & 15).to(torch.uint8)
            wp = (qu[:, :Kd // 2] | (qu[:, Kd // 2:] << 4)).contiguous()
            out.append((K.pack_weight_w4a8(wp), sw, wp))
    return out


def single(a, sa, w, sw, layout, **kw):
    if layout == 2:
        return K.w4a8_matmul(a, sa, w, sw, **kw)[0]
    return K.w8a8_matmul(a, sa, w, sw, **kw)[0]


@pytest.mark.parametrize("layout", [0, 1, 2], ids=["rowmajor", "packed", "w4a8"])
@pytest.mark.parametrize("name", ["qkv", "gate_up", "ragged"])
def test_grouped_equals_single_calls(name, layout):
    Kd = GROUPS[name][0][1]
    mem = members(name, layout, seed=11)
    a, sa = (t.to(DEV) for t in gen.w8a8_acts(300, Kd, seed=12))
    for M in (1, 8, 20, 72, 160, 288, 300):
        for bm, sk in ((None, 0), (16, 0), (128, 0), (None, 4)):
            note(f"grouped {name} layout={layout} M={M} BLOCK_M={bm} split_k={sk}")
            outs, ck = K.w8a8_matmul_grouped(a[:M], sa[:M], [(w, sw) for w, sw, _ in mem], BLOCK_M=bm, split_k=sk)
            refs = [single(a[:M], sa[:M], w, sw, layout, BLOCK_M=bm, split_k=sk) for w, sw, _ in mem]
            torch.cuda.synchronize()
            for g, (o, r) in enumerate(zip(outs, refs)):
                assert torch.equal(o, r), f"member {g} differs from its single call ({name} M={M} bm={bm} sk={sk})"
    if layout == 1:  # and the oracle, at the verification batch
        M = 72
        outs, _ = K.w8a8_matmul_grouped(a[:M], sa[:M], [(w, sw) for w, sw, _ in mem], BLOCK_M=None)
        torch.cuda.synchronize()
        for g, (o, (_, sw, w)) in enumerate(zip(outs, mem)):
            ref = O.w8a8(a[:M].cpu().numpy(), sa[:M].cpu().numpy(), w.cpu().numpy(), sw.cpu().numpy())
            assert_bitexact_fp16(o, ref, f"grouped {name} member {g} vs oracle")


@pytest.mark.parametrize("name", ["qkv", "gate_up"])
def test_grouped_plan_mode_sentinels(name):
    Kd = GROUPS[name][0][1]
    mem = [(w, sw) for w, sw, _ in members(name, 1, seed=21)]
    a, sa = (t.to(DEV) for t in gen.w8a8_acts(288, Kd, seed=22))
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    for tiles in (None, "grid"):
        for M in (1, 9, 45, 72, 200, 288):
            note(f"grouped plan {name} M={M} tiles={tiles}")
            eager, _ = K.w8a8_matmul_grouped(a[:M], sa[:M], mem, BLOCK_M=None)
            plan[0] = M
            outs = [torch.full((288, N), 7.0, dtype=torch.float16, device=DEV) for N, _ in GROUPS[name]]
            K.w8a8_matmul_grouped(a, sa, mem, outs=outs, BLOCK_M=None, plan=plan, grid_m_max=288, plan_tiles=tiles)
            torch.cuda.synchronize()
            for g, (o, e) in enumerate(zip(outs, eager)):
                assert torch.equal(o[:M], e), f"plan member {g} differs at M={M}"
                assert bool((o[M:] == 7.0).all()), f"plan member {g} wrote rows >= M at M={M}"


def test_grouped_argument_checks():
    mem = [(w, sw) for w, sw, _ in members("qkv", 1, seed=31)]
    a, sa = (t.to(DEV) for t in gen.w8a8_acts(8, 4096, seed=32))
    with pytest.raises(RuntimeError, match="1..4"):
        K.w8a8_matmul_grouped(a, sa, mem * 2)
    with pytest.raises(RuntimeError, match="all"):
        K.w8a8_matmul_grouped(a, sa, [mem[0], (mem[1][0].data, mem[1][1])])
    with pytest.raises(RuntimeError, match="outputs"):
        K.w8a8_matmul_grouped(a, sa, mem, outs=[torch.empty((8, 4096), dtype=torch.float16, device=DEV)] * 3)
