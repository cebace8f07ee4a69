"""Grouped W4A16 launches (w4a16_matmul_grouped / specq_w4a16_grouped) on the GPU.

GEMMs that share one fp16 activation -- q, k and v; gate and up -- run as one launch over
separate INT4 weights, scales and outputs.  Every output must be bit-identical to the one-GEMM
call of the same weight with the same split_k (the members keep their own split counts, and
W4A16 results do not depend on the tiles), and so within the stated tolerance of the float64
oracle: on load-time packed, int32 and reference uint8 weights, at the automatic tile and at
forced BLOCK_M / BLOCK_N / split_k, with ragged widths whose last channel block is partial,
with members whose automatic split counts differ (one launch each), and in plan mode, where
rows >= M stay untouched.
"""
import pytest
import torch

import kernels as K
from gpu_util import note
from oracle import oracle as O
from specq import gen
from test_gpu_w4a16 import check_tol

pytestmark = pytest.mark.gpu
DEV = "cuda"
GROUPS = {"qkv": [(4096, 4096), (1024, 4096), (1024, 4096)], "gate_up": [(14336, 4096), (14336, 4096)],
          "ragged": [(1000, 1024), (24, 1024), (520, 1024), (8, 1024)],
          # automatic split counts 4 and 1 (K = 4096): one launch per member unless split_k is set
          "mixed": [(4096, 4096), (14336, 4096)]}


def members(name, layout, seed):
    """[(weight as the launch takes it, fp16 scales, unsigned nibbles [N, K])] of one group."""
    out = []
    for i, (N, Kd) in enumerate(GROUPS[name]):
        qu, sc = gen.int4_weights(N, Kd, seed=seed + i, device=DEV)
        if layout == 0:
            w = gen.pack_u8_reference(qu)
        else:
            w = gen.pack_i32(qu)
            if layout == 2:
                w = K.pack_weight_int4(w)
        out.append((w, sc, qu))
    return out


@pytest.mark.parametrize("layout", [2, 1, 0], ids=["packed", "int32", "uint8"])
@pytest.mark.parametrize("name", ["qkv", "gate_up", "ragged", "mixed"])
def test_w4a16_grouped_equals_single_calls(name, layout):
    Kd = GROUPS[name][0][1]
    mem = members(name, layout, seed=41)
    a = gen.fp16_acts(300, Kd, seed=42, device=DEV)
    cases = ((None, None, 0), (16, None, 0), (144, 128, 0), (None, None, 2))
    for M in (1, 8, 20, 72, 160, 288, 300):
        for bm, bn, sk in cases:
            note(f"w4a16 grouped {name} layout={layout} M={M} BLOCK_M={bm} BLOCK_N={bn} split_k={sk}")
            outs, ck = K.w4a16_matmul_grouped(a[:M], [(w, sc) for w, sc, _ in mem], BLOCK_M=bm, BLOCK_N=bn,
                                              split_k=sk)
            refs = [K.w4a16_matmul(a[:M], w, sc, BLOCK_M=bm, BLOCK_N=bn, split_k=sk)[0] for w, sc, _ in mem]
            torch.cuda.synchronize()
            for g, (o, r) in enumerate(zip(outs, refs)):
                assert torch.equal(o, r), f"member {g} differs from its single call ({name} M={M} bm={bm} sk={sk})"
    if layout == 2:  # and the oracle, at the verification batch
        M = 72
        outs, _ = K.w4a16_matmul_grouped(a[:M], [(w, sc) for w, sc, _ in mem])
        torch.cuda.synchronize()
        for g, (o, (_, sc, qu)) in enumerate(zip(outs, mem)):
            ref = O.w4a16(a[:M].cpu().numpy(), qu.cpu().numpy(), sc.cpu().numpy(), 128)
            check_tol(o, ref, f"grouped {name} member {g} vs oracle")


@pytest.mark.parametrize("name", ["qkv", "gate_up"])
def test_w4a16_grouped_plan_mode_sentinels(name):
    Kd = GROUPS[name][0][1]
    mem = [(w, sc) for w, sc, _ in members(name, 2, seed=51)]
    a = gen.fp16_acts(288, Kd, seed=52, device=DEV)
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    for M in (1, 9, 45, 72, 200, 288):
        note(f"w4a16 grouped plan {name} M={M}")
        eager, _ = K.w4a16_matmul_grouped(a[:M], mem)
        plan[0] = M
        outs = [torch.full((288, N), 7.0, dtype=torch.float16, device=DEV) for N, _ in GROUPS[name]]
        K.w4a16_matmul_grouped(a, mem, outs=outs, plan=plan, grid_m_max=288)
        torch.cuda.synchronize()
        for g, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o[:M], e), f"plan member {g} differs at M={M}"
            assert bool((o[M:] == 7.0).all()), f"plan member {g} wrote rows >= M at M={M}"


def test_w4a16_grouped_in_graph():
    """One captured graph of the grouped launches replays bit-identically to eager, several times."""
    mem = [(w, sc) for w, sc, _ in members("qkv", 2, seed=61)]
    a = gen.fp16_acts(72, 4096, seed=62, device=DEV)
    outs = [torch.empty((72, N), dtype=torch.float16, device=DEV) for N, _ in GROUPS["qkv"]]
    eager, _ = K.w4a16_matmul_grouped(a, mem)
    K.w4a16_matmul_grouped(a, mem, outs=outs)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        K.w4a16_matmul_grouped(a, mem, outs=outs)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        K.w4a16_matmul_grouped(a, mem, outs=outs)
    for rep in range(3):
        for o in outs:
            o.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        for g, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o, e), f"graph replay {rep} member {g} differs from eager"


def test_w4a16_grouped_argument_checks():
    mem = [(w, sc) for w, sc, _ in members("qkv", 2, seed=71)]
    a = gen.fp16_acts(8, 4096, seed=72, device=DEV)
    with pytest.raises(RuntimeError, match="1..4"):
        K.w4a16_matmul_grouped(a, mem * 2)
    with pytest.raises(RuntimeError, match="all"):
        K.w4a16_matmul_grouped(a, [mem[0], (torch.zeros((1024, 512), dtype=torch.int32, device=DEV), mem[1][1])])
    with pytest.raises(RuntimeError, match="outputs"):
        K.w4a16_matmul_grouped(a, mem, outs=[torch.empty((8, 4096), dtype=torch.float16, device=DEV)] * 3)
    with pytest.raises(RuntimeError, match=r"\[N, K/group\]"):
        K.w4a16_matmul_grouped(a, [mem[0], (mem[1][0], mem[1][1][:512]), mem[2]])
    with pytest.raises(RuntimeError, match=r"\[N, K/group\]"):
        K.w4a16_matmul(a, mem[0][0], mem[0][1][:, :16])


@pytest.mark.parametrize("name", ["qkv", "ragged"])
def test_w4a16_grouped_register_stream_path(name):
    """The register-stream family (w4a16_path 1, 16- and 32-row tiles) in grouped launches: its
    per-member selection and split-K column base run only there.  Each member must equal its
    single call on the same family, tile and split count."""
    from specq import _lib

    Kd = GROUPS[name][0][1]
    mem = [(w, sc) for w, sc, _ in members(name, 2, seed=81)]
    a = gen.fp16_acts(64, Kd, seed=82, device=DEV)
    try:
        _lib.set_option("w4a16_path", 1)
        for M in (1, 8, 20, 32):
            for bm in (16, 32):
                for sk in (1, 2):
                    note(f"w4a16 grouped rk {name} M={M} BLOCK_M={bm} split_k={sk}")
                    outs, _ = K.w4a16_matmul_grouped(a[:M], mem, BLOCK_M=bm, split_k=sk)
                    refs = [K.w4a16_matmul(a[:M], w, sc, BLOCK_M=bm, split_k=sk)[0] for w, sc in mem]
                    torch.cuda.synchronize()
                    for g, (o, r) in enumerate(zip(outs, refs)):
                        assert torch.equal(o, r), f"rk member {g} differs ({name} M={M} bm={bm} sk={sk})"
    finally:
        _lib.set_option("w4a16_path", 0)
