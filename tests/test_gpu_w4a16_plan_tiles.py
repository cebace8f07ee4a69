"""Plan-mode W4A16 with automatic tiles: one launch that picks its tiling per 16 rows of the
active M on the device (w4a16_plan.hpp).

The split count, and with it the fp32 summation order, depends only on (N, K), so every tiling
gives the same bits: for every active M = 0..288 the rows of a plan-mode call equal an eager
call's (bench_graphs.py:144-159), rows >= M stay untouched (correctness.py:50-65), on the
config-2 shapes, on the three weight layouts, and in one captured graph replayed over plans.
"""
import pytest
import torch

import kernels as K
from gpu_util import note

pytestmark = pytest.mark.gpu
DEV = "cuda"
M_MAX = 288
SHAPES = {"q": (4096, 4096), "kv": (1024, 4096), "gate": (14336, 4096), "down": (4096, 14336)}


def _weight(N, Kd, seed, layout):
    """Unsigned nibbles as the reference uint8 packing (layout 0), int32 words (layout 1) or
    packed once at load (layout 2)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randint(0, 16, (N, Kd), dtype=torch.uint8, device=DEV, generator=g)
    sc = (torch.rand(N, Kd // 128, device=DEV, generator=g) * 0.018 + 0.002).half()
    if layout == 1:
        return K.pack_int4_i32(q), sc
    wp = (q[:, :Kd // 2] | (q[:, Kd // 2:] << 4)).contiguous()
    return (K.pack_weight_int4(wp) if layout == 2 else wp), sc


def _acts(Kd, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(M_MAX, Kd, device=DEV, generator=g).half()


def test_w4a16_plan_table_reports_a_tiling_per_step():
    for name, (N, Kd) in SHAPES.items():
        rows = []
        for r in range(1, M_MAX // 16 + 1):
            cf = K.KernelInfo(1, 2 | 16, 16 * r, N, Kd, 0, 0, 4, 0).config
            assert cf["block_m"] in (16, 32, 48, 64, 80, 96, 112, 144) and cf["block_n"] in (64, 128)
            rows.append((cf["block_m"], cf["block_n"], cf["split_k"]))
        note(f"w4a16 plan tiles {name}: " + " ".join(f"{16 * (i + 1)}:{t}" for i, t in enumerate(rows)))
        assert rows[0][0] == 16


@pytest.mark.parametrize("name", list(SHAPES))
def test_w4a16_plan_every_M_bit_identical_to_eager(name):
    N, Kd = SHAPES[name]
    wp, sc = _weight(N, Kd, seed=61, layout=2)
    a = _acts(Kd, seed=62)
    ref, _ = K.w4a16_matmul(a, wp, sc, BLOCK_M=None)
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    out = torch.empty((M_MAX, N), dtype=torch.float16, device=DEV)
    note(f"w4a16 plan tiles {name} every M")
    for M in range(0, M_MAX + 1):
        plan[0] = M
        out.fill_(7.0)
        K.w4a16_matmul(a, wp, sc, out=out, plan=plan, grid_m_max=M_MAX, BLOCK_M=None)
        torch.cuda.synchronize()
        assert torch.equal(out[:M], ref[:M]), f"{name}: plan-mode rows differ from eager at M={M}"
        assert bool((out[M:] == 7.0).all()), f"{name}: rows >= M written at M={M}"


@pytest.mark.parametrize("layout", [0, 1])
def test_w4a16_plan_source_layouts(layout):
    N, Kd = SHAPES["q"]
    wp, sc = _weight(N, Kd, seed=63, layout=layout)
    a = _acts(Kd, seed=64)
    ref, _ = K.w4a16_matmul(a, wp, sc, BLOCK_M=None)
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    out = torch.empty((M_MAX, N), dtype=torch.float16, device=DEV)
    for M in (1, 16, 17, 48, 72, 80, 81, 144, 145, 200, 288):
        note(f"w4a16 plan tiles layout {layout} M={M}")
        plan[0] = M
        out.fill_(7.0)
        K.w4a16_matmul(a, wp, sc, out=out, plan=plan, grid_m_max=M_MAX, BLOCK_M=None)
        torch.cuda.synchronize()
        assert torch.equal(out[:M], ref[:M]), f"layout {layout}: plan-mode rows differ from eager at M={M}"
        assert bool((out[M:] == 7.0).all()), f"layout {layout}: rows >= M written at M={M}"


def test_w4a16_plan_graph_replays_every_step():
    N, Kd = SHAPES["down"]
    wp, sc = _weight(N, Kd, seed=65, layout=2)
    a = _acts(Kd, seed=66)
    ref, _ = K.w4a16_matmul(a, wp, sc, BLOCK_M=None)
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    out = torch.full((M_MAX, N), 7.0, dtype=torch.float16, device=DEV)
    plan[0] = M_MAX
    K.w4a16_matmul(a, wp, sc, out=out, plan=plan, grid_m_max=M_MAX, BLOCK_M=None)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        K.w4a16_matmul(a, wp, sc, out=out, plan=plan, grid_m_max=M_MAX, BLOCK_M=None)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        K.w4a16_matmul(a, wp, sc, out=out, plan=plan, grid_m_max=M_MAX, BLOCK_M=None)
    for M in (1, 288, 16, 17, 72, 3, 144, 145, 250, 0, 48, 80, 96):
        note(f"w4a16 plan tiles graph replay M={M}")
        plan.fill_(0)
        plan[0] = M
        out.fill_(7.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[:M], ref[:M]), f"graph replay differs from eager at M={M}"
        assert bool((out[M:] == 7.0).all()), f"graph replay wrote rows >= M at M={M}"
