"""Plan-mode W8A8 with automatic tiles: one launch that picks its tiling per 16 rows of the
active M on the device (w8a8_plan.hpp).

A graph captured at M_MAX = 288 must give, for every active M, the bit-identical rows of an
eager call and leave rows >= M untouched (bench_graphs.py:144-159, correctness.py:50-65).  The
tiling changes with M (direct-activation tiles at M <= 16, 32- to 288-row streaming tiles above,
split-K where the cost model picks it), so every M = 0..288 is checked on the config-1 shapes,
on packed INT8, row-major and packed INT4 (W4A8) weights, single and grouped, in eager calls
and in one captured graph replayed over changing plans.
"""
import pytest
import torch

import kernels as K
from gpu_util import note

pytestmark = pytest.mark.gpu
DEV = "cuda"
M_MAX = 288
SHAPES = {"q": (4096, 4096), "kv": (1024, 4096), "gate": (14336, 4096), "down": (4096, 14336)}


def _weights(N, Kd, seed, layout):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randint(-127, 128, (N, Kd), dtype=torch.int8, device=DEV, generator=g)
    sw = torch.rand(N, device=DEV, generator=g) * 0.009 + 0.001
    if layout == 0:
        return w, sw
    if layout == 1:
        return K.pack_weight_int8(w), sw
    qu = (w.to(torch.int16) & 15).to(torch.uint8)
    return K.pack_weight_w4a8((qu[:, :Kd // 2] | (qu[:, Kd // 2:] << 4)).contiguous()), sw


def _acts(Kd, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    a = torch.randint(-127, 128, (M_MAX, Kd), dtype=torch.int8, device=DEV, generator=g)
    sa = torch.rand(M_MAX, device=DEV, generator=g) * 0.015 + 0.005
    return a, sa


def test_plan_table_reports_a_tiling_per_step():
    # The tiling the launch uses for M = 16 r is the one reported for a grid of 16 r rows.
    for name, (N, Kd) in SHAPES.items():
        rows = []
        for r in range(1, M_MAX // 16 + 1):
            cf = K.KernelInfo(0, 1 | 16, 16 * r, N, Kd, 0, 0, 4, 0).config
            assert cf["block_m"] in (16, 32, 48, 64, 80, 144, 160, 192, 224, 256, 288)
            assert cf["block_n"] in (16, 32, 64, 128)
            rows.append((cf["block_m"], cf["block_n"], cf["split_k"]))
        note(f"plan tiles {name}: " + " ".join(f"{16 * (i + 1)}:{t}" for i, t in enumerate(rows)))
        assert rows[0][0] == 16, f"{name}: M <= 16 runs the direct-activation tile"


@pytest.mark.parametrize("name", list(SHAPES))
def test_plan_every_M_bit_identical_to_eager(name):
    N, Kd = SHAPES[name]
    w, sw = _weights(N, Kd, seed=41, layout=1)
    a, sa = _acts(Kd, seed=42)
    ref, _ = K.w8a8_matmul(a, sa, w, sw, BLOCK_M=None)  # output rows do not depend on M
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    out = torch.empty((M_MAX, N), dtype=torch.float16, device=DEV)
    note(f"w8a8 plan tiles {name} every M")
    for M in range(0, M_MAX + 1):
        plan[0] = M
        out.fill_(7.0)
        K.w8a8_matmul(a, sa, w, sw, out=out, plan=plan, grid_m_max=M_MAX, BLOCK_M=None)
        torch.cuda.synchronize()
        assert torch.equal(out[:M], ref[:M]), f"{name}: plan-mode rows differ from eager at M={M}"
        assert bool((out[M:] == 7.0).all()), f"{name}: rows >= M written at M={M}"


@pytest.mark.parametrize("layout", [0, 2])
def test_plan_layouts_bit_identical_to_eager(layout):
    N, Kd = SHAPES["q"]
    w, sw = _weights(N, Kd, seed=43, layout=layout)
    a, sa = _acts(Kd, seed=44)
    mm = K.w4a8_matmul if layout == 2 else K.w8a8_matmul
    ref, _ = mm(a, sa, w, sw, BLOCK_M=None)
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    out = torch.empty((M_MAX, N), dtype=torch.float16, device=DEV)
    for M in (1, 8, 16, 17, 31, 33, 48, 49, 72, 80, 81, 96, 144, 145, 160, 161, 200, 256, 287, 288):
        note(f"w8a8 plan tiles layout {layout} M={M}")
        plan[0] = M
        out.fill_(7.0)
        mm(a, sa, w, sw, out=out, plan=plan, grid_m_max=M_MAX, BLOCK_M=None)
        torch.cuda.synchronize()
        assert torch.equal(out[:M], ref[:M]), f"layout {layout}: plan-mode rows differ from eager at M={M}"
        assert bool((out[M:] == 7.0).all()), f"layout {layout}: rows >= M written at M={M}"


def test_plan_grouped_every_16_rows():
    Kd = 4096
    mem = [_weights(N, Kd, seed=45 + i, layout=1) for i, N in enumerate((4096, 1024, 1024))]
    a, sa = _acts(Kd, seed=48)
    ref, _ = K.w8a8_matmul_grouped(a, sa, mem, BLOCK_M=None)
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    outs = [torch.empty((M_MAX, N), dtype=torch.float16, device=DEV) for N in (4096, 1024, 1024)]
    for M in sorted(set(list(range(1, M_MAX + 1, 16)) + list(range(16, M_MAX + 1, 16)))):
        note(f"w8a8 plan tiles grouped qkv M={M}")
        plan[0] = M
        for o in outs:
            o.fill_(7.0)
        K.w8a8_matmul_grouped(a, sa, mem, outs=outs, plan=plan, grid_m_max=M_MAX, BLOCK_M=None)
        torch.cuda.synchronize()
        for g, (o, r) in enumerate(zip(outs, ref)):
            assert torch.equal(o[:M], r[:M]), f"grouped member {g} differs at M={M}"
            assert bool((o[M:] == 7.0).all()), f"grouped member {g} wrote rows >= M at M={M}"


def test_plan_graph_replays_every_step():
    # One graph captured at M_MAX, replayed with the plan changing between replays (eager work
    # and synchronisations in between), every replay checked.
    N, Kd = SHAPES["down"]
    w, sw = _weights(N, Kd, seed=49, layout=1)
    a, sa = _acts(Kd, seed=50)
    ref, _ = K.w8a8_matmul(a, sa, w, sw, BLOCK_M=None)
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    out = torch.full((M_MAX, N), 7.0, dtype=torch.float16, device=DEV)
    plan[0] = M_MAX
    K.w8a8_matmul(a, sa, w, sw, out=out, plan=plan, grid_m_max=M_MAX, BLOCK_M=None)  # workspace sized
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        K.w8a8_matmul(a, sa, w, sw, out=out, plan=plan, grid_m_max=M_MAX, BLOCK_M=None)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        K.w8a8_matmul(a, sa, w, sw, out=out, plan=plan, grid_m_max=M_MAX, BLOCK_M=None)
    for M in (1, 288, 16, 17, 72, 3, 144, 145, 250, 0, 48, 80, 96):
        note(f"w8a8 plan tiles graph replay M={M}")
        plan.fill_(0)
        plan[0] = M
        out.fill_(7.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[:M], ref[:M]), f"graph replay differs from eager at M={M}"
        assert bool((out[M:] == 7.0).all()), f"graph replay wrote rows >= M at M={M}"
