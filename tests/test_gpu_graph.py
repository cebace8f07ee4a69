"""One plan-mode hipGraph captured at the maximum grid replays every (B, k) bit-exactly
against eager launches (bench_graphs.py:144-159), for a chained two-layer INT8 stack:
W8A8 qkv -> paged attention -> W8A8 o -> W8A8 gate, up -> SiLU*mul -> INT8 quant -> W8A8 down.
Eager work and synchronisation run between replays, and every replay is checked."""
import random

import pytest
import torch

import kernels as K
from gpu_util import note
from specq import gen
from specq.plan import Plan

pytestmark = pytest.mark.gpu
DEV = "cuda"
HID, QKV, FF = 1024, 1536, 2048
H, H_KV, D = 32, 8, 128
B_MAX, KS = 8, (0, 2, 4, 8)
QL_MAX = max(KS) + 1
M_MAX = B_MAX * QL_MAX


def build_stack(L=2):
    layers = []
    for i in range(L):
        lw = {}
        for j, (name, N, Kd) in enumerate((("qkv", QKV, HID), ("o", HID, HID), ("gate", FF, HID),
                                            ("up", FF, HID), ("down", HID, FF))):
            w, sw = gen.w8a8_weights(N, Kd, seed=100 * i + j)
            lw[name] = (w.to(DEV), sw.to(DEV))
        lw["kv"] = [t.to(DEV) for t in gen.paged_kv(B_MAX, [300 + QL_MAX] * B_MAX, H_KV, D, seed=i)]
        layers.append(lw)
    return layers


def test_plan_graph_replays_every_shape_bit_exact():
    layers = build_stack()
    x_in = [t.to(DEV) for t in gen.w8a8_acts(M_MAX, HID, seed=7)]
    q_buf = gen.queries(B_MAX, QL_MAX, H, D, seed=8).to(DEV)
    bufs = {n: torch.zeros(M_MAX, N, device=DEV, dtype=torch.float16)
            for n, N in (("qkv", QKV), ("o", HID), ("gate", FF), ("up", FF), ("down", HID))}
    o_buf = torch.zeros_like(q_buf)
    hq = torch.zeros(M_MAX, FF, device=DEV, dtype=torch.int8)
    hs = torch.zeros(M_MAX, device=DEV, dtype=torch.float32)
    plan = Plan(DEV)

    def step(B, ql, use_plan):
        M = B * ql
        kw = dict(plan=plan.gemm, grid_m_max=M_MAX) if use_plan else {}
        a, sa = (x_in[0], x_in[1]) if use_plan else (x_in[0][:M], x_in[1][:M])
        for lw in layers:
            K.w8a8_matmul(a, sa, *lw["qkv"], out=bufs["qkv"], BLOCK_M=None, **kw)
            kc, vc, ks, vs, bt, cl = lw["kv"]
            if use_plan:
                K.paged_attention(q_buf, kc, vc, ks, vs, bt, cl, QL_MAX, QPP=QL_MAX, plan=plan.attn, out=o_buf)
            else:
                K.paged_attention(q_buf[:B], kc, vc, ks, vs, bt[:B], cl[:B], ql, QPP=ql, out=o_buf[:B])
            K.w8a8_matmul(a, sa, *lw["o"], out=bufs["o"], BLOCK_M=None, **kw)
            K.w8a8_matmul(a, sa, *lw["gate"], out=bufs["gate"], BLOCK_M=None, **kw)
            K.w8a8_matmul(a, sa, *lw["up"], out=bufs["up"], BLOCK_M=None, **kw)
            g, u = (bufs["gate"], bufs["up"]) if use_plan else (bufs["gate"][:M], bufs["up"][:M])
            K.silu_mul_quant_int8(g, u, q=hq if use_plan else hq[:M], s=hs if use_plan else hs[:M],
                                  plan=kw.get("plan"), grid_m_max=kw.get("grid_m_max"))
            h, hsc = (hq, hs) if use_plan else (hq[:M], hs[:M])
            K.w8a8_matmul(h, hsc, *lw["down"], out=bufs["down"], BLOCK_M=None, **kw)

    note("graph: warm-up eager + plan")
    for B in (1, B_MAX):
        for k in KS:
            step(B, k + 1, False)
    plan.set(B_MAX, QL_MAX)
    step(B_MAX, QL_MAX, True)
    torch.cuda.synchronize()

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step(B_MAX, QL_MAX, True)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(B_MAX, QL_MAX, True)
    torch.cuda.synchronize()

    rng = random.Random(0)
    trace = [(rng.randint(1, B_MAX), rng.choice(KS)) for _ in range(24)] + [(B_MAX, 8), (1, 0)]
    for i, (B, k) in enumerate(trace):
        ql = k + 1
        M = B * ql
        note(f"graph replay {i}: B={B} k={k}")
        step(B, ql, False)
        torch.cuda.synchronize()
        ref = {n: t[:M].clone() for n, t in bufs.items()}
        ref_o = o_buf[:B, :ql].clone()
        ref_h = (hq[:M].clone(), hs[:M].clone())
        for t in list(bufs.values()) + [o_buf, hq, hs]:
            t.zero_()
        plan.set(B, ql)
        graph.replay()
        torch.cuda.synchronize()
        for n, t in bufs.items():
            assert torch.equal(t[:M], ref[n]), f"{n} differs at B={B} k={k}"
            assert bool((t[M:] == 0).all()), f"{n} wrote inactive rows at B={B} k={k}"
        assert torch.equal(o_buf[:B, :ql], ref_o), f"attention differs at B={B} k={k}"
        assert bool((o_buf[B:] == 0).all()) and bool((o_buf[:B, ql:] == 0).all())
        assert torch.equal(hq[:M], ref_h[0]) and torch.equal(hs[:M], ref_h[1])


def test_bucketed_plan_graphs_replay_bit_exact():
    # PlanGraphSet: one plan graph per (B bucket, q_len), its GEMMs on the tiles an eager
    # call of the bucket's row count gets (plan_tiles="grid").  Every replay must equal eager bit for bit and leave rows past M untouched.  The
    # second half of the trace replays back to back without host syncs (outputs copied out on
    # the stream), so the plan's host slots are reused while earlier copies may still pend.
    from specq.plan import PlanGraphSet

    layers = build_stack()
    x_in = [t.to(DEV) for t in gen.w8a8_acts(M_MAX, HID, seed=17)]
    q_buf = gen.queries(B_MAX, QL_MAX, H, D, seed=18).to(DEV)
    bufs = {n: torch.zeros(M_MAX, N, device=DEV, dtype=torch.float16)
            for n, N in (("qkv", QKV), ("o", HID), ("gate", FF), ("up", FF), ("down", HID))}
    o_buf = torch.zeros_like(q_buf)
    hq = torch.zeros(M_MAX, FF, device=DEV, dtype=torch.int8)
    hs = torch.zeros(M_MAX, device=DEV, dtype=torch.float32)

    def step(Bg, qg, plan=None):
        Mg = Bg * qg
        kw = dict(plan=plan.gemm, grid_m_max=Mg) if plan is not None else {}
        gk = dict(kw, plan_tiles=plan.tiles) if plan is not None else {}  # the bucket's eager tiles
        a, sa = x_in[0][:Mg], x_in[1][:Mg]
        for lw in layers:
            K.w8a8_matmul(a, sa, *lw["qkv"], out=bufs["qkv"][:Mg], BLOCK_M=None, **gk)
            kc, vc, ks, vs, bt, cl = lw["kv"]
            K.paged_attention(q_buf[:Bg, :qg], kc, vc, ks, vs, bt[:Bg], cl[:Bg], qg, QPP=qg,
                              plan=plan.attn if plan is not None else None, out=o_buf[:Bg, :qg])
            K.w8a8_matmul(a, sa, *lw["o"], out=bufs["o"][:Mg], BLOCK_M=None, **gk)
            K.w8a8_matmul(a, sa, *lw["gate"], out=bufs["gate"][:Mg], BLOCK_M=None, **gk)
            K.w8a8_matmul(a, sa, *lw["up"], out=bufs["up"][:Mg], BLOCK_M=None, **gk)
            K.silu_mul_quant_int8(bufs["gate"][:Mg], bufs["up"][:Mg], q=hq[:Mg], s=hs[:Mg], **kw)
            K.w8a8_matmul(hq[:Mg], hs[:Mg], *lw["down"], out=bufs["down"][:Mg], BLOCK_M=None, **gk)

    note("bucketed graphs: capture")
    gset = PlanGraphSet(step, B_MAX, [k + 1 for k in KS])
    assert gset.buckets == [1, 2, 3, 4, 6, 8] and len(gset.graphs) == 24

    rng = random.Random(1)
    trace = [(rng.randint(1, B_MAX), rng.choice(KS)) for _ in range(20)] + [(B_MAX, 8), (1, 0), (3, 2)]
    refs = []
    for B, k in trace:
        ql = k + 1
        M = B * ql
        step(B, ql)
        torch.cuda.synchronize()
        refs.append(({n: t[:M].clone() for n, t in bufs.items()}, o_buf[:B, :ql].clone(), hq[:M].clone()))

    def check(i, got, B, ql):
        M = B * ql
        ref, ref_o, ref_h = refs[i]
        for n in bufs:
            assert torch.equal(got[n][:M], ref[n]), f"{n} differs at B={B} q_len={ql} (replay {i})"
            assert bool((got[n][M:] == 0).all()), f"{n} wrote inactive rows at B={B} q_len={ql}"
        assert torch.equal(got["o_buf"][:B, :ql], ref_o), f"attention differs at B={B} q_len={ql}"
        assert bool((got["o_buf"][B:] == 0).all()) and bool((got["o_buf"][:B, ql:] == 0).all())
        assert torch.equal(got["hq"][:M], ref_h)

    half = len(trace) // 2
    for i, (B, k) in enumerate(trace[:half]):  # synchronised replays
        note(f"bucketed replay {i}: B={B} k={k}")
        for t in list(bufs.values()) + [o_buf, hq, hs]:
            t.zero_()
        gset.replay(B, k + 1)
        torch.cuda.synchronize()
        check(i, dict(bufs, o_buf=o_buf, hq=hq), B, k + 1)
    note("bucketed replays back to back")
    snaps = []
    for B, k in trace[half:]:  # no host sync between replays: snapshots taken on the stream
        for t in list(bufs.values()) + [o_buf, hq, hs]:
            t.zero_()
        gset.replay(B, k + 1)
        snaps.append(dict({n: t.clone() for n, t in bufs.items()}, o_buf=o_buf.clone(), hq=hq.clone()))
    torch.cuda.synchronize()
    for j, ((B, k), got) in enumerate(zip(trace[half:], snaps)):
        check(half + j, got, B, k + 1)
