"""Config 4 at its real size: the 4-layer INT8 stack with d_model 4096 (qkv N=6144, o 4096x4096,
gate and up 14336x4096 each as one grouped launch, SiLU*mul fused with the INT8 quantisation,
down 4096x14336) and paged attention at context 1024 (H=32, H_KV=8, D=128, fp32 scales),
B <= 32, k in {0, 2, 4, 8}, M_MAX = 288 -- the stack bench.py times.

One plan-buffer graph captured at B=32, k=8 and the bucketed PlanGraphSet each replay a
seeded trace holding every distinct (B, k) once (random.Random(0) order) plus (32, 8) and
(1, 0).  Every replay is compared with the same step launched eagerly at its exact shape:
every GEMM output, the attention output and the quantised activations are bit-identical on
the active rows, and rows >= M, inactive sequences and query slots past q_len are never
written (bench_graphs.py:144-159).  Eager work and host synchronisation run between replays.
"""
import random

import numpy as np
import pytest
import torch

import kernels as K
from gpu_util import note
from specq import gen
from specq.plan import Plan, PlanGraphSet

pytestmark = pytest.mark.gpu
DEV = "cuda"
L, HID, QKV, FF = 4, 4096, 6144, 14336
H, H_KV, D, CTX = 32, 8, 128, 1024
B_MAX, KS = 32, (0, 2, 4, 8)
QL_MAX = max(KS) + 1
M_MAX = B_MAX * QL_MAX


class Stack:
    def __init__(self, packed: bool):
        self.layers = []
        for i in range(L):
            lw = {}
            for j, (name, N, Kd) in enumerate((("qkv", QKV, HID), ("o", HID, HID), ("gate", FF, HID),
                                                ("up", FF, HID), ("down", HID, FF))):
                w, sw = gen.w8a8_weights(N, Kd, seed=500 + 10 * i + j, device=DEV)
                lw[name] = (K.pack_weight_int8(w) if packed else w, sw)
            lw["kv"] = [t.to(DEV) for t in gen.paged_kv(B_MAX, [CTX + QL_MAX] * B_MAX, H_KV, D, seed=600 + i)]
            self.layers.append(lw)
        self.a, self.sa = (t.to(DEV) for t in gen.w8a8_acts(M_MAX, HID, seed=700))
        self.q = gen.queries(B_MAX, QL_MAX, H, D, seed=701).to(DEV)
        self.o = torch.zeros_like(self.q)
        self.bufs = {n: torch.zeros(M_MAX, N, device=DEV, dtype=torch.float16)
                     for n, N in (("qkv", QKV), ("o", HID), ("gate", FF), ("up", FF), ("down", HID))}
        self.hq = torch.zeros(M_MAX, FF, device=DEV, dtype=torch.int8)
        self.hs = torch.zeros(M_MAX, device=DEV, dtype=torch.float32)

    def step(self, Bg, qg, plan=None):
        """One step with its grids sized for (Bg, qg); with a plan the active (B, q_len) is read
        on the device (the GEMMs of a PlanGraphSet run its bucket's eager tiles)."""
        Mg = Bg * qg
        kw = dict(plan=plan.gemm, grid_m_max=Mg) if plan is not None else {}
        gk = dict(kw, plan_tiles=plan.tiles) if plan is not None else {}
        a, sa, b = self.a[:Mg], self.sa[:Mg], self.bufs
        for lw in self.layers:
            K.w8a8_matmul(a, sa, *lw["qkv"], out=b["qkv"][:Mg], BLOCK_M=None, **gk)
            kc, vc, ks, vs, bt, cl = lw["kv"]
            K.paged_attention(self.q[:Bg, :qg], kc, vc, ks, vs, bt[:Bg], cl[:Bg], qg, QPP=qg,
                              plan=plan.attn if plan is not None else None, out=self.o[:Bg, :qg])
            K.w8a8_matmul(a, sa, *lw["o"], out=b["o"][:Mg], BLOCK_M=None, **gk)
            K.w8a8_matmul_grouped(a, sa, [lw["gate"], lw["up"]], outs=[b["gate"][:Mg], b["up"][:Mg]], BLOCK_M=None,
                                  **gk)
            K.silu_mul_quant_int8(b["gate"][:Mg], b["up"][:Mg], q=self.hq[:Mg], s=self.hs[:Mg], **kw)
            K.w8a8_matmul(self.hq[:Mg], self.hs[:Mg], *lw["down"], out=b["down"][:Mg], BLOCK_M=None, **gk)

    def outputs(self):
        return list(self.bufs.values()) + [self.o, self.hq, self.hs]

    def zero(self):
        for t in self.outputs():
            t.zero_()

    def snapshot(self, B, ql):
        M = B * ql
        return ({n: t[:M].clone() for n, t in self.bufs.items()}, self.o[:B, :ql].clone(),
                self.hq[:M].clone(), self.hs[:M].clone())

    def check(self, ref, B, ql, what):
        M = B * ql
        bufs, o, hq, hs = ref
        for n, t in self.bufs.items():
            assert torch.equal(t[:M], bufs[n]), f"{n} differs from eager ({what})"
            assert bool((t[M:] == 0).all()), f"{n} wrote rows >= M ({what})"
        assert torch.equal(self.o[:B, :ql], o), f"attention differs from eager ({what})"
        assert bool((self.o[B:] == 0).all()) and bool((self.o[:B, ql:] == 0).all()), f"attention wrote inactive slots ({what})"
        assert torch.equal(self.hq[:M], hq) and torch.equal(self.hs[:M], hs), f"quantised h differs ({what})"
        assert bool((self.hq[M:] == 0).all()) and bool((self.hs[M:] == 0).all()), f"h written past M ({what})"


def trace():
    shapes = [(B, k) for B in range(1, B_MAX + 1) for k in KS]
    random.Random(0).shuffle(shapes)
    return shapes + [(B_MAX, 8), (1, 0)]


def replay_and_check(stack, replay, label):
    for i, (B, k) in enumerate(trace()):
        ql = k + 1
        note(f"config4 {label} replay {i}: B={B} k={k}")
        stack.step(B, ql)
        torch.cuda.synchronize()
        ref = stack.snapshot(B, ql)
        stack.zero()
        replay(B, ql)
        torch.cuda.synchronize()
        stack.check(ref, B, ql, f"{label} B={B} k={k}")


@pytest.mark.parametrize("packed", [True, False], ids=["packed", "rowmajor"])
def test_config4_plan_graph_every_shape_bit_exact(packed):
    stack = Stack(packed)
    note(f"config4 plan graph ({'packed' if packed else 'row-major'} weights): warm-up and capture")
    for B, k in ((1, 0), (B_MAX, 8), (7, 2), (19, 4)):
        stack.step(B, k + 1)
    plan = Plan(DEV)
    plan.set(B_MAX, QL_MAX)
    stack.step(B_MAX, QL_MAX, plan)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        stack.step(B_MAX, QL_MAX, plan)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        stack.step(B_MAX, QL_MAX, plan)
    torch.cuda.synchronize()

    def replay(B, ql):
        plan.set(B, ql)
        graph.replay()
    replay_and_check(stack, replay, "plan graph")


def test_config4_bucketed_plan_graphs_every_shape_bit_exact():
    stack = Stack(True)
    note("config4 bucketed plan graphs: capture")
    gset = PlanGraphSet(stack.step, B_MAX, [k + 1 for k in KS])
    assert len(gset.graphs) == len(gset.buckets) * len(KS)
    replay_and_check(stack, gset.replay, "bucketed")


@pytest.mark.parametrize("B,k", [(3, 2), (8, 8)])
def test_config4_eager_layer_against_oracle(B, k):
    """One layer of the config-4 stack, eager at (B, k), against the CPU oracle: the qkv (N =
    6144), o, gate and up GEMMs bit-exact (oracle.w8a8), the fused SiLU*mul quantisation
    bit-exact against the oracle's row quantisation of the device's SiLU*mul (which
    test_gpu_elementwise.py pins to one fp16 ulp of the float64 form), down bit-exact on those
    INT8 activations, and attention at context 1024 within the attention tests' bound."""
    from oracle import oracle as O
    ql = k + 1
    M = B * ql
    lw = {}
    for j, (name, N, Kd) in enumerate((("qkv", QKV, HID), ("o", HID, HID), ("gate", FF, HID), ("up", FF, HID),
                                       ("down", HID, FF))):
        w, sw = gen.w8a8_weights(N, Kd, seed=800 + j)
        lw[name] = (w, sw)
    a, sa = gen.w8a8_acts(M, HID, seed=810)
    kv = gen.paged_kv(B, [CTX + ql] * B, H_KV, D, seed=811)
    q = gen.queries(B, ql, H, D, seed=812)
    note(f"config4 eager layer vs oracle B={B} k={k}")
    dev = {n: (K.pack_weight_int8(w.to(DEV)), sw.to(DEV)) for n, (w, sw) in lw.items()}
    ad, sad = a.to(DEV), sa.to(DEV)
    qkv, _ = K.w8a8_matmul(ad, sad, *dev["qkv"], BLOCK_M=None)
    o, _ = K.w8a8_matmul(ad, sad, *dev["o"], BLOCK_M=None)
    (gate, up), _ = K.w8a8_matmul_grouped(ad, sad, [dev["gate"], dev["up"]], BLOCK_M=None)
    hq, hs = K.silu_mul_quant_int8(gate, up)
    h = K.silu_mul(gate, up)
    down, _ = K.w8a8_matmul(hq, hs, *dev["down"], BLOCK_M=None)
    kvd = [t.to(DEV) for t in kv]
    att, _ = K.paged_attention(q.to(DEV), *kvd, ql, QPP=ql)
    torch.cuda.synchronize()
    an, san = a.numpy(), sa.numpy()
    for name, got in (("qkv", qkv), ("o", o), ("gate", gate), ("up", up)):
        w, sw = lw[name]
        ref = O.w8a8(an, san, w.numpy(), sw.numpy())
        assert np.array_equal(got.cpu().numpy().view(np.uint16), ref.view(np.uint16)), f"{name} differs from the oracle"
    rq, rs = O.quantize_rows_int8(h.cpu().numpy())
    assert np.array_equal(hq.cpu().numpy(), rq) and np.array_equal(hs.cpu().numpy(), rs), "SiLU*mul quantisation"
    w, sw = lw["down"]
    ref = O.w8a8(hq.cpu().numpy(), hs.cpu().numpy(), w.numpy(), sw.numpy())
    assert np.array_equal(down.cpu().numpy().view(np.uint16), ref.view(np.uint16)), "down differs from the oracle"
    ref = O.paged_attention(q.numpy(), *[t.numpy() for t in kv], ql)
    err = np.abs(att.float().cpu().numpy().astype(np.float64) - ref)
    assert (err <= 4e-3 + 2.0 ** -9 * np.abs(ref)).all(), f"attention: max err {err.max():.3e}"
