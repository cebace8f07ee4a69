"""Benchmark of the quantized verification path on one MI355X (prints one JSON line).

Workload: W8A8 GEMMs over the seven linears of a Llama-3-8B layer (N x K:
q 4096x4096, k and v 1024x4096, o 4096x4096, gate and up 14336x4096, down 4096x14336) at the
verification batch M = B*(k+1) = 8*9 = 72.  One step is the linears of one verification
forward: 32 layers x 7 GEMMs streaming 6.98 GB of distinct INT8 weights (far beyond the
256 MiB Infinity Cache, so every step reads its weights from HBM).  The GEMMs that share an
activation in a model layer run as one grouped launch over their separate weight tensors
(q|k|v and gate|up; w8a8_matmul_grouped), so a layer is 4 launches.  Weights are packed once at
load time into the kernel's MFMA-fragment layout (pack_weight_int8; bit-identical results).
The step is captured once into a hipGraph and replayed; inputs are resident in HBM before the
timed region starts.

  value        algorithmic HBM bytes of a step / step time, in GB/s (whole job, one GPU): every
               weight, channel scale and output once, and each launch's activations and token
               scales once
  roofline     the dominant kernel (the grouped gate|up launch, 54% of the bytes): algorithmic
               bytes per launch / its mean launch duration, measured with HIP events around a
               graph of back-to-back launches on the stream the kernels run on, against 8 TB/s
  cpu_baseline the reference's PyTorch formulas on the host cores (oracle/cpu_baseline.py):
               torch._int_mm with the fp32 epilogue on one layer's seven
               linears at M = 72 (the value), plus the fp32 formula, W4A16 and attention timings
  detail       the k=0 decode step (M = 8) and the verify/decode ratio (target <= 1.1); the same
               step as 7 separate launches per layer, on row-major weights, and on the fused
               weights the reference benchmarks (bench_matmul.py:16); per-launch times; the
               per-layer t(B, k) / t(B, 0) grid of W8A8 and W4A16 (REPORT.md:71-78); W4A16 and
               W4A8 steps; INT8 paged verification attention over the reference's B x k x QPP
               grid at ctx 1024 and 4096 (bench_attention.py:16-39); the paged KV-cache append;
               and the plan-buffer graph replay of the config-4 stack.  W8A8 launches, attention
               and the KV append are all timed the same way: graphs of back-to-back launches
               over distinct weights or caches, events on the stream the kernels run on

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu] [--no-detail] [--write-grids DIR]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "specdec-quant-triton_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0  # dense
# The seven linears of a Llama-3-8B layer, and how a layer launches them:
# GEMMs that share an activation run as one grouped launch.
CONFIG1 = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
           ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
LAUNCHES = [("qkv", ("q", "k", "v")), ("o", ("o",)), ("gate_up", ("gate", "up")), ("down", ("down",))]
# The reference's own benchmark fuses the weights instead (bench_matmul.py:16).
LINEARS = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 28672, 4096), ("down", 4096, 14336)]
DOMINANT = "gate_up"
METRIC = "GEMM µs & HBM GB/s vs M=B·(k+1); INT8 verify-attn µs at k=8; graph replay µs"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def w8a8_bytes(M: int, N: int, K: int) -> int:
    """Algorithmic HBM bytes of one W8A8 call: W, A, sa, sw read once, C written once."""
    return N * K + M * K + 4 * M + 4 * N + 2 * M * N


def grouped_bytes(M: int, shapes) -> int:
    """Algorithmic HBM bytes of one launch of GEMMs sharing an activation [M, K]: every weight,
    channel scale and output once, the activation and token scales once."""
    K = shapes[0][1]
    return sum(N * Kd + 4 * N + 2 * M * N for N, Kd in shapes) + M * K + 4 * M


def config1_step_bytes(M: int, layers: int) -> int:
    shape = {n: (N, Kd) for n, N, Kd in CONFIG1}
    return layers * sum(grouped_bytes(M, [shape[m] for m in mem]) for _, mem in LAUNCHES)


def w4a16_bytes(M: int, N: int, K: int, group: int = 128) -> int:
    return N * K // 2 + 2 * N * (K // group) + 2 * M * K + 2 * M * N


def attn_bytes(B: int, L: int, q_len: int, H: int, H_KV: int, D: int, scale_bytes: int, page: int = 16) -> int:
    """K/V int8 + their scales for every context token, q in + out (fp16), block table, lengths."""
    return (B * L * H_KV * (2 * D + 2 * scale_bytes) + 4 * B * q_len * H * D
            + 4 * B * ((L + page - 1) // page) + 4 * B)


def kv_append_bytes(B: int, q_len: int, H_KV: int, D: int, scale_bytes: int) -> int:
    """New K and V rows read (fp16), int8 rows and scales written, block-table entry and length read."""
    return B * q_len * H_KV * 2 * (2 * D + D + scale_bytes) + 4 * B * q_len + 4 * B


# ------------------------------------------------------------------------------------------
# GPU helpers
# ------------------------------------------------------------------------------------------
def capture(fn):
    """Capture fn() (already warmed up) into a graph on a side stream."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_replays(g, steps: int, warmup: int) -> float:
    """Mean ms per replay over `steps` replays bracketed by synchronisation (events on the stream)."""
    import torch

    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def make_weights(K, L: int, seed: int = 0, packed: bool = True, linears=LINEARS):
    """L layers of the linears: int8 weights (packed MFMA fragments, or row-major) and fp32
    per-channel scales, on the GPU."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(seed)
    layers = []
    for _ in range(L):
        lw = {}
        for name, N, Kd in linears:
            w = torch.randint(-127, 128, (N, Kd), dtype=torch.int8, device="cuda", generator=g)
            sw = torch.rand((N,), device="cuda", generator=g) * 0.009 + 0.001
            lw[name] = (K.pack_weight_int8(w) if packed else w, sw)
            del w
        layers.append(lw)
    torch.cuda.synchronize()
    return layers


def w8a8_step_fn(K, layers, acts, M, outs, linears=LINEARS):
    """One launch per linear (each on the activation of its K)."""
    a, sa, a_ff = acts[0][:M], acts[1][:M], acts[2][:M]

    def step():
        for lw in layers:
            for name, N, Kd in linears:
                w, sw = lw[name]
                K.w8a8_matmul(a if Kd == a.shape[1] else a_ff, sa, w, sw, out=outs[name][:M], BLOCK_M=None)
    return step


def config1_step_fn(K, layers, acts, M, outs):
    """A layer's seven linears as 4 launches: q|k|v and gate|up grouped, o and down alone."""
    a, sa, a_ff = acts[0][:M], acts[1][:M], acts[2][:M]
    shape = {n: (N, Kd) for n, N, Kd in CONFIG1}

    def step():
        for lw in layers:
            for _, mem in LAUNCHES:
                x = a if shape[mem[0]][1] == a.shape[1] else a_ff
                if len(mem) == 1:
                    K.w8a8_matmul(x, sa, *lw[mem[0]], out=outs[mem[0]][:M], BLOCK_M=None)
                else:
                    K.w8a8_matmul_grouped(x, sa, [lw[m] for m in mem], outs=[outs[m][:M] for m in mem], BLOCK_M=None)
    return step


def per_launch_us(K, torch, layers, acts, M, outs, args):
    """Mean duration of each of a layer's 4 launches at M: a graph of the launch over every
    layer's weights, timed with events on the stream it runs on."""
    shape = {n: (N, Kd) for n, N, Kd in CONFIG1}
    res = {}
    for lname, mem in LAUNCHES:
        x = acts[0][:M] if shape[mem[0]][1] == acts[0].shape[1] else acts[2][:M]
        sa = acts[1][:M]

        def run(mem=mem, x=x, sa=sa):
            for lw in layers:
                K.w8a8_matmul_grouped(x, sa, [lw[m] for m in mem], outs=[outs[m][:M] for m in mem], BLOCK_M=None)
        run()
        torch.cuda.synchronize()
        g = capture(run)
        ms = time_replays(g, max(5, args.steps), 2)
        us = ms * 1e3 / len(layers)
        b = grouped_bytes(M, [shape[m] for m in mem])
        _, ck = K.w8a8_matmul_grouped(x, sa, [layers[0][m] for m in mem], outs=[outs[m][:M] for m in mem],
                                      BLOCK_M=None)
        res[lname] = dict(us=us, bytes=b, GBps=b / (us * 1e-6) / 1e9, kernel=ck.name, config=ck.config)
        del g
    return res


# ------------------------------------------------------------------------------------------
# Parts of the run
# ------------------------------------------------------------------------------------------
def bench_w8a8(args, K, torch):
    from specq import grids
    g = torch.Generator(device="cuda").manual_seed(2)
    M_max = 300
    a = torch.randint(-127, 128, (M_max, 4096), dtype=torch.int8, device="cuda", generator=g)
    a_ff = torch.randint(-127, 128, (M_max, 14336), dtype=torch.int8, device="cuda", generator=g)
    sa = torch.rand((M_max,), device="cuda", generator=g) * 0.015 + 0.005
    acts = (a, sa, a_ff)
    outs = {name: torch.empty((M_max, N), dtype=torch.float16, device="cuda")
            for name, N, _ in CONFIG1 + LINEARS}
    res = {}
    layers = make_weights(K, args.layers, seed=1, packed=True, linears=CONFIG1)
    for label, M in (("verify", args.B * (args.k + 1)), ("decode", args.B)):
        step = config1_step_fn(K, layers, acts, M, outs)
        step()
        torch.cuda.synchronize()
        graph = capture(step)
        bytes_step = config1_step_bytes(M, args.layers)
        log(f"w8a8 config-1 {label} M={M}: warmup {args.warmup}, timing {args.steps} steps")
        ms = time_replays(graph, args.steps, args.warmup)
        res[label] = dict(M=M, ms=ms, bytes=bytes_step, GBps=bytes_step / (ms * 1e-3) / 1e9)
        del graph
        # The same step as 7 separate launches per layer.
        step = w8a8_step_fn(K, layers, acts, M, outs, linears=CONFIG1)
        step()
        torch.cuda.synchronize()
        graph = capture(step)
        ms = time_replays(graph, args.steps, args.warmup)
        res[label + "_7_launches"] = dict(M=M, ms=ms, GBps=args.layers * sum(w8a8_bytes(M, N, Kd) for _, N, Kd in CONFIG1)
                                          / (ms * 1e-3) / 1e9)
        del graph
    # Per-launch durations at the verification M; the dominant one is the roofline kernel.
    M = res["verify"]["M"]
    res["launches"] = per_launch_us(K, torch, layers, acts, M, outs, args)
    res["launches_decode"] = per_launch_us(K, torch, layers, acts, args.B, outs, args)
    if not args.no_detail:
        # The reference's verification-cost table (REPORT.md:71-78): t(B, k) / t(B, 0) per layer.
        flat = [[lw[m] for _, mem in LAUNCHES for m in mem] for lw in layers]
        log("w8a8 layer grid B x k")
        res["grid_us"], res["grid_ratio"] = grids.layer_ratio_grid(K, flat, "w8a8")
    del layers
    torch.cuda.empty_cache()
    # The same verification step on row-major weights (the reference's w_q layout), as a
    # drop-in caller gets it (each weight packed once, on its first call, by the transparent
    # cache), and on the row-major kernels themselves (cache off).
    layers = make_weights(K, args.layers, seed=1, packed=False, linears=CONFIG1)
    for label, cached in (("verify_rowmajor", True), ("verify_rowmajor_kernel", False)):
        K.set_weight_pack_cache(cached)
        step = config1_step_fn(K, layers, acts, M, outs)
        step()
        torch.cuda.synchronize()
        graph = capture(step)
        ms = time_replays(graph, args.steps, args.warmup)
        res[label] = dict(M=M, ms=ms, GBps=res["verify"]["bytes"] / (ms * 1e-3) / 1e9)
        del graph
        K.clear_weight_pack_cache()
    K.set_weight_pack_cache(True)
    del layers
    torch.cuda.empty_cache()
    # The reference's fused-weight shapes (bench_matmul.py:16), verification and decode.
    layers = make_weights(K, args.layers, seed=1, packed=True, linears=LINEARS)
    for label, Mx in (("verify_fused_weights", M), ("decode_fused_weights", args.B)):
        step = w8a8_step_fn(K, layers, acts, Mx, outs, linears=LINEARS)
        step()
        torch.cuda.synchronize()
        graph = capture(step)
        ms = time_replays(graph, args.steps, args.warmup)
        b = args.layers * sum(w8a8_bytes(Mx, N, Kd) for _, N, Kd in LINEARS)
        res[label] = dict(M=Mx, ms=ms, GBps=b / (ms * 1e-3) / 1e9)
        del graph
    del layers
    torch.cuda.empty_cache()
    return res


def i32_to_u8_reference(wp):
    """The same INT4 weight in the reference's uint8 layout (kernels.py:143-145): byte j of a
    row holds k = j in its low nibble and k = j + K/2 in its high nibble; wp is int32 [N, K/8]
    with nibble i of word j holding k = 8j + i."""
    import torch

    N = wp.shape[0]
    q = torch.stack([(wp >> (4 * i)) & 0xF for i in range(8)], dim=-1).reshape(N, -1).to(torch.uint8)
    half = q.shape[1] // 2
    return (q[:, :half] | (q[:, half:] << 4)).contiguous()


def bench_w4a16(args, K, torch):
    """W4A16 (config 2) over the seven config-1 linears, M = 72 and 8: INT4 weights (int32, 8
    nibbles per word) packed once at load into MFMA fragments (pack_weight_int4).  The step runs
    q|k|v and gate|up as grouped launches over their separate weights (w4a16_matmul_grouped,
    bit-identical to one call per linear), 4 launches per layer like the W8A8 step; the same step
    as 7 launches per layer, and the grouped step on the int32 and the reference's uint8 weights
    as given, go beside it, with the per-layer t(B, k) / t(B, 0) grid."""
    from specq import grids

    g = torch.Generator(device="cuda").manual_seed(3)
    layers, raw = [], []
    for _ in range(args.layers):
        lw, lr = {}, {}
        for name, N, Kd in CONFIG1:
            wp = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, Kd // 8), dtype=torch.int32, device="cuda", generator=g)
            sc = (torch.rand((N, Kd // 128), device="cuda", generator=g) * 0.018 + 0.002).half()
            lw[name] = (K.pack_weight_int4(wp), sc)
            lr[name] = (wp, sc)
        layers.append(lw)
        raw.append(lr)
    x = torch.randn((300, 4096), device="cuda", generator=g).half()
    x_ff = torch.randn((300, 14336), device="cuda", generator=g).half()
    outs = {name: torch.empty((300, N), dtype=torch.float16, device="cuda") for name, N, _ in CONFIG1}
    shape = {n: (N, Kd) for n, N, Kd in CONFIG1}
    res = {}
    vM, dM = args.B * (args.k + 1), args.B
    raw_u8 = [{name: (i32_to_u8_reference(wp), sc) for name, (wp, sc) in lr.items()} for lr in raw]
    for label, M, ls, grouped in (("verify", vM, layers, True), ("decode", dM, layers, True),
                                  ("verify_7_launches", vM, layers, False), ("decode_7_launches", dM, layers, False),
                                  ("verify_int32", vM, raw, True), ("verify_uint8", vM, raw_u8, True),
                                  ("decode_uint8", dM, raw_u8, True)):
        def step():
            for lw in ls:
                if grouped:
                    for _, mem in LAUNCHES:
                        xa = x[:M] if shape[mem[0]][1] == 4096 else x_ff[:M]
                        K.w4a16_matmul_grouped(xa, [lw[m] for m in mem], outs=[outs[m][:M] for m in mem])
                else:
                    for name, N, Kd in CONFIG1:
                        K.w4a16_matmul(x[:M] if Kd == 4096 else x_ff[:M], *lw[name], out=outs[name][:M],
                                       BLOCK_M=None)
        step()
        torch.cuda.synchronize()
        graph = capture(step)
        log(f"w4a16 {label} M={M}")
        ms = time_replays(graph, args.steps, args.warmup)
        # Algorithmic bytes: every weight, scale and output once, each launch's activations once.
        if grouped:
            b = args.layers * sum(sum(w4a16_bytes(M, shape[m][0], shape[m][1]) for m in mem)
                                  - (len(mem) - 1) * 2 * M * shape[mem[0]][1] for _, mem in LAUNCHES)
        else:
            b = args.layers * sum(w4a16_bytes(M, N, Kd) for _, N, Kd in CONFIG1)
        flops = args.layers * sum(2 * M * N * Kd for _, N, Kd in CONFIG1)
        gbps, tflops = b / (ms * 1e-3) / 1e9, flops / (ms * 1e-3) / 1e12
        res[label] = dict(M=M, ms=ms, GBps=gbps, TFLOPs=tflops, hbm_frac=gbps / HBM_PEAK_GBS,
                          mfma_frac=tflops / FP16_MFMA_PEAK_TFLOPS)
        del graph
    log("w4a16 layer grid B x k")
    flat = [[lw[m] for _, mem in LAUNCHES for m in mem] for lw in layers]
    res["grid_us"], res["grid_ratio"] = grids.layer_ratio_grid(K, flat, "w4a16")
    del layers, raw, raw_u8
    torch.cuda.empty_cache()
    return res


def w4a8_bytes(M: int, N: int, K: int) -> int:
    """Algorithmic HBM bytes of one W4A8 call: packed INT4 W, A, sa, sw read once, C written once."""
    return N * K // 2 + M * K + 4 * M + 4 * N + 2 * M * N


def bench_w4a8(args, K, torch):
    """W4A8 (INT4 weights on the INT8 MFMA path, per-channel scale) over the seven config-1
    linears, M = 72 and 8, weights packed once at load (pack_weight_w4a8), q|k|v and gate|up as
    grouped launches like the W8A8 step."""
    g = torch.Generator(device="cuda").manual_seed(4)
    layers = []
    for _ in range(args.layers):
        lw = {}
        for name, N, Kd in CONFIG1:
            wp = torch.randint(0, 256, (N, Kd // 2), dtype=torch.uint8, device="cuda", generator=g)
            sw = torch.rand((N,), device="cuda", generator=g) * 0.009 + 0.001
            lw[name] = (K.pack_weight_w4a8(wp), sw)
            del wp
        layers.append(lw)
    a = torch.randint(-127, 128, (300, 4096), dtype=torch.int8, device="cuda", generator=g)
    a_ff = torch.randint(-127, 128, (300, 14336), dtype=torch.int8, device="cuda", generator=g)
    sa = torch.rand((300,), device="cuda", generator=g) * 0.015 + 0.005
    outs = {name: torch.empty((300, N), dtype=torch.float16, device="cuda") for name, N, _ in CONFIG1}
    shape = {n: (N, Kd) for n, N, Kd in CONFIG1}
    res = {}
    for label, M in (("verify", args.B * (args.k + 1)), ("decode", args.B)):
        def step():
            for lw in layers:
                for _, mem in LAUNCHES:
                    x = a[:M] if shape[mem[0]][1] == 4096 else a_ff[:M]
                    K.w8a8_matmul_grouped(x, sa[:M], [lw[m] for m in mem], outs=[outs[m][:M] for m in mem],
                                          BLOCK_M=None)
        step()
        torch.cuda.synchronize()
        graph = capture(step)
        log(f"w4a8 {label} M={M}")
        ms = time_replays(graph, args.steps, args.warmup)
        b = args.layers * sum(w4a8_bytes(M, N, Kd) for _, N, Kd in CONFIG1)
        res[label] = dict(M=M, ms=ms, GBps=b / (ms * 1e-3) / 1e9)
        del graph
    del layers
    torch.cuda.empty_cache()
    return res


def bench_attention(args, K, torch):
    """INT8 paged verification attention (config 3) and the paged KV-cache append.

    The grid of the reference's attention benchmark (bench_attention.py:16-39): B in
    {1, 2, 4, 8, 16, 32} x k = 0..8 x QPP in {1, k + 1} at context 1024 and 4096, each point the
    mean launch of a graph of back-to-back launches over distinct caches (specq/grids.py), so
    every launch reads HBM and no per-call event overhead is counted; fractions are algorithmic
    bytes / time against 8 TB/s.  The B = 8, k = 8 point is also timed the reference's way
    (events around each call after triton.testing.do_bench's zeroing flush), for comparison
    with its published figures only."""
    from specq import gen, grids
    from specq.timing import do_bench

    H, H_KV, D = 32, 8, 128
    res = {"grid": {}}
    B, ql = args.B, args.k + 1
    for ctx in (1024, 4096):
        log(f"attention grid ctx={ctx}")
        g = grids.attention_grid(K, ctx, H=H, H_KV=H_KV, D=D)
        res["grid"][ctx] = g
        for name, qpp in (("fused", ql), ("qpp1", 1)):
            r = g[(B, args.k, qpp)]
            res[f"ctx{ctx}_{name}"] = dict(us=r["us"], GBps=r["GBps"], hbm_frac=r["frac"], kv_GBps=r["kv_GBps"])
        log(f"attention B={B} k={args.k} ctx={ctx}: fused {res[f'ctx{ctx}_fused']['us']:.1f} us in a graph, "
            f"QPP=1 {res[f'ctx{ctx}_qpp1']['us']:.1f} us")
        # The reference's own method on the same call: events around each call, zeroing flush.
        L = ctx + ql
        kc, vc, ks, vs, bt, cl = grids.make_caches(B, L, H_KV, D, 1, seed=5)[0]
        q = gen.queries(B, ql, H, D, seed=6).cuda()
        out = torch.zeros_like(q)
        fn = lambda: K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=ql, out=out)  # noqa: E731
        ms = do_bench(fn, warmup=5, rep=20, flush="dirty")
        res[f"ctx{ctx}_fused_reference_method"] = dict(us=ms * 1e3)
        del kc, vc, ks, vs, bt, cl
        torch.cuda.empty_cache()
    # The step before attention: the k+1 new tokens' K/V quantised into the cache pages, a graph
    # over distinct caches (each append touches one page per sequence and head).
    for Bx in (B, 32):
        L = 4096 + ql
        copies = 64
        caches = grids.make_caches(Bx, L, H_KV, D, copies, seed=7)
        gq = torch.Generator(device="cuda").manual_seed(8)
        kn = torch.randn((Bx, ql, H_KV, D), device="cuda", generator=gq).half()
        vn = torch.randn((Bx, ql, H_KV, D), device="cuda", generator=gq).half()

        def run(caches=caches, kn=kn, vn=vn):
            for kc, vc, ks, vs, bt, cl in caches:
                K.paged_kv_append(kn, vn, kc, vc, ks, vs, bt, cl, ql)
        us = grids.graph_us(run, copies)
        b = kv_append_bytes(Bx, ql, H_KV, D, 4)
        res[f"kv_append_B{Bx}"] = dict(us=us, GBps=b / (us * 1e-6) / 1e9)
        del caches
        torch.cuda.empty_cache()
    log(f"kv append B={B}: {res[f'kv_append_B{B}']['us']:.2f} us in a graph")
    return res


def bench_plan_graph(args, K, torch):
    """Config 4: a 4-layer INT8 stack (d_model 4096, weights packed at load; gate and up as one
    grouped launch over their separate weights) replayed over a seeded 1000-step (B, k) trace,
    B in 1..32, k in {0, 2, 4, 8}, under the strategies of bench_graphs.py:109-114 and two more:
      eager     every step launched with its exact shapes (a fifth of the trace)
      allshapes one graph per distinct (B, k) of the trace (captured before timing)
      maxpad    one graph per B with k padded to 8, no plan: every step computes B * 9 rows
      maxgrid   one graph at B=32, k=8 (M=288), no plan: every step computes 288 rows
      plan      one plan-buffer graph captured at B=32, k=8, the active (B, k) read on device
      bucketed  plan-buffer graphs per (B bucket 1/2/3/4/6/8/12/16/24/32, k): the GEMMs of each
                bucket run the tiles an eager call of its row count would pick (PlanGraphSet,
                plan_tiles="grid")
    Host perf_counter around plan write + replay + sync per step (bench_graphs.py:126-136); fixed-k
    traces (bench_graphs.py:141-142) give the mean step per k.  Padding waste is reported in
    M-tiles (REPORT.md:147): per step, the BLOCK_M-row tiles a strategy's GEMMs compute beyond the
    ceil(M / BLOCK_M) the active rows need, for BLOCK_M in {16, 32, 64, 128}; plan-mode tiles past
    the active M exit at once and are not counted.  The library's own tiles are reported as rows
    computed beyond M."""
    import random

    from specq import gen
    from specq.plan import Plan, PlanGraphSet

    L, HID, QKV, FF = 4, 4096, 6144, 14336
    H, H_KV, D, CTX = 32, 8, 128, 1024
    B_MAX, KS = 32, (0, 2, 4, 8)
    QL_MAX = max(KS) + 1
    M_MAX = B_MAX * QL_MAX
    gg = torch.Generator(device="cuda").manual_seed(9)

    def w(N, Kd):  # packed at load, as in the headline step
        return (K.pack_weight_int8(torch.randint(-127, 128, (N, Kd), dtype=torch.int8, device="cuda", generator=gg)),
                torch.rand((N,), device="cuda", generator=gg) * 0.009 + 0.001)
    layers = []
    for i in range(L):
        lw = dict(qkv=w(QKV, HID), o=w(HID, HID), gate=w(FF, HID), up=w(FF, HID), down=w(HID, FF))
        lw["kv"] = [t.cuda() for t in gen.paged_kv(B_MAX, [CTX + QL_MAX] * B_MAX, H_KV, D, seed=20 + i)]
        layers.append(lw)
    a = torch.randint(-127, 128, (M_MAX, HID), dtype=torch.int8, device="cuda", generator=gg)
    sa = torch.rand((M_MAX,), device="cuda", generator=gg) * 0.015 + 0.005
    q_buf = gen.queries(B_MAX, QL_MAX, H, D, seed=8).cuda()
    o_buf = torch.zeros_like(q_buf)
    bufs = {n: torch.zeros(M_MAX, N, device="cuda", dtype=torch.float16)
            for n, N in (("qkv", QKV), ("o", HID), ("gate", FF), ("up", FF), ("down", HID))}
    hq = torch.zeros(M_MAX, FF, device="cuda", dtype=torch.int8)
    hs = torch.zeros(M_MAX, device="cuda", dtype=torch.float32)

    def step(Bg, qg, plan=None):
        """One step with grids sized for (Bg, qg): the exact shape without a plan, else the
        maxima of a plan-mode launch whose active (B, q_len) is read on the device."""
        Mg = Bg * qg
        kw = dict(plan=plan.gemm, grid_m_max=Mg) if plan is not None else {}
        gk = dict(kw, plan_tiles=plan.tiles) if plan is not None else {}
        aa, ss = a[:Mg], sa[:Mg]
        for lw in layers:
            K.w8a8_matmul(aa, ss, *lw["qkv"], out=bufs["qkv"][:Mg], BLOCK_M=None, **gk)
            kc, vc, ks, vs, bt, cl = lw["kv"]
            K.paged_attention(q_buf[:Bg, :qg], kc, vc, ks, vs, bt[:Bg], cl[:Bg], qg, QPP=qg,
                              plan=plan.attn if plan is not None else None, out=o_buf[:Bg, :qg])
            K.w8a8_matmul(aa, ss, *lw["o"], out=bufs["o"][:Mg], BLOCK_M=None, **gk)
            K.w8a8_matmul_grouped(aa, ss, [lw["gate"], lw["up"]], outs=[bufs["gate"][:Mg], bufs["up"][:Mg]],
                                  BLOCK_M=None, **gk)
            K.silu_mul_quant_int8(bufs["gate"][:Mg], bufs["up"][:Mg], q=hq[:Mg], s=hs[:Mg], **kw)
            K.w8a8_matmul(hq[:Mg], hs[:Mg], *lw["down"], out=bufs["down"][:Mg], BLOCK_M=None, **gk)

    def rows_computed(Mg, M, plan_mode, grid_tiles=False):
        """Token rows the qkv GEMM computes for active M on a grid of Mg rows (the tile the
        library resolves for that call; plan-mode chunks past M exit without computing).  A
        plan-mode call with automatic tiles runs the tiling of M's 16-row step, which is the
        one reported for a grid of that step's rows."""
        if plan_mode and not grid_tiles:
            Mg = min(Mg, 16 * -(-max(M, 1) // 16))
        bm = K.KernelInfo(0, 1 | (16 if plan_mode and not grid_tiles else 0), Mg, QKV, HID, 0, 0, 4, 0).config["block_m"]
        return bm * -(-M // bm) if plan_mode else bm * -(-Mg // bm)

    rng = random.Random(0)
    trace = [(rng.randint(1, B_MAX), rng.choice(KS)) for _ in range(args.trace)]
    shapes = sorted(set(trace))
    for B, k in shapes:  # warm every exact shape (also sizes the shared workspace)
        step(B, k + 1)
    for B in range(1, B_MAX + 1):
        step(B, QL_MAX)
    torch.cuda.synchronize()

    def timed(run, tr):
        for B, k in tr[:20]:
            run(B, k + 1)
        torch.cuda.synchronize()
        lat = []
        for B, k in tr:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            run(B, k + 1)
            torch.cuda.synchronize()
            lat.append((time.perf_counter() - t0) * 1e3)
        return lat

    t_build = {}
    t0 = time.perf_counter()
    per_shape = {bk: capture(lambda bk=bk: step(bk[0], bk[1] + 1)) for bk in shapes}
    t_build["allshapes"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    per_b = {B: capture(lambda B=B: step(B, QL_MAX)) for B in range(1, B_MAX + 1)}
    t_build["maxpad"] = time.perf_counter() - t0
    gmax = capture(lambda: step(B_MAX, QL_MAX))
    plan1 = Plan("cuda")
    plan1.set(B_MAX, QL_MAX)
    t0 = time.perf_counter()
    gplan = capture(lambda: step(B_MAX, QL_MAX, plan1))
    t_build["plan"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    gset = PlanGraphSet(step, B_MAX, [k + 1 for k in KS])
    t_build["bucketed"] = time.perf_counter() - t0

    def run_plan(B, ql):
        plan1.set(B, ql)
        gplan.replay()
    runs = {"allshapes": lambda B, ql: per_shape[(B, ql - 1)].replay(),
            "maxpad": lambda B, ql: per_b[B].replay(),
            "maxgrid": lambda B, ql: gmax.replay(),
            "plan": run_plan,
            "bucketed": gset.replay}
    res = {"eager": timed(lambda B, ql: step(B, ql), trace[: max(40, args.trace // 5)])}
    for name, fn in runs.items():
        res[name] = timed(fn, trace)

    tokens = sum(B * (k + 1) for B, k in trace)
    out = dict(steps=len(trace), allshapes_graphs=len(shapes), maxpad_graphs=len(per_b),
               bucketed_graphs=len(gset.graphs))
    for name, tb in t_build.items():
        out[f"{name}_build_s"] = tb
    for name, lat in res.items():
        out[f"{name}_p50_ms"] = statistics.median(lat)
        out[f"{name}_p99_ms"] = sorted(lat)[int(0.99 * (len(lat) - 1))]
        if name != "eager":
            out[f"{name}_tokens_per_s"] = tokens / (sum(lat) * 1e-3)
    for name in ("plan", "bucketed", "maxpad"):
        out[f"{name}_p50_over_allshapes"] = out[f"{name}_p50_ms"] / out["allshapes_p50_ms"]
        out[f"{name}_p99_over_allshapes"] = out[f"{name}_p99_ms"] / out["allshapes_p99_ms"]
    # fixed-k traces (bench_graphs.py:141-142): mean ms per step
    for k in KS:
        rk = random.Random(10 + k)
        tr = [(rk.randint(1, B_MAX), k) for _ in range(max(50, args.trace // 10))]
        for name in ("allshapes", "maxpad", "plan", "bucketed"):
            fn = runs[name]
            if name == "allshapes":
                tr_ok = [(B, kk) for B, kk in tr if (B, kk) in per_shape]
                lat = timed(fn, tr_ok) if tr_ok else [float("nan")]
            else:
                lat = timed(fn, tr)
            out[f"fixed_k{k}_{name}_mean_ms"] = statistics.fmean(lat)
    # padding waste in M-tiles per step at each BLOCK_M (REPORT.md:147), and the library's rows
    for bm in (16, 32, 64, 128):
        need = [-(-(B * (k + 1)) // bm) for B, k in trace]
        out[f"pad_tiles_bm{bm}_maxpad"] = statistics.fmean(-(-(B * QL_MAX) // bm) - n for (B, k), n in zip(trace, need))
        out[f"pad_tiles_bm{bm}_maxgrid"] = statistics.fmean(-(-M_MAX // bm) - n for n in need)
        out[f"pad_tiles_bm{bm}_eager_allshapes_plan"] = 0.0
    waste = dict(eager=0.0, maxpad=0.0, maxgrid=0.0, plan=0.0, bucketed=0.0)
    for B, k in trace:
        M = B * (k + 1)
        waste["eager"] += rows_computed(M, M, False) - M
        waste["maxpad"] += rows_computed(B * QL_MAX, M, False) - M
        waste["maxgrid"] += rows_computed(M_MAX, M, False) - M
        waste["plan"] += rows_computed(M_MAX, M, True) - M
        waste["bucketed"] += rows_computed(gset.bucket(B) * (k + 1), M, True, grid_tiles=True) - M
    torch.cuda.synchronize()
    for name, v in waste.items():
        out[f"{name}_pad_rows_per_step"] = v / len(trace)
    out["allshapes_pad_rows_per_step"] = out["eager_pad_rows_per_step"]
    log(f"plan graphs: P50 plan {out['plan_p50_ms']:.3f} / bucketed {out['bucketed_p50_ms']:.3f} / "
        f"allshapes {out['allshapes_p50_ms']:.3f} / maxpad {out['maxpad_p50_ms']:.3f} / "
        f"maxgrid {out['maxgrid_p50_ms']:.3f} / eager {out['eager_p50_ms']:.3f} ms")
    del per_shape, per_b, gmax, gplan, gset
    return out


def cpu_baseline(args, M: int, seconds: float):
    """The reference's PyTorch formulas on the host cores (oracle/cpu_baseline.py), each on a
    bounded sample of the same workload:
      value   torch._int_mm + the fp32 epilogue over one layer's seven config-1 linears at M
      also    the reference test's fp32 formula on the same layer (correctness.py:37), W4A16
              x.float() @ deq.float().T on the same shapes (correctness.py:76), and dense fp32
              attention at B=8, k=8, ctx 4096 (kernels.py:289-309)
    Threads: every CPU the process may run on (os.sched_getaffinity), capped by OMP_NUM_THREADS
    where that is set -- the GPU box gives one GPU's job a share of 16 of the host's CPUs.
    Both the host's CPU count and the threads used are reported."""
    import statistics as st

    import torch

    from oracle import cpu_baseline as C

    host_cpus = os.cpu_count() or 1
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else host_cpus
    omp = os.environ.get("OMP_NUM_THREADS", "")
    cores = min(usable, int(omp)) if omp.isdigit() and int(omp) > 0 else usable
    torch.set_num_threads(cores)
    cores = torch.get_num_threads()
    model = "unknown CPU"
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), model)
    except OSError:
        pass
    g = torch.Generator().manual_seed(0)
    a4 = torch.randint(-127, 128, (M, 4096), dtype=torch.int8, generator=g)
    a14 = torch.randint(-127, 128, (M, 14336), dtype=torch.int8, generator=g)
    sa = torch.rand(M, generator=g) * 0.015 + 0.005
    ws = {}
    for name, N, Kd in CONFIG1:
        w = torch.randint(-127, 128, (N, Kd), dtype=torch.int8, generator=g)
        ws[name] = (w, w.T.contiguous(), torch.rand(N, generator=g) * 0.009 + 0.001)

    def timed(fn, budget):
        t_end, times = time.perf_counter() + budget, []
        fn()  # warm-up
        while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 50):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return st.median(times), len(times)

    def layer_int_mm():
        for name, N, Kd in CONFIG1:
            C.w8a8_int_mm(a4 if Kd == 4096 else a14, sa, ws[name][1], ws[name][2])

    def layer_fp32():
        for name, N, Kd in CONFIG1:
            C.w8a8_fp32_formula(a4 if Kd == 4096 else a14, sa, ws[name][0], ws[name][2])

    b_layer = config1_step_bytes(M, 1)
    t_int, n_int = timed(layer_int_mm, seconds * 0.45)
    t_f32, n_f32 = timed(layer_fp32, seconds * 0.2)
    del ws
    # W4A16 on the same shapes: fp16 activations against the dequantised fp16 weights.
    x4 = torch.randn(M, 4096, generator=g).half()
    x14 = torch.randn(M, 14336, generator=g).half()
    deq = {name: (torch.randn(N, Kd, generator=g) * 0.05).half() for name, N, Kd in CONFIG1}

    def layer_w4a16():
        for name, N, Kd in CONFIG1:
            C.w4a16_fp32(x4 if Kd == 4096 else x14, deq[name])
    t_w4, n_w4 = timed(layer_w4a16, seconds * 0.2)
    del deq
    from specq import gen
    kc, vc, ks, vs, bt, cl = gen.paged_kv(8, [4096 + 9] * 8, 8, 128, seed=5)
    q = gen.queries(8, 9, 32, 128, seed=6)
    t_at, n_at = timed(lambda: C.paged_attention_fp32(q, kc, vc, ks, vs, bt, cl, 9), seconds * 0.15)
    b_att = attn_bytes(8, 4096 + 9, 9, 32, 8, 128, 4)
    return dict(
        value=round(b_layer / t_int / 1e9, 3), unit="GB/s", cores=int(cores), kind="port",
        cpu=model, host_cpus=int(host_cpus), affinity_cpus=int(usable), omp_num_threads=omp or None,
        sample=(f"torch._int_mm + fp32 epilogue (oracle/cpu_baseline.py) over one Llama-3-8B layer's seven "
                f"linears at M={M}: median {t_int * 1e3:.1f} ms of {n_int} reps; bytes counted as for the GPU step"),
        fp32_formula_layer_ms=round(t_f32 * 1e3, 2), fp32_formula_reps=n_f32,
        w4a16_layer_ms=round(t_w4 * 1e3, 2), w4a16_reps=n_w4,
        attention_B8_k8_ctx4096_ms=round(t_at * 1e3, 2), attention_GBps=round(b_att / t_at / 1e9, 3),
        attention_reps=n_at)


def read_traffic(key: str):
    """HBM bytes per launch of the dominant kernel ("kernel@workload") from the committed
    rocprofv3 --pmc summary (profiles/traffic.json, written by specq/profiling.py traffic)."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    e = t.get(key)
    return None if e is None else e.get("bytes_per_launch")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--B", type=int, default=8)
    ap.add_argument("--k", type=int, default=8)
    ap.add_argument("--trace", type=int, default=1000, help="steps of the plan-graph (B, k) trace")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-detail", action="store_true")
    ap.add_argument("--write-grids", metavar="DIR", help="also write the B x k grids as markdown tables into DIR")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: the verification kernels run on one GPU's share "
              "and no multi-GPU path is built; run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (libspecq.so runs on MI355X only)", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    import kernels as K

    M = args.B * (args.k + 1)
    torch.cuda.synchronize()
    w = bench_w8a8(args, K, torch)
    v, d = w["verify"], w["decode"]
    dom = w["launches"][DOMINANT]
    rnd = lambda r: {k: (round(x, 4) if isinstance(x, float) else x) for k, x in r.items()}  # noqa: E731
    detail = {"w8a8_verify": dict(M=v["M"], ms=round(v["ms"], 4), GBps=round(v["GBps"], 1)),
              "w8a8_decode": dict(M=d["M"], ms=round(d["ms"], 4), GBps=round(d["GBps"], 1)),
              "w8a8_verify_over_decode": round(v["ms"] / d["ms"], 4),
              "w8a8_verify_7_launches": rnd(w["verify_7_launches"]),
              "w8a8_decode_7_launches": rnd(w["decode_7_launches"]),
              "w8a8_verify_rowmajor_weights": rnd(w["verify_rowmajor"]),
              "w8a8_verify_rowmajor_kernel": rnd(w["verify_rowmajor_kernel"]),
              "w8a8_verify_fused_weights": rnd(w["verify_fused_weights"]),
              "w8a8_decode_fused_weights": rnd(w["decode_fused_weights"]),
              "w8a8_launch_us_M%d" % M: {k: dict(us=round(r["us"], 3), GBps=round(r["GBps"], 1),
                                                 frac=round(r["GBps"] / HBM_PEAK_GBS, 4))
                                         for k, r in w["launches"].items()},
              "w8a8_launch_us_M%d" % args.B: {k: dict(us=round(r["us"], 3), GBps=round(r["GBps"], 1))
                                              for k, r in w["launches_decode"].items()},
              "dominant_kernel": dict(name=dom["kernel"], us=round(dom["us"], 3), **dom["config"])}
    if "grid_us" in w:
        detail["w8a8_layer_grid"] = {"us": {str(b): {f"k{k}": round(v, 2) for k, v in r.items()} for b, r in w["grid_us"].items()},
                                     "ratio": {str(b): {f"k{k}": round(v, 3) for k, v in r.items()}
                                               for b, r in w["grid_ratio"].items()}}
    if not args.no_detail:
        w4 = bench_w4a16(args, K, torch)
        detail["w4a16_verify"] = {k: round(x, 4) for k, x in w4["verify"].items()}
        detail["w4a16_decode"] = {k: round(x, 4) for k, x in w4["decode"].items()}
        detail["w4a16_verify_int32_weights"] = {k: round(x, 4) for k, x in w4["verify_int32"].items()}
        detail["w4a16_verify_uint8_weights"] = {k: round(x, 4) for k, x in w4["verify_uint8"].items()}
        detail["w4a16_decode_uint8_weights"] = {k: round(x, 4) for k, x in w4["decode_uint8"].items()}
        detail["w4a16_layer_grid"] = {"us": {str(b): {f"k{k}": round(v, 2) for k, v in r.items()} for b, r in w4["grid_us"].items()},
                                      "ratio": {str(b): {f"k{k}": round(v, 3) for k, v in r.items()}
                                                for b, r in w4["grid_ratio"].items()}}
        detail["w4a16_verify_7_launches"] = {k: round(x, 4) for k, x in w4["verify_7_launches"].items()}
        detail["w4a16_decode_7_launches"] = {k: round(x, 4) for k, x in w4["decode_7_launches"].items()}
        detail["w4a16_verify_over_decode"] = round(w4["verify"]["ms"] / w4["decode"]["ms"], 4)
        detail["w4a16_verify_over_w8a8_decode"] = round(w4["verify"]["ms"] / d["ms"], 4)
        w48 = bench_w4a8(args, K, torch)
        detail["w4a8_verify"] = {k: round(x, 4) for k, x in w48["verify"].items()}
        detail["w4a8_decode"] = {k: round(x, 4) for k, x in w48["decode"].items()}
        detail["w4a8_verify_over_decode"] = round(w48["verify"]["ms"] / w48["decode"]["ms"], 4)
        attn = bench_attention(args, K, torch)
        detail["attention_B8_k8"] = {k: {kk: round(x, 4 if kk.endswith("frac") else 2) for kk, x in r.items()}
                                     for k, r in attn.items() if k.startswith("ctx")}
        # µs per launch in a graph, B down, k = 0..8 across (config 3), fused and QPP = 1.
        detail["attention_grid_us"] = {
            f"ctx{ctx}": {mode: {str(Bx): [round(g[(Bx, kk, (kk + 1) if mode == "fused" else 1)]["us"], 1)
                                           for kk in range(9)]
                                 for Bx in sorted({b for b, _, _ in g})}
                          for mode in ("fused", "qpp1")}
            for ctx, g in attn["grid"].items()}
        detail["attention_grid_hbm_frac_fused"] = {
            f"ctx{ctx}": {str(Bx): [round(g[(Bx, kk, kk + 1)]["frac"], 3) for kk in range(9)]
                          for Bx in sorted({b for b, _, _ in g})}
            for ctx, g in attn["grid"].items()}
        detail["kv_append_k8"] = {k: {kk: round(x, 2) for kk, x in r.items()}
                                  for k, r in attn.items() if k.startswith("kv_append")}
        detail["plan_graph_4layer"] = {k: round(x, 4) for k, x in bench_plan_graph(args, K, torch).items()}

    if args.write_grids and not args.no_detail:
        from specq import grids
        os.makedirs(args.write_grids, exist_ok=True)
        cmd = "python bench.py " + " ".join(sys.argv[1:])
        for name, us, ratio in (("w8a8", w["grid_us"], w["grid_ratio"]), ("w4a16", w4["grid_us"], w4["grid_ratio"])):
            with open(os.path.join(args.write_grids, f"{name}_layer_grid.md"), "w") as fh:
                fh.write(f"Command: `{cmd}`\n\n{grids.ratio_grid_md(us, ratio, name.upper())}\n")
        for ctx, g in attn["grid"].items():
            with open(os.path.join(args.write_grids, f"attention_grid_ctx{ctx}.md"), "w") as fh:
                fh.write(f"Command: `{cmd}`\n\n{grids.attention_grid_md(g, ctx)}\n")

    cpu = None
    if not args.no_cpu:
        log(f"cpu baseline (~{args.cpu_seconds:.0f} s)")
        cpu = cpu_baseline(args, M, args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": round(v["GBps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(v["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"BASELINE config 1: W8A8 over the seven Llama-3-8B linears (q, k, v, o, gate, up, "
                               f"down) x {args.layers} layers at M=B*(k+1)={M} (B={args.B}, k={args.k}); q|k|v and "
                               f"gate|up as grouped launches over separate weights (4 launches per layer); weights "
                               f"packed at load; one hipGraph replay per step",
                   "M": M, "layers": args.layers, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(dom["GBps"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["GBps"] / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic(f'{dom["kernel"]}@W8A8 grouped gate|up 2x14336x4096 M={M}'),
                     "kernel": dom["kernel"] + " (grouped gate|up launch)", "algorithmic_bytes": dom["bytes"],
                     "us_per_launch": round(dom["us"], 3)},
        "cpu_baseline": cpu,
        "detail": detail,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
