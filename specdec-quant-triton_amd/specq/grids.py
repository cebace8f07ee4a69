"""The reference's measurement grids, timed one way: graphs of back-to-back launches.

  layer_ratio_grid   per config-1 layer (the seven Llama-3-8B linears as 4 launches: q|k|v and
                     gate|up grouped), the time t(B, k) of M = B * (k + 1) against t(B, 0), for
                     W8A8 and W4A16 -- the table of REPORT.md:71-78, bench_matmul.py:75-103.
  attention_grid     INT8 paged verification attention over B x k x QPP in {1, k + 1} at a
                     context length (bench_attention.py:16-39, REPORT.md:111-119).

Every figure is the mean launch of a captured graph whose launches read distinct weights or
KV caches (more bytes in all than the 256 MiB Infinity Cache), on the stream the kernels run
on, so each launch streams its operands from HBM and no per-call event overhead is included.
The caches of the attention grid are generated on the GPU (uniform int8 K/V, fp32 scales in
[0.005, 0.02], a random permutation block table); timing does not depend on their values.
"""
from __future__ import annotations

import torch

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20


def graph_us(fn, launches: int, reps: int = 10, warmup: int = 2) -> float:
    """Mean µs per launch of fn() (which issues `launches` launches) replayed as one graph."""
    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) * 1e3 / (reps * launches)


# The four launches of a config-1 layer: (members (N, K)); q|k|v and gate|up share their input.
LAYER_LAUNCHES = [((4096, 4096), (1024, 4096), (1024, 4096)), ((4096, 4096),),
                  ((14336, 4096), (14336, 4096)), ((4096, 14336),)]


def layer_ratio_grid(K, layers, kind: str, Bs=(1, 4, 8, 16, 32), ks=(0, 2, 4, 8), reps: int = 10):
    """{B: {k: µs per layer}} and {B: {k: t(B, k) / t(B, 0)}} for one layer of the config-1 step.

    layers: list over layers of [(w, scale) per member, in LAYER_LAUNCHES order flattened];
    kind "w8a8" (int8 weights, fp32 channel scales) or "w4a16" (INT4 weights, fp16 group
    scales).  Each point is a graph over all the layers given, its time divided by their count."""
    M_max = max(Bs) * (max(ks) + 1)
    g = torch.Generator(device="cuda").manual_seed(11)
    if kind == "w8a8":
        x4 = torch.randint(-127, 128, (M_max, 4096), dtype=torch.int8, device="cuda", generator=g)
        x14 = torch.randint(-127, 128, (M_max, 14336), dtype=torch.int8, device="cuda", generator=g)
        sa = torch.rand((M_max,), device="cuda", generator=g) * 0.015 + 0.005
    else:
        x4 = torch.randn((M_max, 4096), device="cuda", generator=g).half()
        x14 = torch.randn((M_max, 14336), device="cuda", generator=g).half()
    outs = [[torch.empty((M_max, N), dtype=torch.float16, device="cuda") for N, _ in mem] for mem in LAYER_LAUNCHES]
    us = {}
    for B in Bs:
        us[B] = {}
        for k in ks:
            M = B * (k + 1)

            def step(M=M):
                for lw in layers:
                    i = 0
                    for li, mem in enumerate(LAYER_LAUNCHES):
                        ws = lw[i:i + len(mem)]
                        i += len(mem)
                        x = x4 if mem[0][1] == 4096 else x14
                        o = [t[:M] for t in outs[li]]
                        if kind == "w8a8":
                            K.w8a8_matmul_grouped(x[:M], sa[:M], ws, outs=o, BLOCK_M=None)
                        else:
                            K.w4a16_matmul_grouped(x[:M], ws, outs=o)
            us[B][k] = graph_us(step, len(layers), reps=reps)
    ratio = {B: {k: us[B][k] / us[B][ks[0]] for k in ks} for B in Bs}
    return us, ratio


def attn_bytes(B: int, L: int, q_len: int, H: int, H_KV: int, D: int, scale_bytes: int, page: int = 16) -> int:
    """K/V int8 + their scales for every context token, q in + out (fp16), block table, lengths."""
    return (B * L * H_KV * (2 * D + 2 * scale_bytes) + 4 * B * q_len * H * D
            + 4 * B * ((L + page - 1) // page) + 4 * B)


def attn_kv_bytes(B: int, L: int, H_KV: int, D: int, scale_bytes: int) -> int:
    """The reference's bandwidth count (bench_attention.py:19): K/V and their scales only."""
    return B * L * H_KV * (2 * D + 2 * scale_bytes)


def make_caches(B: int, L: int, H_KV: int, D: int, copies: int, seed: int = 0, page: int = 16):
    """`copies` independent paged caches of B sequences of L tokens (on the GPU)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    per = (L + page - 1) // page
    out = []
    for _ in range(copies):
        pages = B * per
        kc = torch.randint(-127, 128, (pages, page, H_KV, D), dtype=torch.int8, device="cuda", generator=g)
        vc = torch.randint(-127, 128, (pages, page, H_KV, D), dtype=torch.int8, device="cuda", generator=g)
        ks = torch.rand((pages, page, H_KV), device="cuda", generator=g) * 0.015 + 0.005
        vs = torch.rand((pages, page, H_KV), device="cuda", generator=g) * 0.015 + 0.005
        bt = torch.randperm(pages, device="cuda", generator=g).to(torch.int32).view(B, per)
        cl = torch.full((B,), L, dtype=torch.int32, device="cuda")
        out.append((kc, vc, ks, vs, bt, cl))
    return out


def attention_point(K, caches, q, out, ql: int, qpp: int, reps: int = 10) -> float:
    """Mean µs per launch of paged_attention over the caches, back to back in one graph."""
    def run():
        for kc, vc, ks, vs, bt, cl in caches:
            K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=qpp, out=out)
    return graph_us(run, len(caches), reps=reps)


def attention_grid(K, ctx: int, Bs=(1, 2, 4, 8, 16, 32), ks=tuple(range(9)), H: int = 32, H_KV: int = 8,
                   D: int = 128, reps: int = 5, fused_only: bool = False):
    """{(B, k, qpp): dict(us, GBps, frac, kv_GBps)} at one context length (config 3)."""
    res = {}
    for B in Bs:
        L_max = ctx + max(ks) + 1
        per_copy = attn_bytes(B, L_max, max(ks) + 1, H, H_KV, D, 4)
        copies = max(2, -(-2 * MALL_BYTES // per_copy))
        caches = make_caches(B, L_max, H_KV, D, copies, seed=100 + B)
        g = torch.Generator(device="cuda").manual_seed(7)
        q_all = torch.randn((B, max(ks) + 1, H, D), device="cuda", generator=g).half()
        for k in ks:
            ql = k + 1
            L = ctx + ql
            cs = [(kc, vc, ks_, vs, bt, torch.full((B,), L, dtype=torch.int32, device="cuda"))
                  for kc, vc, ks_, vs, bt, _ in caches]
            q = q_all[:, :ql].contiguous()
            out = torch.zeros_like(q)
            b = attn_bytes(B, L, ql, H, H_KV, D, 4)
            for qpp in ((ql,) if fused_only or ql == 1 else (1, ql)):
                us = attention_point(K, cs, q, out, ql, qpp, reps=reps)
                gbps = b / (us * 1e-6) / 1e9
                res[(B, k, qpp)] = dict(us=us, GBps=gbps, frac=gbps / HBM_PEAK_GBS,
                                        kv_GBps=attn_kv_bytes(B, L, H_KV, D, 4) / (us * 1e-6) / 1e9)
        del caches
        torch.cuda.empty_cache()
    return res


def attention_grid_md(res: dict, ctx: int) -> str:
    """Markdown: µs per launch, fused (QPP = k + 1) and QPP = 1, B down, k across."""
    Bs = sorted({B for B, _, _ in res})
    ks = sorted({k for _, k, _ in res})
    lines = [f"### ctx {ctx}: µs per launch, fused (QPP = k + 1) / QPP = 1", "",
             "| B \\ k | " + " | ".join(str(k) for k in ks) + " |", "|---" * (len(ks) + 1) + "|"]
    for B in Bs:
        cells = []
        for k in ks:
            f = res.get((B, k, k + 1))
            o = res.get((B, k, 1))
            cells.append(f"{f['us']:.1f}" + (f" / {o['us']:.1f}" if o is not None and k > 0 else ""))
        lines.append(f"| {B} | " + " | ".join(cells) + " |")
    lines += ["", f"### ctx {ctx}: fused, share of the 8 TB/s HBM peak (algorithmic bytes / time)", "",
              "| B \\ k | " + " | ".join(str(k) for k in ks) + " |", "|---" * (len(ks) + 1) + "|"]
    for B in Bs:
        lines.append(f"| {B} | " + " | ".join(f"{100 * res[(B, k, k + 1)]['frac']:.1f} %" for k in ks) + " |")
    return "\n".join(lines)


def ratio_grid_md(us: dict, ratio: dict, kind: str) -> str:
    Bs = sorted(us)
    ks = sorted(next(iter(us.values())))
    lines = [f"### {kind}: µs per layer (4 launches) and t(B, k) / t(B, 0)", "",
             "| B \\ k | " + " | ".join(f"k={k}" for k in ks) + " |", "|---" * (len(ks) + 1) + "|"]
    for B in Bs:
        lines.append(f"| {B} | " + " | ".join(f"{us[B][k]:.1f} ({ratio[B][k]:.2f}x)" for k in ks) + " |")
    return "\n".join(lines)
