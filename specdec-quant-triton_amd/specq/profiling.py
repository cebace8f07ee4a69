"""rocprofv3 helpers behind the committed kernel summaries, HBM-traffic and MFMA figures.

Subcommands (run from the repository root):

  probe     the workload of the `--pmc` passes.  `--kinds` lists what to launch, each over
            enough distinct weights / KV caches that every launch reads HBM (more than the
            256 MiB Infinity Cache between two uses of one buffer):
              w8a8:M    the fused gate_up W8A8 GEMM (N=28672, K=4096, packed weights)
              w8a8g:M   gate and up (14336 x 4096 each) as one grouped launch over separate
                        packed weights (the headline's dominant launch)
              w8l:L:M   launch L of a config-1 layer as bench.py runs it (qkv, o, gate_up,
                        down; q|k|v and gate|up grouped over separate packed weights)
              w4a16:M   the same shape in W4A16 (load-time packed INT4, group 128)
              w4l:L:M   launch L of a config-2 layer as bench.py's W4A16 step runs it
              attn:B:k:ctx  INT8 paged verification attention (32/8 heads, D=128, fp32
                        scales, fused QPP=k+1)
              copy      torch.neg over 1 GiB of int32 (reads and writes 1 GiB): the
                        calibration kernel of FETCH_SIZE / WRITE_SIZE
            Each kind is first timed (HIP events around a graph of back-to-back launches on the
            stream they run on), and `--map` receives {kernel: workload, us per launch,
            algorithmic bytes and ops}.
  stats     a markdown table of a `--kernel-trace` run: dispatches grouped by kernel and grid,
            with mean / min duration.
  traffic   reads the FETCH_SIZE and WRITE_SIZE `--pmc` csv files of two probe runs and writes
            the HBM bytes per launch of each probed kernel, scaled by what the same counters
            read for the copy kernel (bytes = counter KiB * 1024 * copy_bytes / copy_counter).
  sq        reads one or more `--pmc` runs of SQ_* (and GRBM_GUI_ACTIVE) counters: per kernel the
            median per dispatch of each counter, instructions per wave (SQ_INSTS_* / SQ_WAVES),
            and the share of wave cycles spent issuing each instruction class
            (SQ_ACTIVE_INST_* / SQ_WAVE_CYCLES, both counted per wave in the same units).
  tiles     graph timing of explicit tilings (auto or BMxBNsS) of the w8l / w4l layer launches
  xcc       the XCD each workgroup of a launch runs on (diagnostics build), for several grids
  timeline  per-workgroup phase times of one launch of each kind (start skew, time to first
            operand data, main loop, stores), from the diagnostics build (libspecq_diag.so),
            whose W8A8 and attention kernels write s_memrealtime marks into a buffer.
  floors    streaming-read floors of the config-1 weight sizes (diagnostics build's plain
            read kernel, best over grid / waves / loads in flight) and an empty launch's cost.
  launches  one derived table per kernel instance over several `--pmc` runs of the same
            kinds: HBM bytes against the algorithmic bytes, wave-cycle shares, MFMA busy, mean
            L1->L2 read latency, L2 hit rate, TA / TD busy.
  mfma      reads a `--pmc SQ_INSTS_VALU_MFMA_MOPS_I8 SQ_INSTS_VALU_MFMA_MOPS_F16` run: the
            MFMA ops issued (512 per MOPS unit) against the algorithmic 2*M*N*K, and achieved
            TOP/s from an unprofiled probe's timing (`--map`) against the dense peak.
  staircase the W8A8 latency staircase over M = B*(k+1): every M = 1..300 with the library's
            tile choice and the reference's BLOCK_M in {16, 32, 64, 128} at the bucket
            boundaries, on the four config-1 shapes, each point the mean launch of a graph
            cycling over enough weight copies to stream from HBM.
  staircase-md  the markdown view of a staircase json.
  tune      the measured tile table: every 16-row step of M on the config-1 launch shapes,
            the automatic tiling against the reference's BLOCK_M and the other channel blocks.
  tune-emit the C++ table (csrc/tuned_tiles.hpp) of a tune json; tune-md its markdown view.
"""
from __future__ import annotations

import argparse
import collections
import csv
import glob
import json
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
COPY_TAG = "at::native"  # the calibration copy is torch's elementwise kernel


def _short(name: str) -> str:
    name = name.split("(")[0]
    return name[5:] if name.startswith("void ") else name


def _key(name: str, grid) -> str:
    """Kernel instance key of the maps and tables: short name and grid (the same template runs
    several launches, told apart by their workgroup counts)."""
    return f"{_short(name)} [{grid}]" if grid else _short(name)


def _row_grid(r):
    """Workgroups of a rocprofv3 csv row (kernel trace: per-axis columns; counters: totals)."""
    if "Grid_Size_X" in r:
        wgs = 1
        for ax in "XYZ":
            wgs *= int(r.get(f"Grid_Size_{ax}", 1) or 1) // max(1, int(r.get(f"Workgroup_Size_{ax}", 1) or 1))
        return wgs
    try:
        return int(r["Grid_Size"]) // max(1, int(r["Workgroup_Size"]))
    except (KeyError, ValueError):
        return None


def _graph_us(fn, launches: int, reps: int = 10) -> float:
    """Mean µs per launch of fn() (which issues `launches` launches) replayed as one graph."""
    import torch

    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * launches)


def _apply_options(args) -> None:
    """Library options given as --set name=value (specq_set_option)."""
    from specq import _lib
    for kv in getattr(args, "set", []) or []:
        name, val = kv.split("=", 1)
        _lib.set_option(name, int(val))


def _make_kind(kind: str, args, K, gen, g, torch):
    """Inputs and a run() for one probe kind (see the module docstring): dict(run, launches,
    ck, workload, bytes, ops), or None for the copy kind, which runs at once."""
    N, Kd = 28672, 4096
    f = kind.split(":")
    if f[0] == "w8a8":
        M = int(f[1])
        layers = []
        for _ in range(args.layers):
            w = torch.randint(-127, 128, (N, Kd), dtype=torch.int8, device="cuda", generator=g)
            layers.append((K.pack_weight_int8(w), torch.rand((N,), device="cuda", generator=g) * 0.009 + 0.001))
            del w
        a = torch.randint(-127, 128, (M, Kd), dtype=torch.int8, device="cuda", generator=g)
        sa = torch.rand((M,), device="cuda", generator=g) * 0.015 + 0.005
        out = torch.empty((M, N), dtype=torch.float16, device="cuda")

        def run(layers=layers, a=a, sa=sa, out=out):
            for w, sw in layers:
                K.w8a8_matmul(a, sa, w, sw, out=out, BLOCK_M=None)
        _, ck = K.w8a8_matmul(a, sa, *layers[0], out=out, BLOCK_M=None)
        bytes_, ops = N * Kd + M * Kd + 4 * M + 4 * N + 2 * M * N, 2 * M * N * Kd
        wl = f"W8A8 N={N} K={Kd} M={M}"
    elif f[0] == "w8a8g":
        # The headline's dominant launch: gate and up (14336 x 4096 each, separate packed
        # weights) as one grouped launch.
        M, Ng = int(f[1]), 14336
        layers = []
        for _ in range(args.layers):
            pair = []
            for _ in range(2):
                w = torch.randint(-127, 128, (Ng, Kd), dtype=torch.int8, device="cuda", generator=g)
                pair.append((K.pack_weight_int8(w), torch.rand((Ng,), device="cuda", generator=g) * 0.009 + 0.001))
                del w
            layers.append(pair)
        a = torch.randint(-127, 128, (M, Kd), dtype=torch.int8, device="cuda", generator=g)
        sa = torch.rand((M,), device="cuda", generator=g) * 0.015 + 0.005
        outs = [torch.empty((M, Ng), dtype=torch.float16, device="cuda") for _ in range(2)]

        def run(layers=layers, a=a, sa=sa, outs=outs):
            for pair in layers:
                K.w8a8_matmul_grouped(a, sa, pair, outs=outs, BLOCK_M=None)
        _, ck = K.w8a8_matmul_grouped(a, sa, layers[0], outs=outs, BLOCK_M=None)
        bytes_ = 2 * (Ng * Kd + 4 * Ng + 2 * M * Ng) + M * Kd + 4 * M
        ops = 2 * 2 * M * Ng * Kd
        wl = f"W8A8 grouped gate|up 2x{Ng}x{Kd} M={M}"
    elif f[0] == "w8l":
        # One of the four launches of a config-1 layer (bench.py's step): qkv and gate_up
        # grouped over their separate packed weights, o and down alone.
        lname, M = f[1], int(f[2])
        shapes = {"qkv": [(4096, 4096), (1024, 4096), (1024, 4096)], "o": [(4096, 4096)],
                  "gate_up": [(14336, 4096), (14336, 4096)], "down": [(4096, 14336)]}[lname]
        Kl = shapes[0][1]
        layers = []
        for _ in range(args.layers):
            mem = []
            for Ng, _k in shapes:
                w = torch.randint(-127, 128, (Ng, Kl), dtype=torch.int8, device="cuda", generator=g)
                mem.append((K.pack_weight_int8(w), torch.rand((Ng,), device="cuda", generator=g) * 0.009 + 0.001))
                del w
            layers.append(mem)
        a = torch.randint(-127, 128, (M, Kl), dtype=torch.int8, device="cuda", generator=g)
        sa = torch.rand((M,), device="cuda", generator=g) * 0.015 + 0.005
        outs = [torch.empty((M, Ng), dtype=torch.float16, device="cuda") for Ng, _k in shapes]

        bm, bn, sk = getattr(args, "tile", None) or (None, None, 0)

        def run(layers=layers, a=a, sa=sa, outs=outs):
            for mem in layers:
                K.w8a8_matmul_grouped(a, sa, mem, outs=outs, BLOCK_M=bm, BLOCK_N=bn, split_k=sk)
        _, ck = K.w8a8_matmul_grouped(a, sa, layers[0], outs=outs, BLOCK_M=bm, BLOCK_N=bn, split_k=sk)
        bytes_ = sum(Ng * Kl + 4 * Ng + 2 * M * Ng for Ng, _k in shapes) + M * Kl + 4 * M
        ops = sum(2 * M * Ng * Kl for Ng, _k in shapes)
        wl = f"W8A8 {lname} ({'+'.join(f'{Ng}x{Kl}' for Ng, _k in shapes)}) M={M}"
    elif f[0] == "w4l":
        # One of the four launches of a config-2 layer (bench.py's W4A16 step): qkv and gate_up
        # grouped over their separate packed INT4 weights, o and down alone.
        lname, M = f[1], int(f[2])
        shapes = {"qkv": [(4096, 4096), (1024, 4096), (1024, 4096)], "o": [(4096, 4096)],
                  "gate_up": [(14336, 4096), (14336, 4096)], "down": [(4096, 14336)]}[lname]
        Kl = shapes[0][1]
        layers = []
        for _ in range(args.layers):
            mem = []
            for Ng, _k in shapes:
                wp = torch.randint(-2 ** 31, 2 ** 31 - 1, (Ng, Kl // 8), dtype=torch.int32, device="cuda", generator=g)
                sc = (torch.rand((Ng, Kl // 128), device="cuda", generator=g) * 0.018 + 0.002).half()
                mem.append((K.pack_weight_int4(wp), sc))
                del wp
            layers.append(mem)
        x = torch.randn((M, Kl), device="cuda", generator=g).half()
        outs = [torch.empty((M, Ng), dtype=torch.float16, device="cuda") for Ng, _k in shapes]

        bm, bn, sk = getattr(args, "tile", None) or (None, None, 0)

        def run(layers=layers, x=x, outs=outs):
            for mem in layers:
                K.w4a16_matmul_grouped(x, mem, outs=outs, BLOCK_M=bm, BLOCK_N=bn, split_k=sk)
        _, ck = K.w4a16_matmul_grouped(x, layers[0], outs=outs, BLOCK_M=bm, BLOCK_N=bn, split_k=sk)
        bytes_ = sum(Ng * Kl // 2 + 2 * Ng * (Kl // 128) + 2 * M * Ng for Ng, _k in shapes) + 2 * M * Kl
        ops = sum(2 * M * Ng * Kl for Ng, _k in shapes)
        wl = f"W4A16 {lname} ({'+'.join(f'{Ng}x{Kl}' for Ng, _k in shapes)}) M={M}"
    elif f[0] == "w4a16":
        M = int(f[1])
        layers = []
        for _ in range(args.layers):
            wp = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, Kd // 8), dtype=torch.int32, device="cuda", generator=g)
            sc = (torch.rand((N, Kd // 128), device="cuda", generator=g) * 0.018 + 0.002).half()
            layers.append((K.pack_weight_int4(wp), sc))
            del wp
        x = torch.randn((M, Kd), device="cuda", generator=g).half()
        out = torch.empty((M, N), dtype=torch.float16, device="cuda")

        def run(layers=layers, x=x, out=out):
            for wp, sc in layers:
                K.w4a16_matmul(x, wp, sc, out=out, BLOCK_M=None)
        _, ck = K.w4a16_matmul(x, *layers[0], out=out, BLOCK_M=None)
        bytes_ = N * Kd // 2 + 2 * N * (Kd // 128) + 2 * M * Kd + 2 * M * N
        ops = 2 * M * N * Kd
        wl = f"W4A16 N={N} K={Kd} M={M} group 128"
    elif f[0] == "attn":
        B, k, ctx = int(f[1]), int(f[2]), int(f[3])
        ql, H, H_KV, D = k + 1, 32, 8, 128
        L = ctx + ql
        caches = [[t.cuda() for t in gen.paged_kv(B, [L] * B, H_KV, D, seed=50 + i)] for i in range(args.layers)]
        q = gen.queries(B, ql, H, D, seed=6).cuda()
        out = torch.zeros_like(q)

        def run(caches=caches, q=q, out=out, ql=ql):
            for kc, vc, ks, vs, bt, cl in caches:
                K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=ql, out=out)
        _, ck = K.paged_attention(q, *caches[0], ql, QPP=ql, out=out)
        pages = (L + 15) // 16
        bytes_ = B * L * H_KV * (2 * D + 8) + 4 * B * ql * H * D + 4 * B * pages + 4 * B
        ops = 4 * B * H * D * ql * L
        wl = f"attention B={B} k={k} ctx={ctx} fused"
    elif f[0] == "copy":
        n = (args.copy_mib << 20) // 4
        src = torch.randint(-2 ** 30, 2 ** 30, (n,), dtype=torch.int32, device="cuda", generator=g)
        dst = torch.empty_like(src)
        for _ in range(args.reps):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        print(f"[probe] copy {args.copy_mib} MiB x {args.reps}", flush=True)
        return None
    else:
        raise SystemExit(f"unknown probe kind {kind}")
    launches = len(layers) if f[0] != "attn" else len(caches)
    return dict(run=run, launches=launches, ck=ck, workload=wl, bytes=bytes_, ops=ops)

def probe(args) -> int:
    import torch

    if PKG not in sys.path:
        sys.path.insert(0, PKG)
    import kernels as K
    from specq import gen

    torch.cuda.set_device(0)
    _apply_options(args)
    g = torch.Generator(device="cuda").manual_seed(1)
    info = {}
    for kind in args.kinds.split(","):
        kd = _make_kind(kind, args, K, gen, g, torch)
        if kd is None:
            continue
        run, ck, wl, bytes_, ops = kd["run"], kd["ck"], kd["workload"], kd["bytes"], kd["ops"]
        us = _graph_us(run, kd["launches"])
        for _ in range(args.reps):
            run()
        torch.cuda.synchronize()
        info[_key(ck.name, ck.config.get("grid"))] = dict(workload=wl, us=round(us, 3), algorithmic_bytes=bytes_, ops=ops,
                             GBps=round(bytes_ / (us * 1e-6) / 1e9, 1), TOPs=round(ops / (us * 1e-6) / 1e12, 2))
        print(f"[probe] {wl}: {ck.name} {us:.2f} us/launch", flush=True)
        del run, kd
        torch.cuda.empty_cache()
    if args.map:
        with open(args.map, "w") as fh:
            json.dump(info, fh, indent=1)
    return 0


# Timestamp marks the diagnostics build writes (csrc/common.hpp tl_mark), per kernel family.
_TL_PHASES = {
    "gemm": [("start skew", None, 0), ("to first data", 0, 1), ("main loop", 1, 2), ("stores issued", 2, 3),
             ("stores done", 3, 4), ("split-K: partials acknowledged", 3, 5), ("split-K: arrival count back", 5, 6),
             ("split-K (last): partials read and summed", 6, 7), ("split-K (last): outputs stored", 7, 4),
             ("whole workgroup", 0, 4)],
    "attn": [("start skew", None, 0), ("page ids + Q", 0, 1), ("to first chunk", 1, 2), ("chunk loop (wave 0)", 2, 3),
             ("wait for the other waves", 3, 7), ("wave merge", 7, 4), ("hand-off / store", 4, 6),
             ("split: partials acknowledged", 4, 5), ("whole workgroup", 0, 6)],
}


def _pcts(x):
    import numpy as np

    return [float(np.percentile(x, q)) for q in (10, 50, 90)] + [float(np.max(x))]


def tiles(args) -> int:
    """Graph timing of explicit tilings of config-1/2 layer launches (kinds w8l:L:M, w4l:L:M):
    each --tiles entry is "auto" or BMxBNsS (BLOCK_M x BLOCK_N, split_k S), every entry timed
    twice (the faster kept) over the kind's distinct weight copies."""
    import torch

    if PKG not in sys.path:
        sys.path.insert(0, PKG)
    import kernels as K
    from specq import gen

    torch.cuda.set_device(0)
    _apply_options(args)
    g = torch.Generator(device="cuda").manual_seed(1)
    out = ["| launch | tile (BLOCK_M x BLOCK_N, split) | kernel [grid] | µs per launch |", "|---|---|---|---|"]
    for kind in args.kinds.split(","):
        for t in args.tiles.split(","):
            if t == "auto":
                args.tile = None
            else:
                bmbn, sk = t.split("s")
                bm, bn = bmbn.split("x")
                args.tile = (int(bm), int(bn), int(sk))
            kd = _make_kind(kind, args, K, gen, g, torch)
            us = min(_graph_us(kd["run"], kd["launches"]) for _ in range(2))
            ck = kd["ck"]
            cfg = ck.config
            tile = f"{cfg.get('block_m')} x {cfg.get('block_n')}, {cfg.get('split_k')}" + (" (auto)" if t == "auto" else "")
            out.append(f"| {kd['workload']} | {tile} | `{_key(ck.name, cfg.get('grid'))}` | {us:.2f} |")
            print(out[-1], flush=True)
            del kd
            torch.cuda.empty_cache()
    text = "\n".join(out)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text + "\n")
    return 0


def xcc(args) -> int:
    """Which XCD each workgroup of a launch runs on (diagnostics build, hardware register
    XCC_ID), against the round-robin deal blockIdx.x mod (number of XCDs), for several grids."""
    import torch

    if PKG not in sys.path:
        sys.path.insert(0, PKG)
    from specq import _lib
    _lib.use_diag()
    torch.cuda.set_device(0)
    grids = [int(x) for x in args.grids.split(",")]
    buf = torch.zeros(max(grids), dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    out = ["| workgroups x threads | launches | XCDs seen | workgroups per XCD | workgroups not on XCD blockIdx mod XCDs |",
           "|---|---|---|---|---|"]
    for n in grids:
        for threads in (256, 512):
            counts, bad, nx = torch.zeros(16, dtype=torch.int64), 0, 0
            for _ in range(args.reps):
                buf.fill_(-1)
                _lib.call("specq_diag_xcc_ids", buf.data_ptr(), n, threads, stream)
                ids = buf[:n].cpu().to(torch.int64)
                nx = max(nx, int(ids.max()) + 1)
                counts += torch.bincount(ids, minlength=16)[:16]
                bad += int((ids != torch.arange(n) % nx).sum())
            out.append(f"| {n} x {threads} | {args.reps} | {nx} | {' / '.join(str(int(v)) for v in counts[:nx])} | {bad} |")
            print(out[-1], flush=True)
    text = "\n".join(out)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text + "\n")
    return 0


def timeline(args) -> int:
    """Per-workgroup phases of one launch of each probe kind, from the diagnostics build's
    s_memrealtime marks (100 MHz): the kind's graph of back-to-back launches over distinct
    weights / caches is replayed and the marks of its last launch are read."""
    import numpy as np
    import torch

    if PKG not in sys.path:
        sys.path.insert(0, PKG)
    from specq import _lib
    _lib.use_diag()
    import kernels as K
    from specq import gen

    torch.cuda.set_device(0)
    _apply_options(args)
    g = torch.Generator(device="cuda").manual_seed(1)
    cap = 1 << 16
    marks = 16  # kTlMarks of csrc/common.hpp
    tl = torch.zeros(cap * marks, dtype=torch.int64, device="cuda")
    _lib.call("specq_diag_set_timeline", tl.data_ptr(), cap)
    out = [f"Per-workgroup timelines (diagnostics build, s_memrealtime at 100 MHz); µs, p10 / p50 / p90 / max "
           f"over the workgroups of the last launch of a graph of back-to-back launches."]
    for kind in args.kinds.split(","):
        kd = _make_kind(kind, args, K, gen, g, torch)
        if kd is None:
            continue
        us = _graph_us(kd["run"], kd["launches"])
        tl.zero_()
        torch.cuda.synchronize()
        # One more replay of the same graph shape: the marks left are those of its last launch.
        kd["run"]()
        torch.cuda.synchronize()
        t = tl.view(cap, marks).cpu().numpy().astype(np.int64)
        ck = kd["ck"]
        grid = int(ck.config.get("grid") or 0)
        fam = "attn" if kind.startswith("attn") else "gemm"
        rows = t[: grid if grid else cap]
        rows = rows[rows[:, 0] != 0]
        # A mark some workgroup index wrote in an earlier launch of the sequence and not in the
        # last one (e.g. the split-K finish of a tile whose last arrival was another split)
        # predates that launch's start mark: drop it.
        rows[:, 1:] = np.where(rows[:, 1:] >= rows[:, :1], rows[:, 1:], 0)
        if not len(rows):
            out.append(f"\n### {kd['workload']}: no marks (kernel without timestamps)")
            continue
        t0 = rows[:, 0].min()
        last = 6 if fam == "attn" else 4
        worked = rows[rows[:, last] != 0]
        span = (worked[:, last].max() - t0) / 100.0 if len(worked) else float("nan")
        out.append(f"\n### {kd['workload']}: `{_key(ck.name, grid)}`\n")
        out.append(f"{len(rows)} workgroups started, {len(worked)} ran to the end; first start to last end "
                   f"{span:.2f} µs; graph launch {us:.2f} µs\n")
        out.append("| phase | p10 | p50 | p90 | max |")
        out.append("|---|---|---|---|---|")
        for name, a, b in _TL_PHASES[fam]:
            sel = worked if b != 0 else rows
            if a is None:
                d = (sel[:, b] - t0) / 100.0
            else:
                ok = (sel[:, a] != 0) & (sel[:, b] != 0)
                d = (sel[ok, b] - sel[ok, a]) / 100.0
            if len(d):
                out.append(f"| {name} | " + " | ".join(f"{v:.2f}" for v in _pcts(d)) + " |")
        if fam == "attn":
            # Spread of the eight waves' loop ends within a workgroup (marks 8..15).
            wl = worked[:, 8:16]
            ok = (wl != 0).all(axis=1)
            if ok.any():
                spread = (wl[ok].max(axis=1) - wl[ok].min(axis=1)) / 100.0
                first = (wl[ok].min(axis=1) - worked[ok, 2]) / 100.0
                out.append("| loop end, last wave - first wave | " + " | ".join(f"{v:.2f}" for v in _pcts(spread)) + " |")
                out.append("| first chunk to the first wave's loop end | " + " | ".join(f"{v:.2f}" for v in _pcts(first)) + " |")
        del kd
        torch.cuda.empty_cache()
    _lib.call("specq_diag_set_timeline", None, 0)
    text = "\n".join(out)
    print(text)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text + "\n")
    return 0


def floors(args) -> int:
    """Streaming-read floors (diagnostics build): a plain read of N bytes (16-byte loads,
    XOR-reduced) timed as a graph of back-to-back launches over distinct buffers (>= 512 MiB in
    all, so every launch reads HBM), best over workgroup count x waves x loads in flight; and
    the cost of an empty launch in the same graph form."""
    import torch

    if PKG not in sys.path:
        sys.path.insert(0, PKG)
    from specq import _lib
    _lib.use_diag()
    torch.cuda.set_device(0)
    sink = torch.zeros(65536, dtype=torch.int32, device="cuda")
    stream = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    out = ["| bytes | what | best µs | TB/s | workgroups | waves | 1 KB loads in flight per wave |",
           "|---|---|---|---|---|---|---|"]
    tiny = torch.zeros(4, dtype=torch.int32, device="cuda")
    us = _graph_us(lambda: [_lib.call("specq_diag_stream_read", tiny.data_ptr(), 16, 1, 4, 2, sink.data_ptr(),
                                      stream()) for _ in range(64)], 64, reps=20)
    out.append(f"| 16 | empty launch (one workgroup) | {us:.2f} | | 1 | 4 | |")
    for spec in args.sizes.split(","):
        name, nb = spec.split(":")
        nb = int(nb)
        nbuf = max(2, -(-(512 << 20) // nb) + 1)
        bufs = [torch.empty(nb, dtype=torch.int8, device="cuda").random_(-128, 127) for _ in range(nbuf)]
        best = None
        for wgs in (256, 512, 1024, 2048):
            for waves in (4, 8):
                for unroll in (2, 4, 8, 16):
                    def run(wgs=wgs, waves=waves, unroll=unroll):
                        for b in bufs:
                            _lib.call("specq_diag_stream_read", b.data_ptr(), nb, wgs, waves, unroll,
                                      sink.data_ptr(), stream())
                    t = _graph_us(run, nbuf, reps=5)
                    if best is None or t < best[0]:
                        best = (t, wgs, waves, unroll)
        t, wgs, waves, unroll = best
        out.append(f"| {nb} | {name} | {t:.2f} | {nb / (t * 1e-6) / 1e12:.2f} | {wgs} | {waves} | {unroll} |")
        print(out[-1], flush=True)
        del bufs
        torch.cuda.empty_cache()
    text = "\n".join(out)
    print(text)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text + "\n")
    return 0


def stats(args) -> int:
    rows = collections.defaultdict(list)
    for f in glob.glob(os.path.join(args.dir, "**", "*kernel_trace.csv"), recursive=True):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                name = r["Kernel_Name"]
                if args.filter and args.filter not in name:
                    continue
                wgs = 1
                for ax in "XYZ":
                    wgs *= int(r.get(f"Grid_Size_{ax}", 1) or 1) // max(1, int(r.get(f"Workgroup_Size_{ax}", 1) or 1))
                dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
                rows[(_short(name), wgs)].append(dur)
    table = sorted(rows.items(), key=lambda kv: -sum(kv[1]))[: args.top]
    print("| kernel | grid (WGs) | calls | avg µs | min µs | total ms |")
    print("|---|---|---|---|---|---|")
    for (name, wgs), d in table:
        print(f"| `{name}` | {wgs} | {len(d)} | {statistics.mean(d):.2f} | {min(d):.2f} | {sum(d) / 1e3:.2f} |")
    return 0


def _counter(dirname: str, counter: str):
    """{kernel short name: [counter value per dispatch]} and the copy kernel's values."""
    vals, copy = collections.defaultdict(list), []
    files = glob.glob(os.path.join(dirname, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {dirname}")
    for f in files:
        with open(f) as fh:
            for r in csv.DictReader(fh):
                if r["Counter_Name"] != counter:
                    continue
                name, v = r["Kernel_Name"], float(r["Counter_Value"])
                if "specq::" in name:
                    vals[_key(name, _row_grid(r))].append(v)
                elif COPY_TAG in name and "neg" in name.lower():
                    copy.append(v)
    return vals, copy


def traffic(args) -> int:
    copy_bytes = 2 * (args.copy_mib << 20)  # read + write of the copy; each counter sees half
    wmap = json.load(open(args.map)) if args.map else {}
    out = {}
    if args.merge and os.path.exists(args.merge):
        out = {k: v for k, v in json.load(open(args.merge)).items() if k != "_calibration"}
    fetch, cf = _counter(args.fetch, "FETCH_SIZE")
    write, cw = _counter(args.write, "WRITE_SIZE")
    if not cf or not cw:
        raise SystemExit("calibration copy kernel not found in the counter files")
    f_scale = (copy_bytes / 2) / (statistics.median(cf) * 1024)
    w_scale = (copy_bytes / 2) / (statistics.median(cw) * 1024)
    for name, fv in fetch.items():
        wv = write.get(name, [0.0])
        # The first launch of a run may find its buffer in the Infinity Cache; the median is
        # the steady state of a launch whose operands come from HBM.
        fb = statistics.median(fv) * 1024 * f_scale
        wb = statistics.median(wv) * 1024 * w_scale
        # Counter rows carry the grid (" [N]"); probe maps may key a kernel without it.
        base, _, grid = name.partition(" [")
        w = wmap.get(name) or wmap.get(base, {})
        tag = w.get("workload", f"M={args.M}")
        out[f"{base}@{tag}"] = dict(fetch_bytes=round(fb), write_bytes=round(wb), bytes_per_launch=round(fb + wb),
                                   launches=len(fv), algorithmic_bytes=w.get("algorithmic_bytes"),
                                   grid=int(grid.rstrip("]")) if grid else None)
    meta = dict(copy_mib=args.copy_mib, fetch_scale=round(f_scale, 4), write_scale=round(w_scale, 4),
                copy_fetch_kib=statistics.median(cf), copy_write_kib=statistics.median(cw))
    res = {"_calibration": meta, **out}
    text = json.dumps(res, indent=1, sort_keys=True)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text + "\n")
    print(text)
    return 0


def _all_counters(dirname: str):
    """{kernel short name: {counter: [value per dispatch]}} of every specq kernel in a run."""
    vals = collections.defaultdict(lambda: collections.defaultdict(list))
    files = glob.glob(os.path.join(dirname, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {dirname}")
    for f in files:
        with open(f) as fh:
            for r in csv.DictReader(fh):
                if "specq::" in r["Kernel_Name"]:
                    vals[_key(r["Kernel_Name"], _row_grid(r))][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return vals


def sq(args) -> int:
    """Per-kernel SQ counter medians and per-wave ratios from one or more --pmc runs."""
    merged = collections.defaultdict(dict)
    for d in args.dirs:
        for name, cs in _all_counters(d).items():
            for c, v in cs.items():
                merged[name][c] = statistics.median(v)
    wmap = json.load(open(args.map)) if args.map else {}
    for name, cs in sorted(merged.items()):
        wl = wmap.get(name, {}).get("workload", "")
        print(f"\n### `{name}` {wl}\n")
        print("| counter | median per dispatch | per wave |")
        print("|---|---|---|")
        waves = cs.get("SQ_WAVES")
        for c in sorted(cs):
            pw = f"{cs[c] / waves:.1f}" if waves and c.startswith("SQ_INSTS") else ""
            print(f"| {c} | {cs[c]:.0f} | {pw} |")
        wc = cs.get("SQ_WAVE_CYCLES")
        if wc:
            shares = [(c[len("SQ_ACTIVE_INST_"):], cs[c] / wc) for c in sorted(cs) if c.startswith("SQ_ACTIVE_INST_")]
            shares += [(c[len("SQ_"):], cs[c] / wc) for c in ("SQ_WAIT_ANY", "SQ_WAIT_INST_ANY") if c in cs]
            print("\nshare of wave cycles: " + ", ".join(f"{k} {100 * v:.1f} %" for k, v in shares))
    return 0


def launches(args) -> int:
    """One derived table over several --pmc runs of the same probe kinds (and the probe's map):
    per kernel instance its launch time, HBM bytes (FETCH_SIZE / WRITE_SIZE scaled by the copy
    kernel) against the algorithmic bytes, where its waves spend their cycles, the mean L1->L2
    read latency and the TA / TD / L2 figures.  Counter units: SQ_* cycle counters are wave
    quad-cycles summed over waves; GRBM_GUI_ACTIVE is summed over the 8 XCDs, so one XCD's
    cycles are GRBM_GUI_ACTIVE / 8; TA_*, TD_*, TCP_* sum over the 256 CUs."""
    merged = collections.defaultdict(dict)
    copy = {}
    for d in args.dirs:
        files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        per = collections.defaultdict(lambda: collections.defaultdict(list))
        for f in files:
            with open(f) as fh:
                for r in csv.DictReader(fh):
                    name, c, v = r["Kernel_Name"], r["Counter_Name"], float(r["Counter_Value"])
                    if "specq::" in name:
                        per[_key(name, _row_grid(r))][c].append(v)
                    elif COPY_TAG in name and "neg" in name.lower():
                        copy.setdefault(c, []).append(v)
        for k, cs in per.items():
            for c, v in cs.items():
                merged[k][c] = statistics.median(v)
    wmap = json.load(open(args.map)) if args.map else {}
    half = (args.copy_mib << 20)  # the copy reads and writes this many bytes
    scale = {c: half / (statistics.median(v) * 1024) for c, v in copy.items() if c in ("FETCH_SIZE", "WRITE_SIZE")}

    def g(cs, c):
        return cs.get(c)

    rows = []
    for k in sorted(merged, key=lambda x: wmap.get(x, {}).get("workload", x)):
        cs, w = merged[k], wmap.get(k, {})
        grbm = g(cs, "GRBM_GUI_ACTIVE")
        wc = g(cs, "SQ_WAVE_CYCLES")
        r = dict(key=k, workload=w.get("workload", ""), us=w.get("us"), alg=w.get("algorithmic_bytes"))
        if "FETCH_SIZE" in cs and "FETCH_SIZE" in scale:
            r["fetch"] = cs["FETCH_SIZE"] * 1024 * scale["FETCH_SIZE"]
        if "WRITE_SIZE" in cs and "WRITE_SIZE" in scale:
            r["write"] = cs["WRITE_SIZE"] * 1024 * scale["WRITE_SIZE"]
        if wc:
            for c in ("SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_VMEM", "SQ_ACTIVE_INST_LDS", "SQ_ACTIVE_INST_SCA",
                      "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY"):
                if c in cs:
                    r[c] = cs[c] / wc
        if g(cs, "TCP_TCC_READ_REQ_sum"):
            r["l2_lat"] = cs.get("TCP_TCC_READ_REQ_LATENCY_sum", 0) / cs["TCP_TCC_READ_REQ_sum"]
            r["l2_req"] = cs["TCP_TCC_READ_REQ_sum"]
        if grbm:
            xcd = grbm / 8
            for c in ("TA_TA_BUSY_sum", "TA_DATA_STALLED_BY_TC_CYCLES_sum", "TD_TD_BUSY_sum", "TD_TC_STALL_sum",
                      "TCP_PENDING_STALL_CYCLES_sum", "TCP_TCP_TA_DATA_STALL_CYCLES_sum"):
                if c in cs:
                    r[c] = cs[c] / (256 * xcd)
            if "SQ_VALU_MFMA_BUSY_CYCLES" in cs:
                r["mfma_busy"] = cs["SQ_VALU_MFMA_BUSY_CYCLES"] / (1024 * xcd)
            if "SQ_LDS_BANK_CONFLICT" in cs:
                r["lds_conflict"] = cs["SQ_LDS_BANK_CONFLICT"] / (256 * xcd)
        if "TCC_HIT_sum" in cs and "TCC_MISS_sum" in cs:
            r["l2_hit"] = cs["TCC_HIT_sum"] / max(1.0, cs["TCC_HIT_sum"] + cs["TCC_MISS_sum"])
        if "SQ_WAVES" in cs:
            for c in ("SQ_INSTS_VMEM_RD", "SQ_INSTS_LDS", "SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_SALU"):
                if c in cs:
                    r["per_wave_" + c[len("SQ_INSTS_"):]] = cs[c] / cs["SQ_WAVES"]
        rows.append(r)

    def pct(x):
        return "" if x is None else f"{100 * x:.1f}"

    def num(x, f="{:.0f}"):
        return "" if x is None else f.format(x)
    print("| kernel [grid] | workload | µs | alg MB | fetch MB | write MB | VALU % | VMEM % | LDS % | WAIT_ANY % "
          "| WAIT_INST % | MFMA busy % | L2 read lat (clk) | L2 hit % | TA busy % | TA stall by TC % "
          "| TD busy % | TCP pending % |")
    print("|---" * 18 + "|")
    for r in rows:
        print(f"| `{r['key']}` | {r['workload']} | {num(r['us'], '{:.2f}')} | {num(r['alg'] and r['alg'] / 1e6, '{:.2f}')} "
              f"| {num(r.get('fetch') and r['fetch'] / 1e6, '{:.2f}')} | {num(r.get('write') and r['write'] / 1e6, '{:.2f}')} "
              f"| {pct(r.get('SQ_ACTIVE_INST_VALU'))} | {pct(r.get('SQ_ACTIVE_INST_VMEM'))} | {pct(r.get('SQ_ACTIVE_INST_LDS'))} "
              f"| {pct(r.get('SQ_WAIT_ANY'))} | {pct(r.get('SQ_WAIT_INST_ANY'))} | {pct(r.get('mfma_busy'))} "
              f"| {num(r.get('l2_lat'))} | {pct(r.get('l2_hit'))} | {pct(r.get('TA_TA_BUSY_sum'))} "
              f"| {pct(r.get('TA_DATA_STALLED_BY_TC_CYCLES_sum'))} | {pct(r.get('TD_TD_BUSY_sum'))} "
              f"| {pct(r.get('TCP_PENDING_STALL_CYCLES_sum'))} |")
    extra = [c for c in ("per_wave_VMEM_RD", "per_wave_LDS", "per_wave_VALU", "per_wave_MFMA", "per_wave_SALU")
             if any(c in r for r in rows)]
    if extra:
        print("\n| kernel [grid] | " + " | ".join(c.replace("per_wave_", "") + " / wave" for c in extra) + " |")
        print("|---" * (len(extra) + 1) + "|")
        for r in rows:
            print(f"| `{r['key']}` | " + " | ".join(num(r.get(c), "{:.1f}") for c in extra) + " |")
    return 0


def mfma(args) -> int:
    """Issued MFMA ops (from the MOPS counters) against 2*M*N*K, and achieved TOP/s per kernel."""
    wmap = json.load(open(args.map))
    mi8, _ = _counter(args.dir, "SQ_INSTS_VALU_MFMA_MOPS_I8")
    mf16, _ = _counter(args.dir, "SQ_INSTS_VALU_MFMA_MOPS_F16")
    print("| kernel | workload | MFMA ops issued / 2MNK | achieved TOP/s | dense peak | % of peak |")
    print("|---|---|---|---|---|---|")
    for name, w in wmap.items():
        if name not in mi8 and name not in mf16:
            continue
        i8 = statistics.median(mi8.get(name, [0])) * 512
        f16 = statistics.median(mf16.get(name, [0])) * 512
        issued = max(i8, f16)
        peak = 5000.0 if i8 >= f16 else 2500.0
        print(f"| `{name}` | {w['workload']} | {issued / w['ops']:.3f} | {w['TOPs']:.1f} | "
              f"{peak:.0f} | {100 * w['TOPs'] / peak:.1f} |")
    return 0


def staircase_md(args) -> int:
    """Markdown view of a `staircase` json: the library's tile choice against fixed BLOCK_M."""
    res = json.load(open(args.json))
    for shape, row in res.items():
        auto = row["auto"]
        fixed = [k for k in ("16", "32", "64", "128") if k in row]
        print(f"\n### N x K = {shape}\n")
        print("| M | auto µs | " + " | ".join(f"BLOCK_M={k} µs" for k in fixed) + " | best fixed / auto |")
        print("|---|---|" + "---|" * len(fixed) + "---|")
        for M in row[fixed[0]]:
            vals = [row[k][M] for k in fixed]
            a = auto.get(M)
            print(f"| {M} | {a} | " + " | ".join(str(v) for v in vals) + f" | {min(vals) / a:.2f} |")
        ms = sorted(int(m) for m in auto)
        print(f"\nauto, every M = 1..300: min {min(auto.values())} µs, max {max(auto.values())} µs; "
              f"M=1 {auto[str(ms[0])]} µs, M=300 {auto[str(ms[-1])]} µs")
    return 0


def staircase(args) -> int:
    """W8A8 (or, with --kind w4a16, W4A16) latency over M on the config-1 shapes: the library's
    tile choice at every M = 1..300 and fixed BLOCK_M at the staircase's edges."""
    import torch

    if PKG not in sys.path:
        sys.path.insert(0, PKG)
    import kernels as K

    torch.cuda.set_device(0)
    g = torch.Generator(device="cuda").manual_seed(3)
    shapes = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]
    bounds = [1, 8, 16, 17, 24, 32, 33, 48, 64, 65, 72, 96, 128, 129, 144, 160, 192, 256, 288, 300]
    res = {}
    w4 = getattr(args, "kind", "w8a8") == "w4a16"
    for N, Kd in shapes:
        wbytes = N * Kd // 2 if w4 else N * Kd
        copies = max(4, -(-600 * (1 << 20) // wbytes))  # > 2x the Infinity Cache per cycle
        if w4:  # INT4 weights packed at load, fp16 group scales and activations (config 2)
            ws = [K.pack_weight_int4(torch.randint(-2 ** 31, 2 ** 31 - 1, (N, Kd // 8), dtype=torch.int32,
                                                   device="cuda", generator=g)) for _ in range(copies)]
            sw = (torch.rand((N, Kd // 128), device="cuda", generator=g) * 0.018 + 0.002).half()
            a = torch.randn((300, Kd), device="cuda", generator=g).half()
        else:
            ws = [K.pack_weight_int8(torch.randint(-127, 128, (N, Kd), dtype=torch.int8, device="cuda", generator=g))
                  for _ in range(copies)]
            sw = torch.rand((N,), device="cuda", generator=g) * 0.009 + 0.001
            a = torch.randint(-127, 128, (300, Kd), dtype=torch.int8, device="cuda", generator=g)
        sa = torch.rand((300,), device="cuda", generator=g) * 0.015 + 0.005
        out = torch.empty((300, N), dtype=torch.float16, device="cuda")
        timed = {}
        row = {}
        kid = 1 if w4 else 0
        for bm in (None, 16, 32, 64, 128):
            for M in (range(1, 301) if bm is None else bounds):
                # A fixed BLOCK_M that resolves to the same tiling as the automatic choice is the
                # same launch: it reuses that timing instead of a second, noisy one.
                cfg = K.KernelInfo(kid, 2 if w4 else 1, M, N, Kd, bm or 0, 0, 4, 0).config
                key = (M, cfg["block_m"], cfg["block_n"], cfg["split_k"])
                if key in timed:
                    row.setdefault(str(bm or "auto"), {})[M] = timed[key]
                    continue

                def run(M=M, bm=bm):
                    for w in ws:
                        if w4:
                            K.w4a16_matmul(a[:M], w, sw, out=out[:M], BLOCK_M=bm)
                        else:
                            K.w8a8_matmul(a[:M], sa[:M], w, sw, out=out[:M], BLOCK_M=bm)
                t = round(min(_graph_us(run, copies, reps=3) for _ in range(2 if bm is None and M not in bounds else 3)), 2)
                timed[key] = t
                row.setdefault(str(bm or "auto"), {})[M] = t
            print(f"[staircase] {N}x{Kd} BLOCK_M={bm or 'auto'} done", flush=True)
        res[f"{N}x{Kd}"] = row
        print(f"[staircase] {'w4a16' if w4 else 'w8a8'} {N}x{Kd} done", flush=True)
        del ws
        torch.cuda.empty_cache()
    with open(args.out, "w") as fh:
        json.dump(res, fh)
    return 0


# The config-1 launch shapes the measured tile table covers: the four N x K of one GEMM and
# the two grouped launches (q|k|v, gate|up) by their members.
TUNE_SHAPES = {"4096x4096": [(4096, 4096)], "1024x4096": [(1024, 4096)], "14336x4096": [(14336, 4096)],
               "4096x14336": [(4096, 14336)], "6144x4096": [(4096, 4096), (1024, 4096), (1024, 4096)],
               "28672x4096": [(14336, 4096), (14336, 4096)]}


def tune(args) -> int:
    """Measured tile table: for each config-1 launch shape and each step of M (M = 1..8, 9..16,
    then 16 rows at a time up to 300; timed at the step's first and last M, the mean of the
    two), the mean launch of every candidate
    tiling -- the automatic one, the reference's four BLOCK_M with the library's channel block
    and split for that depth, and the automatic depth with every channel block -- each as a graph
    cycling over enough weight copies to stream from HBM.  Writes {kind: {shape: {rows16:
    dict(best=[BLOCK_M, BLOCK_N, split_k], us, auto=[...], auto_us)}}} for `tune-emit`."""
    import torch

    if PKG not in sys.path:
        sys.path.insert(0, PKG)
    import kernels as K
    from specq import _lib

    torch.cuda.set_device(0)
    # "auto" below is the cost model's own choice, with any existing table switched off.
    _lib.set_option("tuned_tiles", 0)
    g = torch.Generator(device="cuda").manual_seed(17)
    res = {}
    for kind in args.kinds.split(","):
        w4 = kind == "w4a16"
        res[kind] = {}
        for sname, members in TUNE_SHAPES.items():
            Kd = members[0][1]
            N_total = sum(N for N, _ in members)
            wbytes = sum(N * Kd for N, _ in members) // (2 if w4 else 1)
            copies = max(4, -(-600 * (1 << 20) // wbytes))
            weights = []
            for _ in range(copies):
                mem = []
                for N, _k in members:
                    if w4:
                        wp = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, Kd // 8), dtype=torch.int32, device="cuda",
                                           generator=g)
                        sc = (torch.rand((N, Kd // 128), device="cuda", generator=g) * 0.018 + 0.002).half()
                        mem.append((K.pack_weight_int4(wp), sc))
                    else:
                        w = torch.randint(-127, 128, (N, Kd), dtype=torch.int8, device="cuda", generator=g)
                        mem.append((K.pack_weight_int8(w), torch.rand((N,), device="cuda", generator=g) * 0.009 + 0.001))
                weights.append(mem)
            if w4:
                a = torch.randn((300, Kd), device="cuda", generator=g).half()
            else:
                a = torch.randint(-127, 128, (300, Kd), dtype=torch.int8, device="cuda", generator=g)
            sa = torch.rand((300,), device="cuda", generator=g) * 0.015 + 0.005
            outs = [torch.empty((300, N), dtype=torch.float16, device="cuda") for N, _ in members]
            kid = 1 if w4 else 0
            bns = (64, 128) if w4 else (16, 32, 64, 128)
            # A grouped W4A16 launch runs its members' common split count: resolve tiles with it.
            gsk = K.w4a16_group_split([N for N, _ in members], Kd) if w4 else 0
            table = {}
            lo_step, hi_step = (int(x) for x in getattr(args, "steps", "0-19").split("-"))
            for r in range(lo_step, hi_step + 1):
                # Step 0 is M = 1..8, step 1 M = 9..16, step r >= 2 the 16 rows up to 16 r.  Every
                # M of a step runs its tile: time the candidates at both ends of the step and rank
                # them by the mean.
                lo, M = (1, 8) if r == 0 else ((9, 16) if r == 1 else (16 * (r - 1) + 1, min(16 * r, 300)))
                Ms = sorted({lo, M})
                auto = K.KernelInfo(kid, 2 if w4 else 1, M, N_total, Kd, 0, 0, 4, gsk).config
                reqs = [(None, None)] + [(bm, None) for bm in (16, 32, 64, 128)] + [(auto["block_m"], bn) for bn in bns]
                if w4 and M > 144:
                    reqs.append((160, None))  # the deepest W4A16 tile: M up to 320 in two chunks
                cands = []
                for bm, bn in reqs:
                    c = K.KernelInfo(kid, 2 if w4 else 1, M, N_total, Kd, bm or 0, bn or 0, 4, gsk).config
                    t = (c["block_m"], c["block_n"], c["split_k"])
                    if t not in cands:
                        cands.append(t)
                times, per_m = {}, {}
                for bm, bn, sk in cands:
                    tot = 0.0
                    per_m[(bm, bn, sk)] = {}
                    for Mx in Ms:
                        def run(bm=bm, bn=bn, sk=sk, M=Mx):
                            for mem in weights:
                                o = [x[:M] for x in outs]
                                if w4:
                                    K.w4a16_matmul_grouped(a[:M], mem, outs=o, BLOCK_M=bm, BLOCK_N=bn,
                                                           split_k=sk if len(members) == 1 else 0)
                                else:
                                    K.w8a8_matmul_grouped(a[:M], sa[:M], mem, outs=o, BLOCK_M=bm, BLOCK_N=bn,
                                                          split_k=sk)
                        t = min(_graph_us(run, copies, reps=4), _graph_us(run, copies, reps=4))
                        per_m[(bm, bn, sk)][Mx] = t
                        tot += t
                    times[(bm, bn, sk)] = tot / len(Ms)
                at = (auto["block_m"], auto["block_n"], auto["split_k"])
                # The tile whose worst ratio to the fastest at each measured M of the step is
                # smallest; the automatic tile unless that worst ratio is measurably better (2 %).
                fastest = {Mx: min(per_m[c][Mx] for c in cands) for Mx in Ms}
                regret = {c: max(per_m[c][Mx] / fastest[Mx] for Mx in Ms) for c in cands}
                best = min(cands, key=lambda c: (regret[c], times[c]))
                if regret[best] > regret[at] - 0.02:
                    best = at
                print(f"[tune] {kind} {sname} step {r}: {list(best)}", flush=True)
                table[r] = dict(best=list(best), us=round(times[best], 3), auto=list(at), auto_us=round(times[at], 3),
                                regret=round(regret[best], 4), auto_regret=round(regret[at], 4),
                                candidates={f"{b}x{n}s{k}": {str(m): round(t, 3) for m, t in per_m[(b, n, k)].items()}
                                            for (b, n, k) in cands})
            res[kind][sname] = table
            print(f"[tune] {kind} {sname}: " + ", ".join(f"{r}:{table[r]['best']}" for r in table), flush=True)
            del weights
            torch.cuda.empty_cache()
    with open(args.out, "w") as fh:
        json.dump(res, fh, indent=1)
    return 0


def tune_emit(args) -> int:
    """The C++ table (csrc/tuned_tiles.hpp) of a `tune` json: one entry per kind, launch shape
    and rows16 whose measured best differs from the cost model's choice or not, so the library
    runs the measured tile for every step of M on these shapes."""
    res = json.load(open(args.json))
    lines = ["// Measured tile choices for the Llama-3-8B launch shapes on MI355X (256 CUs).",
             "// Generated by `specq/profiling.py tune-emit` from a `specq/profiling.py tune` run (every",
             "// step of M on each shape -- step 0 is M = 1..8, step 1 M = 9..16, step r >= 2 the 16 rows up",
             "// to 16 r (M <= 300) -- the automatic tiling, the reference's four BLOCK_M and every channel",
             "// block at the automatic depth, each timed at the step's first and last M as graphs of",
             "// back-to-back launches streaming their weights from HBM); the fastest on average, or the",
             "// model's own choice within 2 %.",
             "// kind 0 = W8A8 (BLOCK_M, BLOCK_N, split_k), kind 1 = W4A16 (BLOCK_M, BLOCK_N; its split",
             "// count follows from N and K).  N is the launch's total width (grouped launches: the sum).",
             "#pragma once", "", "namespace specq {", "",
             "struct TunedTile {", "  int kind, N, K, step, block_m, block_n, split_k;", "};", "",
             "constexpr TunedTile kTunedTiles[] = {"]
    n = 0
    for kind, shapes in res.items():
        kid = 1 if kind == "w4a16" else 0
        for sname, table in shapes.items():
            N, Kd = (int(x) for x in sname.split("x"))
            for r in sorted(table, key=int):
                bm, bn, sk = table[r]["best"]
                lines.append(f"    {{{kid}, {N}, {Kd}, {int(r)}, {bm}, {bn}, {sk}}},")
                n += 1
    lines += ["};", f"constexpr int kTunedTileCount = {n};", "", "}  // namespace specq", ""]
    with open(args.out, "w") as fh:
        fh.write("\n".join(lines))
    print(f"{n} entries -> {args.out}")
    return 0


def tune_md(args) -> int:
    """Markdown view of a `tune` json: per shape and rows16 the model's tile, the measured best
    and the gain."""
    res = json.load(open(args.json))
    for kind, shapes in res.items():
        for sname, table in shapes.items():
            print(f"\n### {kind} {sname}\n")
            print("| step (M range) | model tile (BM x BN, split) | µs | measured best | µs | model / best "
                  "| worst ratio to the fastest: model / chosen |")
            print("|---|---|---|---|---|---|---|")
            for r in sorted(table, key=int):
                e = table[r]
                fmt = lambda t: f"{t[0]} x {t[1]}, {t[2]}"  # noqa: E731
                ri = int(r)
                rng = "1-8" if ri == 0 else ("9-16" if ri == 1 else f"{16 * ri - 15}-{min(16 * ri, 300)}")
                print(f"| {r} ({rng}) | {fmt(e['auto'])} | {e['auto_us']:.2f} | {fmt(e['best'])} | "
                      f"{e['us']:.2f} | {e['auto_us'] / e['us']:.3f} | {e.get('auto_regret', 0):.3f} / "
                      f"{e.get('regret', 0):.3f} |")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    p = sub.add_parser("sq")
    p.add_argument("dirs", nargs="+")
    p.add_argument("--map", default=None)
    p = sub.add_parser("probe")
    p.add_argument("--set", action="append", default=[], help="library option name=value (repeatable)")
    p.add_argument("--kinds", default="w8a8:72,copy")
    p.add_argument("--layers", type=int, default=16)
    p.add_argument("--reps", type=int, default=2)
    p.add_argument("--copy-mib", type=int, default=1024)
    p.add_argument("--map")
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("--filter", default="specq::")
    s.add_argument("--top", type=int, default=30)
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--M", type=int, default=72)
    t.add_argument("--copy-mib", type=int, default=1024)
    t.add_argument("--map")
    t.add_argument("--merge", help="existing traffic json whose entries are kept")
    t.add_argument("--out")
    xp = sub.add_parser("xcc")
    xp.add_argument("--grids", default="8,64,192,224,256,384,448,1000,4096,8192")
    xp.add_argument("--reps", type=int, default=5)
    xp.add_argument("--out")
    tl = sub.add_parser("tiles")
    tl.add_argument("--set", action="append", default=[], help="library option name=value (repeatable)")
    tl.add_argument("--kinds", required=True)
    tl.add_argument("--tiles", required=True, help="comma list of auto or BMxBNsS")
    tl.add_argument("--layers", type=int, default=8)
    tl.add_argument("--copy-mib", type=int, default=1024)
    tl.add_argument("--out")
    tp = sub.add_parser("timeline")
    tp.add_argument("--set", action="append", default=[], help="library option name=value (repeatable)")
    tp.add_argument("--kinds", required=True)
    tp.add_argument("--layers", type=int, default=8)
    tp.add_argument("--reps", type=int, default=1)
    tp.add_argument("--copy-mib", type=int, default=1024)
    tp.add_argument("--out")
    fp = sub.add_parser("floors")
    fp.add_argument("--sizes", default="o:16777216,qkv:25165824,down:58720256,gate_up:117440512")
    fp.add_argument("--out")
    lp = sub.add_parser("launches")
    lp.add_argument("dirs", nargs="+")
    lp.add_argument("--map", default=None)
    lp.add_argument("--copy-mib", type=int, default=1024)
    m = sub.add_parser("mfma")
    m.add_argument("dir")
    m.add_argument("--map", required=True)
    sm = sub.add_parser("staircase-md")
    sm.add_argument("json")
    tu = sub.add_parser("tune")
    tu.add_argument("--kinds", default="w8a8,w4a16")
    tu.add_argument("--steps", default="0-19", help="steps of M to tune, lo-hi (step r >= 2: M up to 16 r)")
    tu.add_argument("--out", required=True)
    te = sub.add_parser("tune-emit")
    te.add_argument("json")
    te.add_argument("--out", required=True)
    tm = sub.add_parser("tune-md")
    tm.add_argument("json")
    c = sub.add_parser("staircase")
    c.add_argument("--out", required=True)
    c.add_argument("--kind", choices=("w8a8", "w4a16"), default="w8a8")
    args = ap.parse_args()
    return {"probe": probe, "stats": stats, "traffic": traffic, "mfma": mfma, "staircase": staircase,
            "staircase-md": staircase_md, "sq": sq, "launches": launches, "timeline": timeline, "tiles": tiles, "xcc": xcc,
            "floors": floors, "tune": tune, "tune-emit": tune_emit, "tune-md": tune_md}[args.cmd](args)


if __name__ == "__main__":
    sys.exit(main())
