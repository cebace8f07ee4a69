"""rocprofv3 helpers behind the committed kernel summaries, HBM-traffic and MFMA figures.

Subcommands (run from the repository root):

  probe     the workload of the `--pmc` passes.  `--kinds` lists what to launch, each over
            enough distinct weights / KV caches that every launch reads HBM (more than the
            256 MiB Infinity Cache between two uses of one buffer):
              w8a8:M    the fused gate_up W8A8 GEMM (N=28672, K=4096, packed weights)
              w8a8g:M   gate and up (14336 x 4096 each) as one grouped launch over separate
                        packed weights (the headline's dominant launch)
              w4a16:M   the same shape in W4A16 (load-time packed INT4, group 128)
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
  mfma      reads a `--pmc SQ_INSTS_VALU_MFMA_MOPS_I8 SQ_INSTS_VALU_MFMA_MOPS_F16` run: the
            MFMA ops issued (512 per MOPS unit) against the algorithmic 2*M*N*K, and achieved
            TOP/s from an unprofiled probe's timing (`--map`) against the dense peak.
  staircase the W8A8 latency staircase over M = B*(k+1): every M = 1..300 with the library's
            tile choice and the reference's BLOCK_M in {16, 32, 64, 128} at the bucket
            boundaries, on the four config-1 shapes, each point the mean launch of a graph
            cycling over enough weight copies to stream from HBM.
  staircase-md  the markdown view of a staircase json.
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


def probe(args) -> int:
    import torch

    if PKG not in sys.path:
        sys.path.insert(0, PKG)
    import kernels as K
    from specq import gen

    torch.cuda.set_device(0)
    g = torch.Generator(device="cuda").manual_seed(1)
    N, Kd = 28672, 4096
    info = {}
    for kind in args.kinds.split(","):
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
            continue
        else:
            raise SystemExit(f"unknown probe kind {kind}")
        us = _graph_us(run, len(layers) if f[0] != "attn" else len(caches))
        for _ in range(args.reps):
            run()
        torch.cuda.synchronize()
        info[ck.name] = dict(workload=wl, us=round(us, 3), algorithmic_bytes=bytes_, ops=ops,
                             GBps=round(bytes_ / (us * 1e-6) / 1e9, 1), TOPs=round(ops / (us * 1e-6) / 1e12, 2))
        print(f"[probe] {wl}: {ck.name} {us:.2f} us/launch", flush=True)
        del run
        torch.cuda.empty_cache()
    if args.map:
        with open(args.map, "w") as fh:
            json.dump(info, fh, indent=1)
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
                    vals[_short(name)].append(v)
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
        w = wmap.get(name, {})
        tag = w.get("workload", f"M={args.M}")
        out[f"{name}@{tag}"] = dict(fetch_bytes=round(fb), write_bytes=round(wb), bytes_per_launch=round(fb + wb),
                                   launches=len(fv), algorithmic_bytes=w.get("algorithmic_bytes"))
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
                    vals[_short(r["Kernel_Name"])][r["Counter_Name"]].append(float(r["Counter_Value"]))
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
        row = {}
        for bm in (None, 16, 32, 64, 128):
            for M in (range(1, 301) if bm is None else bounds):
                def run(M=M, bm=bm):
                    for w in ws:
                        if w4:
                            K.w4a16_matmul(a[:M], w, sw, out=out[:M], BLOCK_M=bm)
                        else:
                            K.w8a8_matmul(a[:M], sa[:M], w, sw, out=out[:M], BLOCK_M=bm)
                row.setdefault(str(bm or "auto"), {})[M] = round(_graph_us(run, copies, reps=3), 2)
        res[f"{N}x{Kd}"] = row
        print(f"[staircase] {'w4a16' if w4 else 'w8a8'} {N}x{Kd} done", flush=True)
        del ws
        torch.cuda.empty_cache()
    with open(args.out, "w") as fh:
        json.dump(res, fh)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    p = sub.add_parser("sq")
    p.add_argument("dirs", nargs="+")
    p.add_argument("--map", default=None)
    p = sub.add_parser("probe")
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
    m = sub.add_parser("mfma")
    m.add_argument("dir")
    m.add_argument("--map", required=True)
    sm = sub.add_parser("staircase-md")
    sm.add_argument("json")
    c = sub.add_parser("staircase")
    c.add_argument("--out", required=True)
    c.add_argument("--kind", choices=("w8a8", "w4a16"), default="w8a8")
    args = ap.parse_args()
    return {"probe": probe, "stats": stats, "traffic": traffic, "mfma": mfma, "staircase": staircase,
            "staircase-md": staircase_md, "sq": sq}[args.cmd](args)


if __name__ == "__main__":
    sys.exit(main())
