"""rocprofv3 helpers behind the committed kernel summaries and the HBM-traffic figure.

Subcommands (run from the repository root):

  probe   the workload of the `--pmc` passes: the dominant W8A8 kernel (fused gate_up shape,
          N=28672, K=4096, packed weights) at M, launched once per layer over `--layers`
          layers so every launch reads its weight from HBM, then a plain elementwise copy
          (torch.neg on int32, reads and writes `--copy-mib` MiB) as the calibration kernel.
  stats   a markdown table of a `--kernel-trace` run: dispatches grouped by kernel and grid,
          with mean / min duration.
  traffic reads the FETCH_SIZE and WRITE_SIZE `--pmc` csv files of two probe runs and writes
          the HBM bytes per launch of each probed kernel, scaled by what the same counters
          read for the copy kernel (bytes = counter KiB * 1024 * copy_bytes / copy_counter).
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


def probe(args) -> int:
    import torch

    if PKG not in sys.path:
        sys.path.insert(0, PKG)
    import kernels as K

    torch.cuda.set_device(0)
    g = torch.Generator(device="cuda").manual_seed(1)
    N, Kd, M = 28672, 4096, args.M
    layers = []
    for _ in range(args.layers):
        w = torch.randint(-127, 128, (N, Kd), dtype=torch.int8, device="cuda", generator=g)
        sw = torch.rand((N,), device="cuda", generator=g) * 0.009 + 0.001
        layers.append((K.pack_weight_int8(w), sw))
        del w
    a = torch.randint(-127, 128, (M, Kd), dtype=torch.int8, device="cuda", generator=g)
    sa = torch.rand((M,), device="cuda", generator=g) * 0.015 + 0.005
    out = torch.empty((M, N), dtype=torch.float16, device="cuda")
    for _ in range(args.reps):
        for w, sw in layers:
            K.w8a8_matmul(a, sa, w, sw, out=out, BLOCK_M=None)
    n = (args.copy_mib << 20) // 4
    src = torch.randint(-2 ** 30, 2 ** 30, (n,), dtype=torch.int32, device="cuda", generator=g)
    dst = torch.empty_like(src)
    for _ in range(args.reps):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(f"[probe] w8a8 N={N} K={Kd} M={M}: {args.reps * args.layers} launches; "
          f"copy {args.copy_mib} MiB x {args.reps}", flush=True)
    return 0


def stats(args) -> int:
    rows = collections.defaultdict(list)
    for f in glob.glob(os.path.join(args.dir, "**", "*kernel_trace.csv"), recursive=True):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                name = r["Kernel_Name"]
                if args.filter and args.filter not in name:
                    continue
                wgs = int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"]))
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
    out = {}
    fetch, cf = _counter(args.fetch, "FETCH_SIZE")
    write, cw = _counter(args.write, "WRITE_SIZE")
    if not cf or not cw:
        raise SystemExit("calibration copy kernel not found in the counter files")
    f_scale = (copy_bytes / 2) / (statistics.median(cf) * 1024)
    w_scale = (copy_bytes / 2) / (statistics.median(cw) * 1024)
    for name, fv in fetch.items():
        wv = write.get(name, [0.0])
        # The first launch of a run may find its weight in the Infinity Cache; the median is
        # the steady state of a launch whose weight comes from HBM.
        fb = statistics.median(fv) * 1024 * f_scale
        wb = statistics.median(wv) * 1024 * w_scale
        out[f"{name}@M={args.M}"] = dict(fetch_bytes=round(fb), write_bytes=round(wb),
                                         bytes_per_launch=round(fb + wb), launches=len(fv))
    meta = dict(copy_mib=args.copy_mib, fetch_scale=round(f_scale, 4), write_scale=round(w_scale, 4),
                copy_fetch_kib=statistics.median(cf), copy_write_kib=statistics.median(cw))
    res = {"_calibration": meta, **out}
    text = json.dumps(res, indent=1, sort_keys=True)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text + "\n")
    print(text)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    p = sub.add_parser("probe")
    p.add_argument("--M", type=int, default=72)
    p.add_argument("--layers", type=int, default=16)
    p.add_argument("--reps", type=int, default=2)
    p.add_argument("--copy-mib", type=int, default=1024)
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("--filter", default="specq::")
    s.add_argument("--top", type=int, default=30)
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--M", type=int, default=72)
    t.add_argument("--copy-mib", type=int, default=1024)
    t.add_argument("--out")
    args = ap.parse_args()
    return {"probe": probe, "stats": stats, "traffic": traffic}[args.cmd](args)


if __name__ == "__main__":
    sys.exit(main())
