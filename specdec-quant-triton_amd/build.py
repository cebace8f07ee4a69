"""Build libspecq.so (the gfx950 kernels and their C ABI) in-tree with hipcc.

Usage: python build.py [--jobs N] [--quiet]

Every csrc/*.hip translation unit is compiled in parallel for gfx950 and linked into
specdec-quant-triton_amd/libspecq.so.  The per-kernel register / LDS / scratch / occupancy
report of the compiler (-Rpass-analysis=kernel-resource-usage) is kept next to the library
as libspecq.resources.txt; the Python layer reads it for ck.n_regs / ck.n_spills.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libspecq.so")
RES = os.path.join(HERE, "libspecq.resources.txt")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed FP32 VALU ops are kept out of every kernel on this platform.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Rpass-analysis=kernel-resource-usage",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(src: str) -> tuple[str, str, float]:
    obj = os.path.join(OBJ, os.path.basename(src).replace(".hip", ".o"))
    t0 = time.time()
    proc = subprocess.run([hipcc(), *HIPCC_FLAGS, "-c", src, "-o", obj], capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{proc.stderr[-6000:]}")
    remarks = [ln for ln in proc.stderr.splitlines() if "remark:" in ln]
    return obj, "\n".join(remarks), time.time() - t0


def build(jobs: int | None = None, quiet: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    jobs = jobs or min(len(srcs), max(1, os.cpu_count() or 1))
    t0 = time.time()
    objs, remarks = [], []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for obj, rem, dt in ex.map(_compile, srcs):
            objs.append(obj)
            remarks.append(rem)
            if not quiet:
                print(f"  compiled {os.path.basename(obj)} in {dt:.1f}s", flush=True)
    tmp = LIB + ".tmp"
    proc = subprocess.run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-o", tmp, *objs],
                          capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr[-6000:]}")
    os.replace(tmp, LIB)
    with open(RES, "w") as f:
        f.write("\n".join(r for r in remarks if r) + "\n")
    if not quiet:
        print(f"built {LIB} in {time.time() - t0:.1f}s", flush=True)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--quiet", action="store_true")
    a = ap.parse_args()
    try:
        build(a.jobs, a.quiet)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
