"""Build libspecq.so (the gfx950 kernels and their C ABI) in-tree with hipcc.

Usage: python build.py [--jobs N] [--quiet] [--no-diag]

Every csrc/*.hip translation unit is compiled in parallel for gfx950 and linked into
specdec-quant-triton_amd/libspecq.so.  The per-kernel register / LDS / scratch / occupancy
report of the compiler (-Rpass-analysis=kernel-resource-usage) is kept next to the library
as libspecq.resources.txt; the Python layer reads it for ck.n_regs / ck.n_spills.

The same sources compiled with -DSPECQ_DIAG give libspecq_diag.so, the measurement build:
its W8A8 and attention kernels write per-workgroup timestamps when a timeline buffer is set
(specq_diag_set_timeline) and it carries a plain streaming-read kernel
(specq_diag_stream_read).  Only specq/profiling.py loads it; the product path never does.
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


DIAG_OBJ = os.path.join(HERE, "_build_diag")
DIAG_LIB = os.path.join(HERE, "libspecq_diag.so")


def _compile(job: tuple[str, bool]) -> tuple[str, str, float]:
    src, diag = job
    obj = os.path.join(DIAG_OBJ if diag else OBJ, os.path.basename(src).replace(".hip", ".o"))
    t0 = time.time()
    flags = HIPCC_FLAGS + (["-DSPECQ_DIAG"] if diag else [])
    proc = subprocess.run([hipcc(), *flags, "-c", src, "-o", obj], capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{proc.stderr[-6000:]}")
    remarks = [ln for ln in proc.stderr.splitlines() if "remark:" in ln]
    return obj, "\n".join(remarks), time.time() - t0


def _link(objs: list[str], lib: str) -> None:
    tmp = lib + ".tmp"
    proc = subprocess.run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-o", tmp, *objs],
                          capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr[-6000:]}")
    os.replace(tmp, lib)


def build(jobs: int | None = None, quiet: bool = False, diag: bool = True) -> str:
    """Compile libspecq.so (and, unless diag=False, libspecq_diag.so); returns the product path."""
    os.makedirs(OBJ, exist_ok=True)
    if diag:
        os.makedirs(DIAG_OBJ, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    work = [(s_, False) for s_ in srcs] + ([(s_, True) for s_ in srcs] if diag else [])
    jobs = jobs or min(len(work), max(1, os.cpu_count() or 1))
    t0 = time.time()
    objs, dobjs, remarks = [], [], []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for (src, is_diag), (obj, rem, dt) in zip(work, ex.map(_compile, work)):
            (dobjs if is_diag else objs).append(obj)
            if not is_diag:
                remarks.append(rem)
            if not quiet:
                print(f"  compiled {os.path.basename(obj)}{' (diag)' if is_diag else ''} in {dt:.1f}s", flush=True)
    _link(objs, LIB)
    if diag:
        _link(dobjs, DIAG_LIB)
    with open(RES, "w") as f:
        f.write("\n".join(r for r in remarks if r) + "\n")
    if not quiet:
        print(f"built {LIB}{' and ' + DIAG_LIB if diag else ''} in {time.time() - t0:.1f}s", flush=True)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--quiet", action="store_true")
    ap.add_argument("--no-diag", action="store_true", help="skip the measurement build libspecq_diag.so")
    a = ap.parse_args()
    try:
        build(a.jobs, a.quiet, diag=not a.no_diag)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
