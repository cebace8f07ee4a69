"""Benchmark timing with an Infinity-Cache flush (replaces triton.testing.do_bench).

MI355X has a 256 MiB memory-side cache (MALL), so the flush writes 512 MiB between reps;
without it a 16-56 MiB weight would be served from the MALL instead of HBM.  Each rep is
bracketed by events on the current stream; the median is returned in milliseconds.
"""
from __future__ import annotations

import statistics

import torch

_flush = {}


def flush_cache(device=None, nbytes: int = 512 << 20) -> None:
    dev = torch.device(device or "cuda")
    key = (dev.index, nbytes)
    buf = _flush.get(key)
    if buf is None:
        buf = _flush[key] = torch.empty(nbytes // 4, dtype=torch.int32, device=dev)
    buf.zero_()


def do_bench(fn, warmup: int = 10, rep: int = 40, flush: bool = True, return_mode: str = "median"):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(rep)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(rep)]
    for i in range(rep):
        if flush:
            flush_cache()
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    ts = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    if return_mode == "median":
        return statistics.median(ts)
    if return_mode == "min":
        return min(ts)
    if return_mode == "mean":
        return sum(ts) / len(ts)
    return ts


def cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b


def next_power_of_2(n: int) -> int:
    return 1 if n <= 1 else 1 << (n - 1).bit_length()
