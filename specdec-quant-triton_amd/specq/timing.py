"""Benchmark timing with an Infinity-Cache flush (replaces triton.testing.do_bench).

MI355X has a 256 MiB memory-side cache (MALL) behind 8 x 4 MiB of L2, so the flush touches
512 MiB between reps; without it a 16-70 MiB operand would be served from the MALL instead
of HBM.  triton.testing.do_bench flushes by zeroing a buffer.  On this GPU that leaves up to
about 290 MiB of dirty lines in the caches, and the next kernel pays for writing them back to
HBM while it reads its own data: at B=8, k=8, ctx 4096 the paged attention measured 49.2 us
after a zeroing flush, against 35.5 us after a flush that reads last, and 33.2 us with no
flush.  The default flush therefore zeroes the buffer and then reads it back (a sum into one
scalar), so the timed kernel starts with cold, clean caches, the state the reference's flush
produced on its 2 MiB L2.  `do_bench` keeps triton.testing.do_bench's zeroing-only flush as
its default (`flush="dirty"`), so the reference's bench scripts run through this drop-in
measure what they measured before; `flush="clean"` asks for the zero-then-read flush.
Each rep is bracketed by events on the current stream; the median is returned in
milliseconds.  An empty kernel timed this way takes about 6.4 us (the events' own launch
latency), a floor every figure from here carries.
"""
from __future__ import annotations

import statistics

import torch

_flush = {}


def flush_cache(device=None, nbytes: int = 512 << 20, mode: str = "clean") -> None:
    """Evict the caches: zero `nbytes`, then (mode "clean") read them back into one scalar."""
    if mode not in ("clean", "dirty"):
        raise ValueError(f"flush mode must be 'clean' or 'dirty', not {mode!r}")
    dev = torch.device(device or "cuda")
    key = (dev.index, nbytes)
    bufs = _flush.get(key)
    if bufs is None:
        bufs = _flush[key] = (torch.empty(nbytes // 4, dtype=torch.int32, device=dev),
                              torch.zeros((), dtype=torch.int64, device=dev))
    buf, sink = bufs
    buf.zero_()
    if mode == "clean":
        torch.sum(buf, dim=0, dtype=torch.int64, out=sink)


def do_bench(fn, warmup: int = 10, rep: int = 40, flush="dirty", return_mode: str = "median"):
    """Median (or min / mean / all) event time of fn in ms; flush: "dirty" (zeroing only, as
    triton.testing.do_bench), "clean" (zero, then read back) or False."""
    if flush is True:
        flush = "dirty"
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(rep)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(rep)]
    for i in range(rep):
        if flush:
            flush_cache(mode=flush)
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
