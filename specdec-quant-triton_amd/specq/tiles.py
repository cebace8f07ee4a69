"""M-tile selection (the reference's BLOCK_M choice, bench_matmul.py:76-99, REPORT.md:81).

The reference sweeps tile configs per M and reports that BLOCK_M should follow M.  Here a
BLOCK_M of 0 hands the choice to the library, whose rule follows from measured sweeps on
MI355X: W8A8 takes one chunk of token rows covering M (up to 304 rows), so every weight byte
is read from HBM once, with the direct-activation streaming kernel for 16-row chunks and the
LDS-staged-activation kernel above; W4A16 likewise takes one chunk of up to 256 rows (the
register-stream kernel for 16 rows, LDS-staged activations above).  With a plan both cap the
chunk at 80 rows so chunks past the active M exit early.  STAIRCASE overrides it per
(kind, N, K) with the best measured BLOCK_M for each M bucket.
"""
from __future__ import annotations

# (kind, N, K) -> sorted list of (max_M, BLOCK_M); filled from measured sweeps.
STAIRCASE: dict = {}

_MAX_BM = {"w8a8": 304, "w4a16": 256}


def default_block_m(kind: str, m: int) -> int:
    """One chunk covering M rounded up to 16 rows, split evenly above the kernel's maximum."""
    cap = _MAX_BM[kind]
    rows16 = max(1, (m + 15) // 16)
    chunks = (rows16 * 16 + cap - 1) // cap
    return ((rows16 + chunks - 1) // chunks) * 16


def pick_block_m(kind: str, m: int, N: int, K: int) -> int:
    """BLOCK_M for an M of m: the STAIRCASE entry if one covers it, else 0 (library rule)."""
    table = STAIRCASE.get((kind, N, K))
    if table:
        for max_m, bm in table:
            if m <= max_m:
                return bm
    return 0
