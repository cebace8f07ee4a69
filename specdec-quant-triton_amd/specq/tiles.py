"""BLOCK_M selection (the reference's M-tile choice, bench_matmul.py:76-99, REPORT.md:81).

The reference sweeps tile configs per M and reports that BLOCK_M should follow M
(16 for M <= 16, 32 up to 32, 64 up to 64, 128 above).  On MI355X the kernels keep a whole
M-chunk of up to 320 (W8A8) or 256 (W4A16) rows in registers while the weights stream
through once, so the default is one chunk covering M rounded up to 16 rows; STAIRCASE can
override it per (kind, N, K) with the best measured value for each M bucket.
"""
from __future__ import annotations

# (kind, N, K) -> sorted list of (max_M, BLOCK_M); filled from measured sweeps.
STAIRCASE: dict = {}

_MAX_BM = {"w8a8": 320, "w4a16": 256}


def default_block_m(kind: str, m: int) -> int:
    cap = _MAX_BM[kind]
    rows16 = max(1, (m + 15) // 16)
    chunks = (rows16 * 16 + cap - 1) // cap
    return ((rows16 + chunks - 1) // chunks) * 16


def pick_block_m(kind: str, m: int, N: int, K: int) -> int:
    table = STAIRCASE.get((kind, N, K))
    if table:
        for max_m, bm in table:
            if m <= max_m:
                return bm
    return default_block_m(kind, m)
