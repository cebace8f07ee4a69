"""Device plan buffer (the reference's `plan` tensor, bench_graphs.py:42-43, 67-69).

Layout (int32[8]): [M, B, q_len, 0...].  GEMMs read plan[0]; attention is handed plan[1:]
and reads (n_seqs, q_len).  set() writes a pinned host copy and issues one asynchronous
host-to-device copy on the current stream, ordered before the graph replay that reads it.
"""
from __future__ import annotations

import torch


class Plan:
    def __init__(self, device="cuda"):
        self.dev = torch.zeros(8, dtype=torch.int32, device=device)
        self.host = torch.zeros(8, dtype=torch.int32).pin_memory()

    def set(self, B: int, q_len: int) -> None:
        self.host[0], self.host[1], self.host[2] = B * q_len, B, q_len
        self.dev.copy_(self.host, non_blocking=True)

    @property
    def gemm(self) -> torch.Tensor:
        return self.dev

    @property
    def attn(self) -> torch.Tensor:
        return self.dev[1:]
