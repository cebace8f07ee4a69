"""Device plan buffer (the reference's `plan` tensor, bench_graphs.py:42-43, 67-69) and plan graphs.

Layout (int32[8]): [M, B, q_len, 0...].  GEMMs read plan[0]; attention is handed plan[1:]
and reads (n_seqs, q_len).  set() writes a pinned host slot and issues one asynchronous
host-to-device copy on the current stream, ordered before the graph replay that reads it.
The host slots form a ring, and a slot is rewritten only after the event recorded behind its
previous copy has completed, so back-to-back set() + replay() calls without a host sync
never overwrite a value an earlier copy has yet to read.
"""
from __future__ import annotations

import torch


class Plan:
    SLOTS = 4

    def __init__(self, device="cuda"):
        # GEMM tile policy for calls made with this plan (w8a8_matmul's plan_tiles): None for a
        # graph captured at the maximum grid, "grid" when the active M stays close to the grid.
        self.tiles = None
        self.dev = torch.zeros(8, dtype=torch.int32, device=device)
        self._host = [torch.zeros(8, dtype=torch.int32).pin_memory() for _ in range(self.SLOTS)]
        self._host_np = [h.numpy() for h in self._host]  # views of the pinned slots (cheap writes)
        self._done = [torch.cuda.Event() for _ in range(self.SLOTS)]
        self._used = [False] * self.SLOTS
        self._i = 0

    def set(self, B: int, q_len: int) -> None:
        i = self._i
        self._i = (i + 1) % self.SLOTS
        if self._used[i]:
            self._done[i].synchronize()  # the copy that last read this slot has completed
        h = self._host_np[i]
        h[0], h[1], h[2] = B * q_len, B, q_len
        self.dev.copy_(self._host[i], non_blocking=True)
        self._done[i].record()
        self._used[i] = True

    @property
    def gemm(self) -> torch.Tensor:
        return self.dev

    @property
    def attn(self) -> torch.Tensor:
        return self.dev[1:]


def b_buckets(b_max: int) -> list:
    """Sequence-count buckets of a PlanGraphSet: 1, 2, 3, 4, 6, 8, 12, 16, 24, ... (powers of two
    and 1.5 x powers of two) below b_max, then b_max.  From 2 on, consecutive buckets differ by
    at most 1.5x, so a plan-mode grid covers at most ~1.5x the sequences that are active."""
    out, p = [1], 2
    while p < b_max:
        out.append(p)
        if p + p // 2 < b_max and p >= 2:
            out.append(p + p // 2)
        p *= 2
    return sorted(set(b for b in out if b < b_max)) + [b_max]


class PlanGraphSet:
    """Plan-buffer graphs bucketed by shape (the reference's PolyGraph with K > 1 buckets,
    REPORT.md:149, 158: one graph per tile bucket instead of one frozen at the maximum).

    One graph is captured per (B bucket, q_len): the step is launched with its grids sized for
    (B bucket, q_len), so the GEMMs of a bucket run the tile the library picks for that many
    rows, while the exact (B, q_len) inside the bucket still comes from the device plan.
    `step(B_grid, ql_grid, plan)` must launch one step sized for those maxima, reading
    `plan.gemm` / `plan.attn`.  replay(B, q_len) writes the plan and replays the graph of the
    smallest bucket that holds B.  Every bucket is warmed up eagerly before any is captured,
    so workspaces reach their final size outside capture.
    """

    def __init__(self, step, b_max: int, q_lens, buckets=None, device="cuda"):
        self.plan = Plan(device)
        # The active M of a bucket's graph is at least 2/3 of its grid (buckets 1.5x apart),
        # so its GEMMs can run the tiles an eager call of the grid's M would pick.
        self.plan.tiles = "grid"
        self.buckets = sorted(buckets or b_buckets(b_max))
        if self.buckets[-1] < b_max:
            raise ValueError("the largest bucket must hold b_max")
        keys = [(bb, ql) for ql in sorted(set(q_lens)) for bb in self.buckets]
        for bb, ql in keys:
            self.plan.set(bb, ql)
            step(bb, ql, self.plan)
        torch.cuda.synchronize()
        self.graphs = {}
        for bb, ql in keys:
            self.plan.set(bb, ql)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                step(bb, ql, self.plan)
            self.graphs[(bb, ql)] = g
        torch.cuda.synchronize()

    def bucket(self, B: int) -> int:
        for bb in self.buckets:
            if B <= bb:
                return bb
        raise ValueError(f"B={B} exceeds the largest bucket {self.buckets[-1]}")

    def replay(self, B: int, q_len: int) -> None:
        g = self.graphs.get((self.bucket(B), q_len))
        if g is None:
            raise ValueError(f"no graph for q_len={q_len}")
        self.plan.set(B, q_len)
        g.replay()
