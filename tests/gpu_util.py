"""Shared helpers for the GPU tests (imported by tests only)."""
import sys

import numpy as np
import torch


def note(msg: str) -> None:
    """Name the case about to run on the GPU (flushed, so it survives a crash)."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def bits16(t) -> np.ndarray:
    a = t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)
    return a.view(np.uint16)


def assert_bitexact_fp16(got: torch.Tensor, ref: np.ndarray, what: str) -> None:
    g = bits16(got.contiguous())
    r = np.asarray(ref, np.float16).view(np.uint16)
    if not np.array_equal(g, r):
        bad = np.argwhere(g != r)
        i = tuple(bad[0])
        raise AssertionError(f"{what}: {len(bad)} fp16 mismatches, first at {i}: "
                             f"got {got.detach().cpu().numpy()[i]} want {np.asarray(ref)[i]}")
