"""Seeded synthetic inputs for the benchmark configurations.

All tensors are drawn on the CPU from a torch.Generator and then copied to the target
device, so a CPU check and a GPU run see identical bytes.

  config 0/1  W8A8: A, W int8 uniform[-127, 127]; sa fp32 U[0.005, 0.02] (per token);
              sw fp32 U[0.001, 0.01] (per channel).
  config 2    W4A16: a fp16 ~N(0, 1); q int4 uniform[-8, 7] stored as q + 8, packed 8 per
              int32 along K (or the reference's uint8 layout); scales fp16 U[0.002, 0.02]
              per (channel, 128-wide K group).
  config 3    INT8 paged KV: K/V int8 uniform[-127, 127], fp32 scales U[0.005, 0.02] per
              (page, slot, kv head); randomly permuted block table over a shared pool;
              q fp16 ~N(0, 1) with q_len = k + 1 tokens appended after the context.
"""
from __future__ import annotations

import torch

LLAMA3_8B_LINEARS = {  # name: (N, K)
    "q": (4096, 4096),
    "k": (1024, 4096),
    "v": (1024, 4096),
    "o": (4096, 4096),
    "gate": (14336, 4096),
    "up": (14336, 4096),
    "down": (4096, 14336),
}
CONFIG1_SHAPES = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]


def _gen(seed: int) -> torch.Generator:
    return torch.Generator(device="cpu").manual_seed(int(seed))


def _uniform(g, shape, lo, hi, dtype=torch.float32):
    return (torch.rand(shape, generator=g, dtype=torch.float32) * (hi - lo) + lo).to(dtype)


def w8a8_inputs(M: int, N: int, K: int, seed: int = 0, device="cpu"):
    """(a int8 [M,K], w int8 [N,K], sa fp32 [M], sw fp32 [N])."""
    g = _gen(seed)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sa = _uniform(g, (M,), 0.005, 0.02)
    sw = _uniform(g, (N,), 0.001, 0.01)
    return tuple(t.to(device) for t in (a, w, sa, sw))


def w8a8_weights(N: int, K: int, seed: int = 0, device="cpu"):
    g = _gen(seed)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sw = _uniform(g, (N,), 0.001, 0.01)
    return w.to(device), sw.to(device)


def w8a8_acts(M: int, K: int, seed: int = 0, device="cpu"):
    g = _gen(seed)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    sa = _uniform(g, (M,), 0.005, 0.02)
    return a.to(device), sa.to(device)


def w8a8_epilogue_midpoints(M: int, N: int, seed: int = 0):
    """W8A8 inputs on which rounding order shows: for every channel n, the output of token row
    n % M is a case where fp16(fp32(fp32(acc * sa) * sw)) (the reference order, two
    roundings) differs from the product acc * sa * sw rounded to fp16 once.

    K = 64, W is all ones and row m of A sums to a chosen acc_m, so acc[m, n] = acc_m; the
    channel scales are drawn from U[0.001, 0.01] and kept where the two orders disagree.
    Returns (a int8 [M, 64], w int8 [N, 64], sa fp32 [M], sw fp32 [N], hit bool [M, N])."""
    import numpy as np

    rng = np.random.default_rng(seed)
    K = 64
    acc = rng.integers(64, 127 * K + 1, size=M) * rng.choice(np.array([-1, 1]), size=M)
    base = np.floor_divide(acc, K)  # in [-127, 127]; entries are base or base + 1 <= 127
    rem = acc - base * K
    a = np.repeat(base[:, None], K, axis=1)
    a += (np.arange(K)[None, :] < rem[:, None])
    sa = rng.uniform(0.005, 0.02, size=M).astype(np.float32)
    sw = np.empty(N, dtype=np.float32)
    for m in range(M):
        cols = np.arange(m, N, M)
        p1 = np.float32(acc[m]) * sa[m]
        found = np.empty(0, dtype=np.float32)
        while found.size < cols.size:
            cand = rng.uniform(0.001, 0.01, size=1 << 18).astype(np.float32)
            twice = (p1 * cand).astype(np.float16)
            once = (np.float64(p1) * cand.astype(np.float64)).astype(np.float16)
            found = np.concatenate([found, cand[twice != once]])
        sw[cols] = found[:cols.size]
    w = np.ones((N, K), dtype=np.int8)
    p1 = acc.astype(np.float32)[:, None] * sa[:, None]
    twice = (p1 * sw[None, :]).astype(np.float16)
    once = (p1.astype(np.float64) * sw[None, :].astype(np.float64)).astype(np.float16)
    return (torch.from_numpy(a.astype(np.int8)), torch.from_numpy(w), torch.from_numpy(sa),
            torch.from_numpy(sw), torch.from_numpy(twice != once))


def int4_weights(N: int, K: int, group: int = 128, seed: int = 0, device="cpu"):
    """(q unsigned nibbles uint8 [N,K] in 0..15, scales fp16 [N, K/group])."""
    g = _gen(seed)
    q = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int16) + 8
    sc = _uniform(g, (N, K // group), 0.002, 0.02, torch.float16)
    return q.to(torch.uint8).to(device), sc.to(device)


def pack_u8_reference(qu: torch.Tensor) -> torch.Tensor:
    """Reference packing (kernels.py:143-145): byte j = q[:, j] | q[:, j + K/2] << 4."""
    K = qu.shape[1]
    lo, hi = qu[:, : K // 2].to(torch.int16), qu[:, K // 2:].to(torch.int16)
    return (lo | (hi << 4)).to(torch.uint8).contiguous()


def pack_i32(qu: torch.Tensor) -> torch.Tensor:
    """int32 [N, K/8]: nibble i of word j holds k = 8j + i."""
    N, K = qu.shape
    v = qu.to(torch.int64).reshape(N, K // 8, 8)
    shifts = torch.arange(0, 32, 4, dtype=torch.int64, device=qu.device)
    w = (v << shifts).sum(-1)
    w = torch.where(w >= 2 ** 31, w - 2 ** 32, w)
    return w.to(torch.int32).contiguous()


def fp16_acts(M: int, K: int, seed: int = 0, device="cpu"):
    return torch.randn((M, K), generator=_gen(seed)).to(torch.float16).to(device)


def paged_kv(B: int, ctx_lens, H_KV: int = 8, D: int = 128, PAGE: int = 16, seed: int = 0,
             device="cpu", scale_dtype=torch.float32):
    """(kc, vc, ks, vs, block_tbl, ctx_len) with int8 K/V uniform[-127,127] and U[0.005,0.02] scales."""
    g = _gen(seed)
    pages = [(int(L) + PAGE - 1) // PAGE for L in ctx_lens]
    total = sum(pages)
    perm = torch.randperm(total, generator=g)
    bt = torch.zeros((B, max(pages)), dtype=torch.int32)
    start = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[start:start + n].to(torch.int32)
        start += n
    kc = torch.randint(-127, 128, (total, PAGE, H_KV, D), generator=g, dtype=torch.int8)
    vc = torch.randint(-127, 128, (total, PAGE, H_KV, D), generator=g, dtype=torch.int8)
    ks = _uniform(g, (total, PAGE, H_KV), 0.005, 0.02, scale_dtype)
    vs = _uniform(g, (total, PAGE, H_KV), 0.005, 0.02, scale_dtype)
    cl = torch.tensor([int(L) for L in ctx_lens], dtype=torch.int32)
    return tuple(t.to(device) for t in (kc, vc, ks, vs, bt, cl))


def queries(B: int, q_len: int, H: int = 32, D: int = 128, seed: int = 0, device="cpu"):
    return torch.randn((B, q_len, H, D), generator=_gen(seed)).to(torch.float16).to(device)
