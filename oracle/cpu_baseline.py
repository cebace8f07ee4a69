"""The reference's PyTorch formulas on the host CPU -- TEST INFRASTRUCTURE ONLY.

These are the computations the CPU baseline leg of bench.py times on the GPU box's host
cores, beside the MI355X kernels.  They restate, in torch on the CPU, the formulas the
reference itself uses to check its kernels:

  w8a8_int_mm         exact INT32 product through torch._int_mm, then the fp32 epilogue in
                      the kernel's order, fp16((fp32(acc) * sa) * sw)   (kernels.py:51-55)
  w8a8_fp32_formula   the reference test's float formula (a.float() @ w.float().T) * sa * sw
                                                                        (correctness.py:37)
  w4a16_fp32          x.float() @ deq.float().T, cast to fp16           (correctness.py:76)
  paged_attention_fp32  dense fp32 verification attention over the paged INT8 cache
                                                                        (kernels.py:289-309)

Only tests/ and bench.py's cpu_baseline leg import this module.  Each function is checked
against the numpy oracle (oracle/oracle.py, itself pinned by closed forms, brute force and
library routines) in tests/test_oracle.py.
"""
from __future__ import annotations

import math

import torch

__all__ = ["w8a8_int_mm", "w8a8_fp32_formula", "w4a16_fp32", "paged_attention_fp32"]


def w8a8_int_mm(a: torch.Tensor, sa: torch.Tensor, w_t: torch.Tensor, sw: torch.Tensor) -> torch.Tensor:
    """fp16((fp32(a @ w_t) * sa[:, None]) * sw[None, :]) with an exact INT32 product.

    a int8 [M, K]; w_t int8 [K, N] (the weight transposed once, as torch._int_mm takes it);
    sa fp32 [M]; sw fp32 [N].  Bit-identical to the kernel's output (kernels.py:51-55).
    """
    acc = torch._int_mm(a, w_t)
    return ((acc.float() * sa[:, None]) * sw[None, :]).half()


def w8a8_fp32_formula(a: torch.Tensor, sa: torch.Tensor, w: torch.Tensor, sw: torch.Tensor) -> torch.Tensor:
    """The reference test's reference, (a.float() @ w.float().T) * sa * sw in fp32 (correctness.py:37).

    Exact in its product only while every partial sum stays below 2**24 (127 * 127 * K < 2**24
    holds for K <= 1040); above that the fp32 sums round.
    """
    return (a.float() @ w.float().T) * sa[:, None] * sw[None, :]


def w4a16_fp32(x: torch.Tensor, deq: torch.Tensor) -> torch.Tensor:
    """fp16(x.float() @ deq.float().T): the reference's W4A16 check (correctness.py:76)."""
    return (x.float() @ deq.float().T).half()


def paged_attention_fp32(q, kc, vc, ks, vs, block_tbl, ctx_len, q_len: int) -> torch.Tensor:
    """Dense fp32 attention over the paged INT8 cache, causal over the last q_len positions.

    For sequence b with L = ctx_len[b] (which counts the q_len query tokens), query i sits at
    position L - q_len + i and sees positions 0..L - q_len + i; K and V are dequantised with
    their per-(page, slot, head) scales and each KV head serves H / H_KV query heads
    (kernels.py:289-309).  Returns fp16 [B, QLMAX, H, D] with zeros past q_len.
    """
    B, _, H, D = q.shape
    PAGE, H_KV = kc.shape[1], kc.shape[2]
    G = H // H_KV
    out = torch.zeros(q.shape, dtype=torch.float32)
    for b in range(B):
        L = int(ctx_len[b])
        pos = torch.arange(L)
        page = block_tbl[b, pos // PAGE].long()
        slot = pos % PAGE
        k = kc[page, slot].float() * ks[page, slot].float()[..., None]          # [L, H_KV, D]
        v = vc[page, slot].float() * vs[page, slot].float()[..., None]
        qq = q[b, :q_len].float().reshape(q_len, H_KV, G, D).permute(1, 0, 2, 3).reshape(H_KV, q_len * G, D)
        s = torch.bmm(qq, k.permute(1, 2, 0).contiguous()) / math.sqrt(D)       # [H_KV, q_len*G, L]
        qpos = (L - q_len + torch.arange(q_len)).repeat_interleave(G)
        s = s.masked_fill(pos[None, None, :] > qpos[None, :, None], float("-inf"))
        o = torch.bmm(s.softmax(-1), v.permute(1, 0, 2).contiguous())           # [H_KV, q_len*G, D]
        out[b, :q_len] = o.reshape(H_KV, q_len, G, D).permute(1, 0, 2, 3).reshape(q_len, H, D)
    return out.half()
