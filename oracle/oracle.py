"""CPU oracle for the quantized verification kernels -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module,
and only as the checker (or, for the CPU baseline, as the thing timed on the host).  The
product path (libspecq.so behind kernels.py) never calls it.

Each function restates one formula of the reference (Vaibhav1067/specdec-quant-triton) in
numpy, citing the reference file:line it follows.  How each one is pinned independently of
this restatement (closed forms, library routines, brute force, invariants) is listed in
tests/test_oracle.py; none is "parity unpinned".

Arithmetic conventions:
  * Integer work is exact: int8 x int8 products are summed in float64 through BLAS, which
    is exact because every partial sum stays below 2**53 (|sum| <= 16129 * K).
  * fp32 / fp16 steps use numpy's IEEE float32 / float16 with round-to-nearest-even, in
    the reference's operation order, so the fp16 outputs of W8A8 are bit-exact.
  * Floating-point GEMM and attention references accumulate in float64.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "w8a8_int32", "w8a8",
    "quantize_rows_int8",
    "quantize_weight_int4", "unpack_int4_u8", "pack_int4_u8", "unpack_int4_i32", "pack_int4_i32",
    "dequant_int4", "w4a16",
    "paged_attention",
    "silu_mul", "silu_mul_quant_int8",
    "paged_kv_append",
    "quantize_weight_int4_channel", "w4a8",
]


# ------------------------------------------------------------------------------------------
# W8A8 (kernels.py:27-55, correctness.py:37)
# ------------------------------------------------------------------------------------------
def w8a8_int32(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """INT32 accumulators acc[m, n] = sum_k a[m,k] * w[n,k] (kernels.py:44-48: tl.dot int8 -> int32)."""
    a = np.asarray(a, dtype=np.int8)
    w = np.asarray(w, dtype=np.int8)
    acc = a.astype(np.float64) @ w.astype(np.float64).T
    return acc.astype(np.int64).astype(np.int32)


def w8a8(a, sa, w, sw) -> np.ndarray:
    """fp16 output of the W8A8 kernel: fp16((fp32(acc) * sa[m]) * sw[n]) (kernels.py:51-55).

    The two scale products are applied left to right in fp32, as `acc.to(tl.float32) *
    sa[:, None] * sw[None, :]` evaluates, then cast to fp16 with round-to-nearest-even.
    """
    acc = w8a8_int32(a, w).astype(np.float32)
    sa = np.asarray(sa, dtype=np.float32)
    sw = np.asarray(sw, dtype=np.float32)
    c = (acc * sa[:, None]) * sw[None, :]
    return c.astype(np.float16)


# ------------------------------------------------------------------------------------------
# Per-row INT8 quantisation (kernels.py:58-68)
# ------------------------------------------------------------------------------------------
def quantize_rows_int8(x) -> tuple:
    """s = max(amax_row |x|, 1e-8) / 127 in fp32; q = clamp(rne(x / s), -127, 127) (kernels.py:60-61)."""
    xf = np.asarray(x).astype(np.float32)
    amax = np.abs(xf).max(axis=-1)
    s = (np.maximum(amax, np.float32(1e-8)) / np.float32(127.0)).astype(np.float32)
    q = np.clip(np.rint(xf / s[..., None]), -127, 127).astype(np.int8)
    return q, s


# ------------------------------------------------------------------------------------------
# INT4 packing and W4A16 (kernels.py:89-92, 94-135, 138-147)
# ------------------------------------------------------------------------------------------
def quantize_weight_int4(w, group: int = 128):
    """(packed u8 [N, K/2], scales fp16 [N, K/G], deq fp16 [N, K]) as kernels.py:138-147.

    sc = max(amax_group, 1e-8) / 7 in fp32; q = clamp(rne(w / sc), -8, 7) + 8; byte j holds
    q[:, j] | q[:, j + K/2] << 4; deq = fp16((q - 8) * sc) with the fp32 scale.
    """
    w = np.asarray(w).astype(np.float32)
    N, K = w.shape
    assert K % 2 == 0 and (K // 2) % group == 0
    wg = w.reshape(N, K // group, group)
    sc = (np.maximum(np.abs(wg).max(-1), np.float32(1e-8)) / np.float32(7.0)).astype(np.float32)
    q = np.clip(np.rint(wg / sc[..., None]), -8, 7).reshape(N, K).astype(np.int16) + 8
    packed = pack_int4_u8(q.astype(np.uint8))
    deq = ((q - 8).astype(np.float32).reshape(N, K // group, group) * sc[..., None]).reshape(N, K)
    return packed, sc.astype(np.float16), deq.astype(np.float16)


def pack_int4_u8(qu) -> np.ndarray:
    """Unsigned nibbles [N, K] -> reference bytes [N, K/2]: low = k, high = k + K/2 (kernels.py:143-145)."""
    qu = np.asarray(qu, dtype=np.uint8)
    half = qu.shape[1] // 2
    return (qu[:, :half] | (qu[:, half:] << 4)).astype(np.uint8)


def unpack_int4_u8(packed) -> np.ndarray:
    """Reference bytes [N, K/2] -> unsigned nibbles [N, K] (kernels.py:117-118 with kk, kk + HALF)."""
    p = np.asarray(packed, dtype=np.uint8)
    return np.concatenate([p & 0xF, p >> 4], axis=1).astype(np.uint8)


def pack_int4_i32(qu) -> np.ndarray:
    """Unsigned nibbles [N, K] -> int32 [N, K/8] with nibble i of word j holding k = 8j + i."""
    qu = np.asarray(qu, dtype=np.uint64)
    N, K = qu.shape
    v = qu.reshape(N, K // 8, 8)
    words = np.zeros((N, K // 8), dtype=np.uint64)
    for i in range(8):
        words |= v[:, :, i] << np.uint64(4 * i)
    return words.astype(np.uint32).view(np.int32)


def unpack_int4_i32(words) -> np.ndarray:
    w = np.asarray(words, dtype=np.int32).view(np.uint32)
    N, K8 = w.shape
    out = np.empty((N, K8, 8), dtype=np.uint8)
    for i in range(8):
        out[:, :, i] = (w >> np.uint32(4 * i)) & 0xF
    return out.reshape(N, K8 * 8)


def dequant_int4(qu, sc, group: int) -> np.ndarray:
    """fp16 weights of the W4A16 kernel: fp16(fp16(q - 8) * sc16) (kernels.py:117-127).

    fp16(q - 8) is exact; the product of two fp16 numbers is exact in fp32, so rounding it
    once to fp16 equals the fp16 multiply of the kernel.
    """
    q = np.asarray(qu).astype(np.int16) - 8
    sc = np.asarray(sc, dtype=np.float16)
    N, K = q.shape
    s_full = np.repeat(sc, group, axis=1)[:, :K]
    return (q.astype(np.float32) * s_full.astype(np.float32)).astype(np.float16)


def w4a16(a, qu, sc, group: int = 128) -> np.ndarray:
    """float64 sum_k a[m,k] * deq[n,k] (kernels.py:132-133 with the fp16 dequantised tiles)."""
    deq = dequant_int4(qu, sc, group).astype(np.float64)
    return np.asarray(a, np.float16).astype(np.float64) @ deq.T


# ------------------------------------------------------------------------------------------
# Paged verification attention (kernels.py:178-236, 289-309)
# ------------------------------------------------------------------------------------------
def paged_attention(q, kc, vc, ks, vs, block_tbl, ctx_len, q_len: int, magnitude: bool = False):
    """float64 dense restatement of paged_attention_ref (kernels.py:289-309).

    out[b, i, h] = sum_t softmax_t(q . k_t * ks_t / sqrt(D), t <= L - q_len + i) * v_t * vs_t
    with K/V gathered through the block table (page = bt[b, t // PAGE], slot = t % PAGE) and
    the GQA group of query head h reading KV head h // G.  The kernel rounds each normalised
    softmax weight times vs_t to fp16 before the PV product (kernels.py:232), a per-term
    relative perturbation of at most 2**-11 that the tests bound against `mag` below.
    Rows i >= q_len are left at zero.  Returns float64 [B, QLMAX, H, D]; with magnitude=True
    also mag[b, i, h] = sum_t p_t * |v_t * vs_t| (same shape), the scale against which the
    rounding of each p_t * vs_t term is measured (it bounds |out| and equals it when every
    v_t * vs_t >= 0).
    """
    q = np.asarray(q, dtype=np.float16).astype(np.float64)
    kc = np.asarray(kc, dtype=np.int8)
    vc = np.asarray(vc, dtype=np.int8)
    ks = np.asarray(ks).astype(np.float64)
    vs = np.asarray(vs).astype(np.float64)
    bt = np.asarray(block_tbl, dtype=np.int64)
    cl = np.asarray(ctx_len, dtype=np.int64)
    B, QL, H, D = q.shape
    PAGE, H_KV = kc.shape[1], kc.shape[2]
    G = H // H_KV
    out = np.zeros((B, QL, H, D), dtype=np.float64)
    mag = np.zeros((B, QL, H, D), dtype=np.float64) if magnitude else None
    for b in range(B):
        L = int(cl[b])
        pos = np.arange(L)
        page = bt[b, pos // PAGE]
        slot = pos % PAGE
        k = kc[page, slot].astype(np.float64) * ks[page, slot][..., None]      # [L, H_KV, D]
        v_int = vc[page, slot].astype(np.float64)
        v_sc = vs[page, slot]                                                  # [L, H_KV]
        # query row r = i * G + g is token i of query head kh * G + g
        qpos = np.repeat(L - q_len + np.arange(q_len), G)
        for kh in range(H_KV):
            qq = q[b, :q_len, kh * G:(kh + 1) * G, :].reshape(q_len * G, D)
            s = qq @ k[:, kh, :].T / np.sqrt(D)                                # [q_len * G, L]
            s = np.where(pos[None, :] > qpos[:, None], -np.inf, s)
            mx = s.max(axis=1, keepdims=True)
            mx = np.where(np.isfinite(mx), mx, 0.0)
            e = np.exp(s - mx)
            den = e.sum(axis=1, keepdims=True)
            p = np.where(den > 0, e / np.where(den > 0, den, 1.0), 0.0)
            pv = p * v_sc[None, :, kh]
            out[b, :q_len, kh * G:(kh + 1) * G, :] = (pv @ v_int[:, kh, :]).reshape(q_len, G, D)
            if magnitude:
                mag[b, :q_len, kh * G:(kh + 1) * G, :] = (np.abs(pv) @ np.abs(v_int[:, kh, :])).reshape(q_len, G, D)
    return (out, mag) if magnitude else out


# ------------------------------------------------------------------------------------------
# SiLU * mul and its fused quantisation (the build's own layer step; no reference code)
# ------------------------------------------------------------------------------------------
def silu_mul(gate, up) -> np.ndarray:
    """float64 silu(gate) * up = gate / (1 + exp(-gate)) * up on fp16 inputs."""
    g = np.asarray(gate, np.float16).astype(np.float64)
    u = np.asarray(up, np.float16).astype(np.float64)
    return g / (1.0 + np.exp(-g)) * u


def silu_mul_quant_int8(h_fp16) -> tuple:
    """Quantisation of an fp16 activation row block (kernels.py:58-62 applied to h)."""
    return quantize_rows_int8(np.asarray(h_fp16, np.float16))


# ------------------------------------------------------------------------------------------
# Paged INT8 KV-cache append (kernels.py:265-286: the q8 of make_paged_kv, applied to the
# new tokens and scattered through the block table)
# ------------------------------------------------------------------------------------------
def paged_kv_append(k_new, v_new, kc, vc, ks, vs, block_tbl, ctx_len, q_len: int, n_seqs=None) -> tuple:
    """Copies of (kc, vc, ks, vs) with the q_len new tokens of each sequence written in.

    Token i of sequence b goes to position pos = ctx_len[b] - q_len + i (ctx_len counts the
    new tokens, kernels.py:173), page block_tbl[b, pos // PAGE], slot pos % PAGE.  Each
    (token, head) row of D values is quantised as q8 does (kernels.py:280-283):
    s = max(amax |x|, 1e-8) / 127 in fp32, q = clamp(rne(x / s), -127, 127), and s is stored
    in the scale tensor's dtype (fp16 as kernels.py:283 returns it, or fp32).  Rows whose
    position or page falls outside the cache are skipped.
    """
    kc, vc = np.array(kc, dtype=np.int8), np.array(vc, dtype=np.int8)
    ks, vs = np.array(ks), np.array(vs)
    bt = np.asarray(block_tbl, dtype=np.int64)
    cl = np.asarray(ctx_len, dtype=np.int64)
    B = bt.shape[0] if n_seqs is None else int(n_seqs)
    PAGE, max_pages, n_pages = kc.shape[1], bt.shape[1], kc.shape[0]
    for src, cache, scales in ((k_new, kc, ks), (v_new, vc, vs)):
        x = np.asarray(src, dtype=np.float16)
        for b in range(B):
            for i in range(q_len):
                pos = int(cl[b]) - q_len + i
                if pos < 0 or pos // PAGE >= max_pages:
                    continue
                page = int(bt[b, pos // PAGE])
                if page < 0 or page >= n_pages:
                    continue
                q, s = quantize_rows_int8(x[b, i])          # rows = heads, [H_KV, D]
                cache[page, pos % PAGE] = q
                scales[page, pos % PAGE] = s.astype(scales.dtype)
    return kc, vc, ks, vs


# ------------------------------------------------------------------------------------------
# W4A8: INT4 weights with a per-channel scale on the W8A8 arithmetic (the INT4 packing of
# kernels.py:138-147 at one group per row; the epilogue of kernels.py:51-55)
# ------------------------------------------------------------------------------------------
def quantize_weight_int4_channel(w) -> tuple:
    """(unsigned nibbles [N, K], scale fp32 [N]): sc = max(amax_row, 1e-8) / 7 in fp32,
    q = clamp(rne(w / sc), -8, 7) + 8 -- kernels.py:140-142 with the group spanning the row."""
    w = np.asarray(w).astype(np.float32)
    sc = (np.maximum(np.abs(w).max(-1), np.float32(1e-8)) / np.float32(7.0)).astype(np.float32)
    q = np.clip(np.rint(w / sc[:, None]), -8, 7).astype(np.int16) + 8
    return q.astype(np.uint8), sc


def w4a8(a, sa, qu, sw) -> np.ndarray:
    """fp16((fp32(sum_k a[m,k] * (q[n,k] - 8)) * sa[m]) * sw[n]): W8A8 on the unpacked INT4 weight."""
    q = (np.asarray(qu, dtype=np.int16) - 8).astype(np.int8)
    return w8a8(a, sa, q, sw)
