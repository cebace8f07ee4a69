"""Quantized speculative-decoding verification kernels for MI355X (gfx950).

Drop-in counterpart of the reference's kernels.py: the same public names, signatures,
defaults and return values, so correctness and benchmark scripts written against the
reference run unchanged (`from kernels import *`).  The kernels themselves are hand-written
HIP for gfx950 in csrc/, reached through the C ABI of libspecq.so (include/specq.h):

  w8a8_matmul      INT8 x INT8 -> INT32 MFMA GEMM, per-token x per-channel scale epilogue
                   (reference kernels.py:27-55, 71-86)
  w4a16_matmul     packed-INT4 (group scales) x FP16 GEMM, dequantised once per weight
                   element and fed to FP16 MFMA (reference kernels.py:94-135, 150-166)
  paged_attention  INT8 paged-KV verification attention, GQA x (k+1) rows packed per
                   program, QPP=1 (decode style) or QPP=q_len (fused)
                   (reference kernels.py:178-236, 239-262)

and the steps either side of them on the device: paged_kv_append (the new tokens' K/V
quantised into the cache pages, the q8 of kernels.py:280-284), silu_mul /
silu_mul_quant_int8 / quantize_act_int8_gpu (kernels.py:58-62 on the device), and
w4a8_matmul (INT4 weights on the INT8 MFMA path, the reference's REPORT.md:156
recommendation; no reference kernel).

Every launcher takes `plan` (an int32 device tensor read by the kernel at run time) and a
fixed grid size, so a single captured graph replays every (B, k) (reference kernels.py:14-17).
Launches go to torch's current stream and never synchronise or allocate (except the
optional output allocation and the first growth of the shared workspace).

The host-side helpers (quantizers, INT4 packer, paged-KV generator, dense attention
reference) restate the reference formulas in torch and run on any device.

Differences a caller may notice:
  * BLOCK_K and num_stages are accepted and ignored (the MFMA K step and register
    pipelining are fixed per kernel).  BLOCK_M=None (or 0) picks the tile from the measured
    M staircase; BLOCK_N defaults to None (the channel width and split-K are then picked
    from M, N and K by a cost model fitted to measured latencies; the reference's default
    is 64).  Every tile choice gives bit-identical results.  W8A8 BLOCK_M
    is at most 304; BLOCK_N is 16/32/64/128 channels per workgroup (larger values are taken as
    128); W4A16 BLOCK_N is 64 or 128.
  * w8a8_matmul also accepts a PackedWeightInt8 (pack_weight_int8), the weight pre-packed
    once into MFMA fragments, with bit-identical results.
  * `ck` is a KernelInfo with n_regs / n_spills / metadata.shared like Triton's compiled
    kernel, plus the resolved tile configuration.
  * w4a16_matmul also accepts the int32 "8 nibbles per word along K" packing and a
    PackedWeightInt4 (pack_weight_int4), bit-identical to the int32 packing; its fp32
    summation order depends only on (N, K), split_k and whether the weight is the reference
    uint8 packing (whose bytes pair k with k + K/2), so every W4A16 tile choice is
    bit-identical too.
    W4A16 BLOCK_M is at most 256 (tiles deeper than 144 rows run as equal chunks of at most
    144 rows); its LDS-staged kernels run 8 waves whatever num_warps says.
"""
from __future__ import annotations

import ctypes
import math
import os
import sys

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
if _HERE not in sys.path:
    sys.path.insert(0, _HERE)

from specq import _lib  # noqa: E402
from specq import workspace as _ws  # noqa: E402

__all__ = [
    "w8a8_matmul", "w4a16_matmul", "paged_attention",
    "quantize_act_int8", "quantize_weight_int8", "quantize_weight_int4",
    "make_paged_kv", "paged_attention_ref",
    "silu_mul", "quantize_act_int8_gpu", "silu_mul_quant_int8", "paged_kv_append",
    "pack_int4_i32", "KernelInfo", "PackedWeightInt8", "pack_weight_int8", "PackedWeightInt4", "pack_weight_int4",
    "w4a8_matmul", "quantize_weight_int4_channel", "PackedWeightW4A8", "pack_weight_w4a8",
    "w8a8_matmul_grouped", "w4a16_matmul_grouped", "set_weight_pack_cache", "clear_weight_pack_cache",
]


# ----------------------------------------------------------------------------------------
# Kernel bookkeeping: the reference's `ck` object and the JIT-cache stand-ins read by
# correctness.py:18-24 (n_compiled).
# ----------------------------------------------------------------------------------------
class _Meta:
    def __init__(self, shared: int):
        self.shared = shared

    def __getitem__(self, key):
        return getattr(self, key)


class KernelInfo:
    """Resource usage of the kernel a call launched (lazy: queried on first access)."""

    def __init__(self, kind: int, variant: int, m_grid: int, N: int, K: int, block_m: int, block_n: int,
                 num_warps: int, split_k: int):
        # The kernel also depends on the library options (kernel-family overrides), so the
        # cache key carries them and a first-time query happens now, under the options the
        # call ran with.
        self._key = (kind, variant, m_grid, N, K, block_m, block_n, num_warps, split_k)
        try:
            self._attrs, self._err = _attrs_cached(self._key, _lib.options_key()), None
        except RuntimeError as e:  # reported when the attributes are read
            self._attrs, self._err = None, e

    def _get(self):
        if self._err is not None:
            raise self._err
        return self._attrs

    @property
    def name(self) -> str:
        return self._get().name.decode()

    @property
    def n_regs(self) -> int:
        return self._get().num_regs

    @property
    def n_spills(self) -> int:
        return self._get().scratch_bytes // 4

    @property
    def metadata(self) -> _Meta:
        return _Meta(self._get().lds_bytes)

    @property
    def config(self) -> dict:
        a = self._get()
        return dict(block_m=a.block_m, block_n=a.block_n, num_warps=a.num_warps, split_k=a.split_k,
                    threads=a.threads, grid=a.grid)

    def __repr__(self):
        return f"KernelInfo({self.name}, regs={self.n_regs}, spills={self.n_spills}, lds={self.metadata.shared})"


_ATTRS: dict = {}


def _attrs_cached(key, options):
    a = _ATTRS.get((key, options))
    if a is None:
        a = _ATTRS[(key, options)] = _lib.kernel_attrs(*key)
    return a


class _KernelRegistry:
    """Stand-in for a Triton JITFunction's cache: counts the distinct binaries launched."""

    def __init__(self, name: str):
        self.__name__ = name
        self.device_caches: dict = {}

    def _note(self, device_index: int, key) -> None:
        self.device_caches.setdefault(device_index, (set(),))[0].add(key)

    @property
    def cache(self) -> dict:
        return {d: v[0] for d, v in self.device_caches.items()}


_w8a8_kernel = _KernelRegistry("_w8a8_kernel")
_w4a16_kernel = _KernelRegistry("_w4a16_kernel")
_paged_attn_kernel = _KernelRegistry("_paged_attn_kernel")


def _stream_ptr(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def _require_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if t.device.type != "cuda":
            raise RuntimeError(f"specq kernels run on the GPU only; got a {t.device} tensor")


def _rowmajor(t: torch.Tensor) -> torch.Tensor:
    """2-D view with a unit inner stride (copies only when the inner stride is not 1)."""
    return t if t.stride(-1) == 1 else t.contiguous()


def _check_out(out: torch.Tensor, M: int, N: int, who: str) -> None:
    """The kernels write rows < M and columns < N of out: it must hold at least that."""
    if out.dim() != 2 or out.shape[0] < M or out.shape[1] < N:
        raise RuntimeError(f"{who}: out {tuple(out.shape)} is smaller than [M, N] = [{M}, {N}]")


def _check_w4_scales(sc: torch.Tensor, N: int, K: int, group: int, who: str) -> None:
    """W4A16 scales are fp16 [N, K/group]; a smaller tensor would be read past its end."""
    if group <= 0 or K % group:
        raise RuntimeError(f"{who}: K={K} is not a multiple of group={group}")
    if sc.dim() != 2 or tuple(sc.shape) != (N, K // group):
        raise RuntimeError(f"{who}: scales {tuple(sc.shape)} must be [N, K/group] = [{N}, {K // group}]")


def _plan_ptr(plan) -> int:
    if plan is None:
        return 0
    if plan.dtype != torch.int32 or plan.device.type != "cuda":
        raise RuntimeError("plan must be an int32 device tensor")
    return plan.data_ptr()


# ----------------------------------------------------------------------------------------
# W8A8
# ----------------------------------------------------------------------------------------
def _w8a8_block_n(block_n) -> int:
    if not block_n:
        return 0
    return 16 if block_n <= 16 else (32 if block_n <= 32 else (64 if block_n <= 64 else 128))


class PackedWeightInt8:
    """An int8 weight [N, K] pre-packed once into MFMA fragments for w8a8_matmul.

    Fragments are stored K-step-major: fragment (64-byte K step s, 16-row tile t) is the 1 KB
    at (s * ceil(N/16) + t) KB holding, for lane l and byte b, w[16t + l%16][64s + 16*(l/16) + b]
    (zero-padded), so every load is 1 KB contiguous and the workgroups running at one time
    read one compact window.  Results are bit-identical to passing the row-major weight.
    """

    def __init__(self, w_q: torch.Tensor):
        _require_gpu(w_q)
        if w_q.dtype != torch.int8 or w_q.dim() != 2:
            raise RuntimeError("PackedWeightInt8 expects an int8 [N, K] weight")
        w_q = _rowmajor(w_q)
        self.N, self.K = w_q.shape
        self.shape = (self.N, self.K)
        self.device = w_q.device
        nbytes = _lib.lib().specq_w8a8_packed_bytes(self.N, self.K)
        self.data = torch.empty(nbytes, dtype=torch.int8, device=w_q.device)
        _lib.call("specq_w8a8_pack_weight", w_q.data_ptr(), w_q.stride(0), self.N, self.K, self.data.data_ptr(),
                  _stream_ptr(w_q))


def pack_weight_int8(w_q):
    """Pack an int8 [N, K] weight for w8a8_matmul (see PackedWeightInt8)."""
    return PackedWeightInt8(w_q)


class _WeightPackCache:
    """Row-major int8 weights packed once, for callers that pass the reference's w_q layout.

    w8a8_matmul and w8a8_matmul_grouped given a row-major int8 weight (as the reference's
    scripts pass it, bench_graphs.py:55-64, correctness.py:36) look it up here and run the
    packed-fragment kernels on its PackedWeightInt8: the results are bit-identical (the INT32
    sums do not depend on the weight layout), and the packed layout streams each weight as 1 KB
    contiguous fragments where the row-major one reads half cache lines.  An entry is keyed on
    the weight's storage, offset, shape and strides and remembers the storage's version counter,
    so an in-place update of the weight (through it or any view of it) repacks it on the next
    call; the entry holds the source storage, so its memory cannot be reused under the key while
    cached.  A miss inside graph capture does not pack (that would allocate): the call runs the
    row-major kernel, with the same results.  Entries beyond the byte budget are evicted least
    recently used first.  Controls: set_weight_pack_cache(enabled, budget_bytes),
    clear_weight_pack_cache(); the environment variable SPECQ_PACK_CACHE=0 starts it disabled.
    """

    def __init__(self):
        import collections
        import threading
        self.enabled = os.environ.get("SPECQ_PACK_CACHE", "1") != "0"
        self.budget = 64 << 30
        self.bytes = 0
        self._d = collections.OrderedDict()
        self._lock = threading.Lock()

    @staticmethod
    def _key(w: torch.Tensor):
        return (w.device.index, w.untyped_storage().data_ptr(), w.storage_offset(), tuple(w.shape), tuple(w.stride()))

    def lookup(self, w: torch.Tensor):
        """The PackedWeightInt8 of w (packing it now on a miss), or None (disabled, or a miss
        during graph capture)."""
        if not self.enabled or w.dtype != torch.int8 or w.dim() != 2 or w.stride(-1) != 1:
            return None
        key = self._key(w)
        with self._lock:
            e = self._d.get(key)
            if e is not None:
                if e[1] == w._version:
                    self._d.move_to_end(key)
                    return e[0]
                del self._d[key]
                self.bytes -= e[0].data.numel()
        if torch.cuda.is_current_stream_capturing():
            return None
        packed = PackedWeightInt8(w)
        with self._lock:
            old = self._d.pop(key, None)
            if old is not None:
                self.bytes -= old[0].data.numel()
            self._d[key] = (packed, w._version, w.untyped_storage())
            self.bytes += packed.data.numel()
            while self.bytes > self.budget and len(self._d) > 1:
                _, (pw, _, _) = self._d.popitem(last=False)
                self.bytes -= pw.data.numel()
        return packed

    def clear(self):
        with self._lock:
            self._d.clear()
            self.bytes = 0


_pack_cache = _WeightPackCache()


def set_weight_pack_cache(enabled: bool = True, budget_bytes: int | None = None) -> None:
    """Turn the transparent packing of row-major W8A8 weights on or off, and set its byte budget."""
    _pack_cache.enabled = bool(enabled)
    if budget_bytes is not None:
        _pack_cache.budget = int(budget_bytes)
    if not enabled:
        _pack_cache.clear()


def clear_weight_pack_cache() -> None:
    """Drop every packed copy the transparent cache holds (their memory returns to torch)."""
    _pack_cache.clear()


def _aligned16(a_q: torch.Tensor, K: int) -> bool:
    """The packed-fragment kernels read 16-byte pieces of the activation rows."""
    return a_q.data_ptr() % 16 == 0 and (a_q.stride(0) % 16 == 0 or a_q.shape[0] <= 1) and K % 16 == 0


def w8a8_matmul(a_q, sa, w_q, sw, out=None, BLOCK_M=16, BLOCK_N=None, BLOCK_K=128,
                num_warps=4, num_stages=3, plan=None, grid_m_max=None, split_k=0, workspace=None,
                plan_tiles=None):
    """C[M, N] = fp16((int32(a_q @ w_q.T) * sa[:, None]) * sw[None, :]).  Returns (out, ck).

    a_q int8 [M, K]; w_q int8 [N, K] (or a PackedWeightInt8); sa fp32 [M]; sw fp32 [N].
    With `plan`, M is read from plan[0] on the device and the grid covers grid_m_max rows
    (reference kernels.py:71-86).  Plan-mode calls with an automatic BLOCK_M use tiles of at
    most 80 rows, so a small active M leaves the later chunks idle; plan_tiles="grid" instead
    runs the tiles an eager call of grid_m_max rows would pick (for plan graphs whose active M
    stays close to the grid, e.g. one graph per shape bucket).  The INT32 sums are exact, so
    every tile gives the same result.
    """
    packed = isinstance(w_q, PackedWeightInt8)
    _require_gpu(a_q, sa, sw)
    if not packed:
        _require_gpu(w_q)
    if a_q.dtype != torch.int8 or (not packed and w_q.dtype != torch.int8):
        raise RuntimeError("w8a8_matmul expects int8 activations and weights")
    M, K = a_q.shape
    N = w_q.shape[0]
    if w_q.shape[1] != K:
        raise RuntimeError(f"w8a8_matmul: K mismatch {tuple(a_q.shape)} vs {tuple(w_q.shape)}")
    a_q = _rowmajor(a_q)
    if not packed:
        w_q = _rowmajor(w_q)
        if _aligned16(a_q, K):
            pw = _pack_cache.lookup(w_q)
            if pw is not None:
                w_q, packed = pw, True
    sa = sa.float().contiguous()
    sw = sw.float().contiguous()
    if sa.numel() < M or sw.numel() != N:
        raise RuntimeError(f"w8a8_matmul: scales sa {tuple(sa.shape)} / sw {tuple(sw.shape)} do not cover M={M} / N={N}")
    if out is None:
        out = torch.empty((M, N), device=a_q.device, dtype=torch.float16)
    if out.dtype != torch.float16 or out.stride(-1) != 1:
        raise RuntimeError("w8a8_matmul: out must be fp16 with unit inner stride")
    _check_out(out, M, N, "w8a8_matmul")
    m_grid = int(grid_m_max) if grid_m_max is not None else M
    bm = int(BLOCK_M) if BLOCK_M else 0  # 0: the library picks the tile (cost model over M, N, K)
    bn = _w8a8_block_n(BLOCK_N)
    nw = int(num_warps) if num_warps else 4
    if plan is not None and plan_tiles is not None:
        if plan_tiles != "grid":
            raise RuntimeError(f"w8a8_matmul: plan_tiles={plan_tiles!r} (None or 'grid')")
        if not bm:
            cfg = KernelInfo(0, 1 if packed else 0, m_grid, N, K, 0, bn, nw, split_k).config
            bm, bn, split_k = cfg["block_m"], cfg["block_n"], cfg["split_k"]
    ws = workspace or _ws.shared(a_q.device)
    if packed:
        need = _lib.lib().specq_w8a8_packed_workspace_size(m_grid, N, K, bm, bn, nw, split_k)
        wptr, wbytes = ws.ensure(need)
        _lib.call("specq_w8a8_packed", a_q.data_ptr(), a_q.stride(0), w_q.data.data_ptr(),
                  sa.data_ptr(), sw.data_ptr(), out.data_ptr(), out.stride(0),
                  M, N, K, int(grid_m_max or 0), _plan_ptr(plan), bm, bn, nw, split_k,
                  wptr, wbytes, _stream_ptr(a_q))
    else:
        need = _lib.lib().specq_w8a8_workspace_size(m_grid, N, K, bm, bn, nw, split_k)
        wptr, wbytes = ws.ensure(need)
        _lib.call("specq_w8a8", a_q.data_ptr(), a_q.stride(0), w_q.data_ptr(), w_q.stride(0),
                  sa.data_ptr(), sw.data_ptr(), out.data_ptr(), out.stride(0),
                  M, N, K, int(grid_m_max or 0), _plan_ptr(plan), bm, bn, nw, split_k,
                  wptr, wbytes, _stream_ptr(a_q))
    _w8a8_kernel._note(a_q.device.index or 0, (bm, bn, nw))
    return out, KernelInfo(0, (1 if packed else 0) | (16 if plan is not None else 0), m_grid, N, K, bm, bn, nw, split_k)


def w8a8_matmul_grouped(a_q, sa, weights, outs=None, BLOCK_M=16, BLOCK_N=None, num_warps=4, plan=None,
                        grid_m_max=None, split_k=0, workspace=None, plan_tiles=None):
    """Up to four W8A8 GEMMs that share one activation (q, k and v; gate and up) in one launch.

    outs[g] = fp16((int32(a_q @ W_g.T) * sa[:, None]) * sw_g[None, :]) for weights[g] = (W_g, sw_g),
    bit-identical to one w8a8_matmul (or w4a8_matmul) call per GEMM.  The W_g are all int8 [N_g, K]
    tensors, all PackedWeightInt8 or all PackedWeightW4A8.  The launch uses the tiles of one GEMM
    of width sum(N_g), as the reference's fused qkv / gate_up weights do (bench_matmul.py:16),
    while the weights and outputs stay separate.  Other arguments as w8a8_matmul.  Returns
    (outs, ck).
    """
    n = len(weights)
    if not 1 <= n <= 4:
        raise RuntimeError(f"w8a8_matmul_grouped: {n} GEMMs (1..4 supported)")
    ws_ = [w for w, _ in weights]
    if all(isinstance(w, PackedWeightInt8) for w in ws_):
        layout = 1
    elif all(isinstance(w, PackedWeightW4A8) for w in ws_):
        layout = 2
    elif all(isinstance(w, torch.Tensor) and w.dtype == torch.int8 for w in ws_):
        layout = 0
    else:
        raise RuntimeError("w8a8_matmul_grouped: weights must all be int8 tensors, all PackedWeightInt8 "
                           "or all PackedWeightW4A8")
    _require_gpu(a_q, sa, *(sw for _, sw in weights))
    if layout == 0:
        _require_gpu(*ws_)
        ws_ = [_rowmajor(w) for w in ws_]
    if a_q.dtype != torch.int8:
        raise RuntimeError("w8a8_matmul_grouped expects int8 activations")
    M, K = a_q.shape
    Ns = [int(w.shape[0]) if layout == 0 else int(w.N) for w in ws_]
    for w in ws_:
        if (w.shape[1] if layout == 0 else w.K) != K:
            raise RuntimeError(f"w8a8_matmul_grouped: K mismatch {tuple(a_q.shape)} vs {tuple(w.shape)}")
    a_q = _rowmajor(a_q)
    if layout == 0 and _aligned16(a_q, K):
        pws = [_pack_cache.lookup(w) for w in ws_]
        if all(pw is not None for pw in pws):
            ws_, layout = pws, 1
    sa = sa.float().contiguous()
    sws = [sw.float().contiguous() for _, sw in weights]
    for sw, N in zip(sws, Ns):
        if sw.numel() != N:
            raise RuntimeError(f"w8a8_matmul_grouped: channel scale of {sw.numel()} entries for N={N}")
    if outs is None:
        outs = [torch.empty((M, N), device=a_q.device, dtype=torch.float16) for N in Ns]
    if len(outs) != n:
        raise RuntimeError("w8a8_matmul_grouped: one output per GEMM")
    for o, N in zip(outs, Ns):
        if o.dtype != torch.float16 or o.stride(-1) != 1 or tuple(o.shape) != (M, N):
            raise RuntimeError(f"w8a8_matmul_grouped: outputs must be fp16 [M, N] with unit inner stride, got "
                               f"{tuple(o.shape)} for N={N}")
    m_grid = int(grid_m_max) if grid_m_max is not None else M
    N_total = sum(Ns)
    bm = int(BLOCK_M) if BLOCK_M else 0
    bn = _w8a8_block_n(BLOCK_N)
    nw = int(num_warps) if num_warps else 4
    if plan is not None and plan_tiles is not None:
        if plan_tiles != "grid":
            raise RuntimeError(f"w8a8_matmul_grouped: plan_tiles={plan_tiles!r} (None or 'grid')")
        if not bm:
            cfg = KernelInfo(0, layout, m_grid, N_total, K, 0, bn, nw, split_k).config
            bm, bn, split_k = cfg["block_m"], cfg["block_n"], cfg["split_k"]
    arr = lambda ct, vals: (ct * n)(*vals)  # noqa: E731
    n_arr = arr(ctypes.c_int, Ns)
    w_arr = arr(ctypes.c_void_p, [w.data_ptr() if layout == 0 else w.data.data_ptr() for w in ws_])
    ldw_arr = arr(ctypes.c_int64, [w.stride(0) if layout == 0 else 0 for w in ws_])
    sw_arr = arr(ctypes.c_void_p, [sw.data_ptr() for sw in sws])
    c_arr = arr(ctypes.c_void_p, [o.data_ptr() for o in outs])
    ldc_arr = arr(ctypes.c_int64, [o.stride(0) for o in outs])
    ws = workspace or _ws.shared(a_q.device)
    need = _lib.lib().specq_w8a8_grouped_workspace_size(layout, m_grid, n, n_arr, K, bm, bn, nw, split_k)
    wptr, wbytes = ws.ensure(need)
    _lib.call("specq_w8a8_grouped", layout, a_q.data_ptr(), a_q.stride(0), sa.data_ptr(), n, w_arr, ldw_arr, sw_arr,
              c_arr, ldc_arr, n_arr, M, K, int(grid_m_max or 0), _plan_ptr(plan), bm, bn, nw, split_k,
              wptr, wbytes, _stream_ptr(a_q))
    _w8a8_kernel._note(a_q.device.index or 0, (bm, bn, nw, "grouped", layout))
    return outs, KernelInfo(0, layout | (16 if plan is not None else 0), m_grid, N_total, K, bm, bn, nw, split_k)


def quantize_act_int8(x):
    """Dynamic per-token symmetric INT8 quantisation (reference kernels.py:58-62)."""
    s = x.abs().amax(dim=-1).float().clamp(min=1e-8) / 127.0
    q = torch.round(x.float() / s[:, None]).clamp(-127, 127).to(torch.int8)
    return q, s


def quantize_weight_int8(w):
    """Per-output-channel symmetric INT8 quantisation (reference kernels.py:65-68)."""
    s = w.abs().amax(dim=-1).float().clamp(min=1e-8) / 127.0
    q = torch.round(w.float() / s[:, None]).clamp(-127, 127).to(torch.int8)
    return q, s


# ----------------------------------------------------------------------------------------
# W4A16
# ----------------------------------------------------------------------------------------
def quantize_weight_int4(w, group=128):
    """Group-wise symmetric INT4 (reference kernels.py:138-147).

    Returns (packed uint8 [N, K/2], scales fp16 [N, K/group], dequantised fp16 [N, K]).
    Byte j of a packed row holds k = j (low nibble) and k = j + K/2 (high nibble), each as
    q + 8 with q in [-8, 7].
    """
    N, K = w.shape
    assert K % 2 == 0 and (K // 2) % group == 0
    wg = w.float().reshape(N, K // group, group)
    sc = wg.abs().amax(-1).clamp(min=1e-8) / 7.0
    q = torch.round(wg / sc[..., None]).clamp(-8, 7).reshape(N, K).to(torch.int16) + 8
    half = K // 2
    packed = (q[:, :half] | (q[:, half:] << 4)).to(torch.uint8).contiguous()
    deq = ((q - 8).float().reshape(N, K // group, group) * sc[..., None]).reshape(N, K)
    return packed, sc.to(torch.float16).contiguous(), deq.to(torch.float16)


def pack_int4_i32(q_unsigned):
    """Pack unsigned nibbles [N, K] (values 0..15) as int32 [N, K/8]: nibble i of word j = k 8j+i."""
    N, K = q_unsigned.shape
    assert K % 8 == 0
    v = q_unsigned.to(torch.int64).reshape(N, K // 8, 8)
    shifts = torch.arange(0, 32, 4, device=v.device, dtype=torch.int64)
    word = (v << shifts).sum(-1)
    word = torch.where(word >= 2 ** 31, word - 2 ** 32, word)
    return word.to(torch.int32).contiguous()


class PackedWeightInt4:
    """A W4A16 weight (uint8 [N, K/2] reference packing or int32 [N, K/8]) re-packed once into
    MFMA fragments for w4a16_matmul.

    Fragment (128-wide K block b, 16-row tile t) is the 1 KB at (b * ceil(N/16) + t) KB; lane
    l's 16 bytes hold row 16t + l%16 at k = 128b + 32*(l/16) + 8u + j as word u, nibble j at
    bits 4p..4p+3 with p = j/2 for even j and 4 + j/2 for odd j (each pair of weights then
    becomes two fp16 with one AND-OR).  Every weight load is 1 KB contiguous.  The
    group scales are not repacked.  Results are bit-identical to passing the int32 packing of
    the same weight (the reference uint8 packing sums K in another order, so it agrees to
    fp32 rounding).
    """

    def __init__(self, wp: torch.Tensor):
        _require_gpu(wp)
        if wp.dim() != 2 or wp.dtype not in (torch.uint8, torch.int32):
            raise RuntimeError("PackedWeightInt4 expects uint8 [N, K/2] or int32 [N, K/8] packed weights")
        wp = _rowmajor(wp)
        layout = 0 if wp.dtype == torch.uint8 else 1
        self.N = wp.shape[0]
        self.K = wp.shape[1] * (2 if layout == 0 else 8)
        self.shape = (self.N, self.K)
        self.device = wp.device
        nbytes = _lib.lib().specq_w4a16_packed_bytes(self.N, self.K)
        if nbytes == 0:
            raise RuntimeError(f"PackedWeightInt4: K={self.K} must be a multiple of 128")
        self.data = torch.empty(nbytes, dtype=torch.uint8, device=wp.device)
        _lib.call("specq_w4a16_pack_weight", wp.data_ptr(), wp.stride(0), layout, self.N, self.K,
                  self.data.data_ptr(), _stream_ptr(wp))


def pack_weight_int4(wp):
    """Pack a W4A16 weight for w4a16_matmul (see PackedWeightInt4)."""
    return PackedWeightInt4(wp)


def w4a16_matmul(a, wp, sc, group=128, out=None, BLOCK_M=16, BLOCK_N=None, BLOCK_K=64,
                 num_warps=4, num_stages=3, plan=None, grid_m_max=None, split_k=0, workspace=None):
    """C[M, N] = fp16(a @ dequant(wp, sc).T) (reference kernels.py:150-166).  Returns (out, ck).

    a fp16 [M, K].  wp is uint8 [N, K/2] (reference packing), int32 [N, K/8] (8 nibbles per
    word along K) or a PackedWeightInt4.  sc fp16 [N, K/group].
    """
    _require_gpu(a, sc)
    assert BLOCK_K <= group and group % BLOCK_K == 0
    M, K = a.shape
    N = wp.shape[0]
    if isinstance(wp, PackedWeightInt4):
        layout = 2
        if wp.K != K:
            raise RuntimeError(f"w4a16_matmul: packed weight K={wp.K} does not match K={K}")
    elif wp.dtype == torch.uint8:
        layout = 0
        if wp.shape[1] * 2 != K:
            raise RuntimeError(f"w4a16_matmul: packed uint8 weights {tuple(wp.shape)} do not match K={K}")
    elif wp.dtype == torch.int32:
        layout = 1
        if wp.shape[1] * 8 != K:
            raise RuntimeError(f"w4a16_matmul: packed int32 weights {tuple(wp.shape)} do not match K={K}")
    else:
        raise RuntimeError("w4a16_matmul: wp must be uint8 [N, K/2], int32 [N, K/8] or a PackedWeightInt4")
    if a.dtype != torch.float16 or sc.dtype != torch.float16:
        raise RuntimeError("w4a16_matmul expects fp16 activations and fp16 scales")
    _check_w4_scales(sc, N, K, int(group), "w4a16_matmul")
    a, sc = _rowmajor(a), _rowmajor(sc)
    if layout == 2:
        w_ptr, w_ld = wp.data.data_ptr(), 0
    else:
        _require_gpu(wp)
        wp = _rowmajor(wp)
        w_ptr, w_ld = wp.data_ptr(), wp.stride(0)
    if a.data_ptr() % 16 or a.stride(0) % 8:
        a = a.contiguous() if a.data_ptr() % 16 == 0 else a.clone()
    if out is None:
        out = torch.empty((M, N), device=a.device, dtype=torch.float16)
    if out.dtype != torch.float16 or out.stride(-1) != 1:
        raise RuntimeError("w4a16_matmul: out must be fp16 with unit inner stride")
    _check_out(out, M, N, "w4a16_matmul")
    m_grid = int(grid_m_max) if grid_m_max is not None else M
    bm = int(BLOCK_M) if BLOCK_M else 0
    bn = 0 if not BLOCK_N else (64 if BLOCK_N <= 64 else 128)
    ws = workspace or _ws.shared(a.device)
    need = _lib.lib().specq_w4a16_workspace_size(m_grid, N, K, bm, bn, 4, split_k)
    wptr, wbytes = ws.ensure(need)
    _lib.call("specq_w4a16", a.data_ptr(), a.stride(0), w_ptr, w_ld, layout,
              sc.data_ptr(), sc.stride(0), out.data_ptr(), out.stride(0),
              M, N, K, int(group), int(grid_m_max or 0), _plan_ptr(plan), bm, bn, 4, split_k,
              wptr, wbytes, _stream_ptr(a))
    _w4a16_kernel._note(a.device.index or 0, (bm, bn, layout))
    return out, KernelInfo(1, layout | (16 if plan is not None else 0), m_grid, N, K, bm, bn, 4, split_k)


def w4a16_matmul_grouped(a, weights, group=128, outs=None, BLOCK_M=None, BLOCK_N=None, num_warps=4, plan=None,
                         grid_m_max=None, split_k=0, workspace=None):
    """Up to four W4A16 GEMMs that share one fp16 activation (q, k and v; gate and up) in one launch.

    outs[g] = fp16(a @ dequant(wp_g, sc_g).T) for weights[g] = (wp_g, sc_g), bit-identical to one
    w4a16_matmul call per GEMM with the same split_k.  The wp_g are all PackedWeightInt4, all int32
    [N_g, K/8] or all uint8 [N_g, K/2].  The launch uses the tiles of one GEMM of width sum(N_g), as
    the reference's fused qkv / gate_up weights do (bench_matmul.py:16), while the weights and
    outputs stay separate; members whose automatic split counts differ run as one launch each.
    Other arguments as w4a16_matmul.  Returns (outs, ck).
    """
    n = len(weights)
    if not 1 <= n <= 4:
        raise RuntimeError(f"w4a16_matmul_grouped: {n} GEMMs (1..4 supported)")
    wps = [w for w, _ in weights]
    if all(isinstance(w, PackedWeightInt4) for w in wps):
        layout = 2
    elif all(isinstance(w, torch.Tensor) and w.dtype == torch.int32 for w in wps):
        layout = 1
    elif all(isinstance(w, torch.Tensor) and w.dtype == torch.uint8 for w in wps):
        layout = 0
    else:
        raise RuntimeError("w4a16_matmul_grouped: weights must all be PackedWeightInt4, all int32 [N, K/8] "
                           "or all uint8 [N, K/2]")
    scs = [sc for _, sc in weights]
    _require_gpu(a, *scs)
    if a.dtype != torch.float16 or any(sc.dtype != torch.float16 for sc in scs):
        raise RuntimeError("w4a16_matmul_grouped expects fp16 activations and fp16 scales")
    assert BLOCK_N is None or BLOCK_N in (64, 128)
    M, K = a.shape
    if layout == 2:
        Ns = [w.N for w in wps]
        if any(w.K != K for w in wps):
            raise RuntimeError(f"w4a16_matmul_grouped: packed weight K does not match K={K}")
        w_ptrs, w_lds = [w.data.data_ptr() for w in wps], [0] * n
    else:
        _require_gpu(*wps)
        wps = [_rowmajor(w) for w in wps]
        per = 2 if layout == 0 else 8
        Ns = [int(w.shape[0]) for w in wps]
        if any(w.shape[1] * per != K for w in wps):
            raise RuntimeError(f"w4a16_matmul_grouped: packed weights do not match K={K}")
        w_ptrs, w_lds = [w.data_ptr() for w in wps], [w.stride(0) for w in wps]
    for sc, N in zip(scs, Ns):
        _check_w4_scales(sc, N, K, int(group), "w4a16_matmul_grouped")
    a = _rowmajor(a)
    scs = [_rowmajor(sc) for sc in scs]
    if a.data_ptr() % 16 or a.stride(0) % 8:
        a = a.contiguous() if a.data_ptr() % 16 == 0 else a.clone()
    if outs is None:
        outs = [torch.empty((M, N), device=a.device, dtype=torch.float16) for N in Ns]
    if len(outs) != n:
        raise RuntimeError("w4a16_matmul_grouped: one output per GEMM")
    for o, N in zip(outs, Ns):
        if o.dtype != torch.float16 or o.stride(-1) != 1 or tuple(o.shape) != (M, N):
            raise RuntimeError(f"w4a16_matmul_grouped: outputs must be fp16 [M, N] with unit inner stride, got "
                               f"{tuple(o.shape)} for N={N}")
    m_grid = int(grid_m_max) if grid_m_max is not None else M
    bm = int(BLOCK_M) if BLOCK_M else 0
    bn = 0 if not BLOCK_N else int(BLOCK_N)
    arr = lambda ct, vals: (ct * n)(*vals)  # noqa: E731
    n_arr = arr(ctypes.c_int, Ns)
    ws = workspace or _ws.shared(a.device)
    need = _lib.lib().specq_w4a16_grouped_workspace_size(m_grid, n, n_arr, K, bm, bn, 4, split_k)
    wptr, wbytes = ws.ensure(need)
    _lib.call("specq_w4a16_grouped", a.data_ptr(), a.stride(0), n, arr(ctypes.c_void_p, w_ptrs),
              arr(ctypes.c_int64, w_lds), layout, arr(ctypes.c_void_p, [sc.data_ptr() for sc in scs]),
              arr(ctypes.c_int64, [sc.stride(0) for sc in scs]), arr(ctypes.c_void_p, [o.data_ptr() for o in outs]),
              arr(ctypes.c_int64, [o.stride(0) for o in outs]), n_arr, M, K, int(group), int(grid_m_max or 0),
              _plan_ptr(plan), bm, bn, 4, split_k, wptr, wbytes, _stream_ptr(a))
    _w4a16_kernel._note(a.device.index or 0, (bm, bn, "grouped", layout))
    # The launch runs the members' common split count: report the tiles of that launch.
    sk = w4a16_group_split(Ns, K, split_k) if n > 1 else split_k
    return outs, KernelInfo(1, layout | (16 if plan is not None else 0), m_grid, sum(Ns), K, bm, bn, 4,
                            sk if sk > 0 else split_k)


def w4a16_group_split(Ns, K: int, split_k: int = 0) -> int:
    """The split count a grouped W4A16 launch of members of widths Ns runs, or 0 when their
    counts differ (the members then run as one launch each)."""
    arr = (ctypes.c_int * len(Ns))(*[int(n) for n in Ns])
    return int(_lib.lib().specq_w4a16_grouped_split(len(Ns), arr, int(K), int(split_k)))


# ----------------------------------------------------------------------------------------
# Paged verification attention
# ----------------------------------------------------------------------------------------
def paged_attention(q, kc, vc, ks, vs, block_tbl, ctx_len, q_len, QPP=None, BLOCK_N=64,
                    num_warps=4, num_stages=2, plan=None, n_seqs=None, out=None, workspace=None):
    """Verification attention over an INT8 paged KV cache (reference kernels.py:239-262).

    q fp16 [B, QLMAX, H, D]; kc/vc int8 [pages, PAGE, H_KV, D]; ks/vs fp16 or fp32
    [pages, PAGE, H_KV]; block_tbl int32 [B, max_pages]; ctx_len int32 [B] (includes the
    q_len query tokens; block-table ids outside [0, pages) mask their page's tokens).  QPP
    query tokens per program (default q_len = fused).  With
    `plan`, (n_seqs, q_len) = plan[0:2] on the device and the grid covers (B, QLMAX).
    Returns (out, ck).
    """
    _require_gpu(q, kc, vc, ks, vs, block_tbl, ctx_len)
    B, QLMAX, H, D = q.shape
    PAGE, H_KV = kc.shape[1], kc.shape[2]
    if QPP is None:
        QPP = q_len
    if out is None:
        out = torch.zeros_like(q)
    n_seqs = B if n_seqs is None else n_seqs
    if q.dtype != torch.float16 or out.dtype != torch.float16:
        raise RuntimeError("paged_attention expects fp16 q and out")
    if kc.dtype != torch.int8 or vc.dtype != torch.int8:
        raise RuntimeError("paged_attention expects an int8 KV cache")
    if kc.stride() != vc.stride() or ks.stride() != vs.stride() or ks.dtype != vs.dtype:
        raise RuntimeError("paged_attention: K and V (and their scales) must share layout and dtype")
    if ks.dtype not in (torch.float16, torch.float32):
        raise RuntimeError("paged_attention: scales must be fp16 or fp32")
    if q.stride(3) != 1 or out.stride(3) != 1 or kc.stride(3) != 1:
        raise RuntimeError("paged_attention: head_dim must be contiguous")
    if block_tbl.dtype != torch.int32 or ctx_len.dtype != torch.int32:
        raise RuntimeError("paged_attention: block_tbl and ctx_len must be int32")
    if out.shape != q.shape:
        raise RuntimeError(f"paged_attention: out {tuple(out.shape)} must have q's shape {tuple(q.shape)}")
    if kc.shape != vc.shape or kc.shape[3] != D or H % H_KV != 0:
        raise RuntimeError(f"paged_attention: cache {tuple(kc.shape)} does not fit q {tuple(q.shape)}")
    if tuple(ks.shape) != tuple(kc.shape[:3]) or ks.shape != vs.shape:
        raise RuntimeError(f"paged_attention: scales {tuple(ks.shape)} must be [pages, PAGE, H_KV]")
    if int(QPP) < 1:
        raise RuntimeError(f"paged_attention: QPP={QPP} must be at least 1")
    if plan is None and not (0 <= int(n_seqs) <= B and 0 <= int(q_len) <= QLMAX):
        raise RuntimeError(f"paged_attention: need 0 <= n_seqs <= {B} and 0 <= q_len <= {QLMAX}")
    block_tbl = _rowmajor(block_tbl)
    ctx_len = ctx_len.contiguous()
    B_grid = B if plan is not None else int(n_seqs)
    if block_tbl.dim() != 2 or block_tbl.shape[0] < B_grid or ctx_len.numel() < B_grid:
        raise RuntimeError("paged_attention: block_tbl and ctx_len must cover every sequence of the grid")
    G = H // H_KV
    max_pages = block_tbl.shape[1]
    ws = workspace or _ws.shared(q.device)
    need = _lib.lib().specq_paged_attn_workspace_size(B_grid, H, H_KV, QLMAX, int(QPP), max_pages, PAGE)
    wptr, wbytes = ws.ensure(need)
    _lib.call("specq_paged_attn",
              q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
              kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2),
              ks.data_ptr(), vs.data_ptr(), ks.stride(0), ks.stride(1), ks.stride(2),
              1 if ks.dtype == torch.float32 else 0,
              block_tbl.data_ptr(), block_tbl.stride(0), max_pages, min(kc.shape[0], 2**31 - 1), ctx_len.data_ptr(),
              out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
              B_grid, int(n_seqs), int(q_len), QLMAX, H, H_KV, D, PAGE, int(QPP),
              1.0 / math.sqrt(D), _plan_ptr(plan), wptr, wbytes, _stream_ptr(q))
    rows = int(QPP) * G
    _paged_attn_kernel._note(q.device.index or 0, (D, (rows + 15) // 16, str(ks.dtype)))
    return out, KernelInfo(2, D | (1 << 16 if ks.dtype == torch.float32 else 0), 0, 0, 0, rows, 0, 4, 0)


def make_paged_kv(B, ctx_len, H_KV, D, PAGE=16, device="cuda", seed=0):
    """Random INT8 KV cache with a shuffled page table (reference kernels.py:265-286).

    Same generator calls in the same order as the reference, so a given seed yields the
    same cache.  Returns (kc, vc, ks, vs, block_tbl, ctx_len) with fp16 scales.
    """
    g = torch.Generator(device="cpu").manual_seed(seed)
    pages_per_seq = [(int(l) + PAGE - 1) // PAGE for l in ctx_len]
    total = sum(pages_per_seq)
    perm = torch.randperm(total, generator=g)
    bt = torch.zeros((B, max(pages_per_seq)), dtype=torch.int32)
    start = 0
    for b, n in enumerate(pages_per_seq):
        bt[b, :n] = perm[start:start + n].to(torch.int32)
        start += n
    kf = torch.randn((total, PAGE, H_KV, D), generator=g).half()
    vf = torch.randn((total, PAGE, H_KV, D), generator=g).half()

    def q8(x):
        s = x.float().abs().amax(-1).clamp(min=1e-8) / 127.0
        return torch.round(x.float() / s[..., None]).clamp(-127, 127).to(torch.int8), s.half()

    kc, ks = q8(kf)
    vc, vs = q8(vf)
    dev = lambda t: t.to(device).contiguous()  # noqa: E731
    return dev(kc), dev(vc), dev(ks), dev(vs), dev(bt), torch.tensor(list(ctx_len), dtype=torch.int32, device=device)


def paged_attention_ref(q, kc, vc, ks, vs, block_tbl, ctx_len, q_len):
    """Dense fp32 verification attention (reference kernels.py:289-309), any device."""
    B, _, H, D = q.shape
    PAGE, H_KV = kc.shape[1], kc.shape[2]
    G = H // H_KV
    out = torch.zeros(q.shape, dtype=torch.float32, device=q.device)
    for b in range(B):
        L = int(ctx_len[b])
        pos = torch.arange(L, device=q.device)
        page = block_tbl[b, pos // PAGE].long()
        slot = pos % PAGE
        k = (kc[page, slot].float() * ks[page, slot].float()[..., None]).repeat_interleave(G, dim=1)
        v = (vc[page, slot].float() * vs[page, slot].float()[..., None]).repeat_interleave(G, dim=1)
        qq = q[b, :q_len].float()
        s = torch.einsum("qhd,khd->hqk", qq, k) / math.sqrt(D)
        qpos = L - q_len + torch.arange(q_len, device=q.device)
        s = s.masked_fill(pos[None, None, :] > qpos[None, :, None], float("-inf"))
        out[b, :q_len] = torch.einsum("hqk,khd->qhd", s.softmax(-1), v)
    return out.half()


# ----------------------------------------------------------------------------------------
# Device-side steps of a verification layer (no reference counterpart on the device)
# ----------------------------------------------------------------------------------------
def silu_mul(gate, up, out=None, plan=None, grid_m_max=None):
    """h = fp16(silu(gate) * up) on the GPU; gate/up fp16 [M, N]."""
    _require_gpu(gate, up)
    M, N = gate.shape
    gate, up = _rowmajor(gate), _rowmajor(up)
    if out is None:
        out = torch.empty((M, N), device=gate.device, dtype=torch.float16)
    _lib.call("specq_silu_mul", gate.data_ptr(), gate.stride(0), up.data_ptr(), up.stride(0),
              out.data_ptr(), out.stride(0), M, N, int(grid_m_max or 0), _plan_ptr(plan), _stream_ptr(gate))
    return out


def quantize_act_int8_gpu(x, q=None, s=None, plan=None, grid_m_max=None):
    """quantize_act_int8 on the GPU (bit-identical to the torch formula); x fp16 [M, K]."""
    _require_gpu(x)
    M, K = x.shape
    x = _rowmajor(x)
    q = torch.empty((M, K), device=x.device, dtype=torch.int8) if q is None else q
    s = torch.empty((M,), device=x.device, dtype=torch.float32) if s is None else s
    _lib.call("specq_quantize_act_int8", x.data_ptr(), x.stride(0), q.data_ptr(), q.stride(0), s.data_ptr(),
              M, K, int(grid_m_max or 0), _plan_ptr(plan), _stream_ptr(x))
    return q, s


def silu_mul_quant_int8(gate, up, q=None, s=None, plan=None, grid_m_max=None):
    """quantize_act_int8(silu_mul(gate, up)) fused on the GPU; returns (int8 [M, N], fp32 [M])."""
    _require_gpu(gate, up)
    M, N = gate.shape
    gate, up = _rowmajor(gate), _rowmajor(up)
    q = torch.empty((M, N), device=gate.device, dtype=torch.int8) if q is None else q
    s = torch.empty((M,), device=gate.device, dtype=torch.float32) if s is None else s
    _lib.call("specq_silu_mul_quant_int8", gate.data_ptr(), gate.stride(0), up.data_ptr(), up.stride(0),
              q.data_ptr(), q.stride(0), s.data_ptr(), M, N, int(grid_m_max or 0), _plan_ptr(plan),
              _stream_ptr(gate))
    return q, s


# ----------------------------------------------------------------------------------------
# Paged INT8 KV-cache append (the device-side counterpart of make_paged_kv's q8)
# ----------------------------------------------------------------------------------------
def paged_kv_append(k_new, v_new, kc, vc, ks, vs, block_tbl, ctx_len, q_len=None, plan=None, n_seqs=None):
    """Quantise the new tokens' K/V into the paged INT8 cache, in place (kernels.py:280-284).

    k_new, v_new fp16 [B, QLMAX, H_KV, D] (the q_len tokens being verified); kc/vc int8
    [pages, PAGE, H_KV, D]; ks/vs fp16 or fp32 [pages, PAGE, H_KV]; block_tbl int32
    [B, max_pages]; ctx_len int32 [B], already counting the new tokens, so token i of
    sequence b goes to position ctx_len[b] - q_len + i.  Each (token, head) row gets
    s = max(amax, 1e-8) / 127 and q = clamp(rne(x / s), -127, 127), exactly as the
    reference quantises its cache.  With `plan`, (n_seqs, q_len) = plan[0:2] on the device
    and the grid covers (B, QLMAX).  Slots of inactive sequences and tokens are not written.
    """
    _require_gpu(k_new, v_new, kc, vc, ks, vs, block_tbl, ctx_len)
    B, QLMAX, H_KV, D = k_new.shape
    if v_new.shape != k_new.shape:
        raise RuntimeError("paged_kv_append: k_new and v_new must have the same shape")
    if k_new.dtype != torch.float16 or v_new.dtype != torch.float16:
        raise RuntimeError("paged_kv_append expects fp16 k_new and v_new")
    if kc.dtype != torch.int8 or vc.dtype != torch.int8 or kc.shape != vc.shape:
        raise RuntimeError("paged_kv_append expects int8 K/V caches of one shape")
    if kc.shape[2] != H_KV or kc.shape[3] != D:
        raise RuntimeError(f"paged_kv_append: cache {tuple(kc.shape)} does not match new K/V {tuple(k_new.shape)}")
    if kc.stride() != vc.stride() or ks.stride() != vs.stride() or ks.dtype != vs.dtype:
        raise RuntimeError("paged_kv_append: K and V (and their scales) must share layout and dtype")
    if ks.dtype not in (torch.float16, torch.float32):
        raise RuntimeError("paged_kv_append: scales must be fp16 or fp32")
    if block_tbl.dtype != torch.int32 or ctx_len.dtype != torch.int32:
        raise RuntimeError("paged_kv_append: block_tbl and ctx_len must be int32")
    if kc.stride(3) != 1:
        raise RuntimeError("paged_kv_append: head_dim of the cache must be contiguous")
    if k_new.stride() != v_new.stride() or k_new.stride(3) != 1:
        k_new, v_new = k_new.contiguous(), v_new.contiguous()
    block_tbl = _rowmajor(block_tbl)
    ctx_len = ctx_len.contiguous()
    q_len = QLMAX if q_len is None else int(q_len)
    n_seqs = B if n_seqs is None else int(n_seqs)
    if not (0 <= n_seqs <= B and 0 <= q_len <= QLMAX):
        raise RuntimeError(f"paged_kv_append: need 0 <= n_seqs <= {B} and 0 <= q_len <= {QLMAX}")
    B_grid = B if plan is not None else n_seqs
    ql_grid = QLMAX if plan is not None else q_len
    if block_tbl.dim() != 2 or block_tbl.shape[0] < B_grid or ctx_len.numel() < B_grid:
        raise RuntimeError("paged_kv_append: block_tbl and ctx_len must cover every sequence of the grid")
    _lib.call("specq_kv_append_int8",
              k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), k_new.stride(1), k_new.stride(2),
              kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2),
              ks.data_ptr(), vs.data_ptr(), ks.stride(0), ks.stride(1), ks.stride(2),
              1 if ks.dtype == torch.float32 else 0,
              block_tbl.data_ptr(), block_tbl.stride(0), block_tbl.shape[1], kc.shape[0], ctx_len.data_ptr(),
              B_grid, n_seqs, q_len, ql_grid, H_KV, D, kc.shape[1], _plan_ptr(plan), _stream_ptr(k_new))


# ----------------------------------------------------------------------------------------
# W4A8: INT4 weights on the INT8 MFMA path, per-channel scale in the W8A8 epilogue
# ----------------------------------------------------------------------------------------
def quantize_weight_int4_channel(w):
    """Per-channel symmetric INT4 weight for w4a8_matmul: (packed uint8 [N, K/2], scale fp32 [N]).

    The reference quantiser with one group per row (kernels.py:138-147 at group = K) and the
    scale kept in fp32: sc = max(amax_row, 1e-8) / 7, q = clamp(round(w / sc), -8, 7) + 8,
    packed as the reference packs (byte j = q[:, j] | q[:, j + K/2] << 4).
    """
    N, K = w.shape
    if K % 2:
        raise RuntimeError("quantize_weight_int4_channel: K must be even")
    wf = w.float()
    sc = wf.abs().amax(-1).clamp(min=1e-8) / 7.0
    q = (torch.round(wf / sc[:, None]).clamp(-8, 7) + 8).to(torch.uint8)
    half = K // 2
    return (q[:, :half] | (q[:, half:] << 4)).contiguous(), sc


class PackedWeightW4A8:
    """An INT4 weight packed once into the W4A8 kernel's 512-byte MFMA fragments.

    Source: the reference uint8 packing [N, K/2] (byte j holds k = j and k = j + K/2) or the
    int32 packing [N, K/8] (nibble i of word j holds k = 8j + i), nibbles with offset 8.
    Fragment (64-wide K step s, 16-row tile t) is the 512 bytes at (s * ceil(N/16) + t) * 512.
    """

    def __init__(self, wq: torch.Tensor, K: int = None):
        _require_gpu(wq)
        if wq.dim() != 2 or wq.dtype not in (torch.uint8, torch.int32):
            raise RuntimeError("PackedWeightW4A8 expects a uint8 [N, K/2] or int32 [N, K/8] INT4 weight")
        wq = _rowmajor(wq)
        layout = 0 if wq.dtype == torch.uint8 else 1
        self.N = wq.shape[0]
        self.K = int(K) if K is not None else wq.shape[1] * (2 if layout == 0 else 8)
        self.shape = (self.N, self.K)
        self.device = wq.device
        nbytes = _lib.lib().specq_w4a8_packed_bytes(self.N, self.K)
        self.data = torch.empty(nbytes, dtype=torch.int8, device=wq.device)
        _lib.call("specq_w4a8_pack_weight", wq.data_ptr(), wq.stride(0), layout, self.N, self.K,
                  self.data.data_ptr(), _stream_ptr(wq))


def pack_weight_w4a8(wq, K: int = None):
    """Pack an INT4 weight (uint8 [N, K/2] or int32 [N, K/8]) for w4a8_matmul."""
    return PackedWeightW4A8(wq, K)


def w4a8_matmul(a_q, sa, wq, sw, out=None, BLOCK_M=16, BLOCK_N=None, BLOCK_K=128, num_warps=4,
                num_stages=3, plan=None, grid_m_max=None, split_k=0, workspace=None):
    """C[M, N] = fp16((int32(a_q @ (q - 8).T) * sa[:, None]) * sw[None, :]).  Returns (out, ck).

    a_q int8 [M, K] with per-token scale sa fp32 [M] (quantize_act_int8); wq a
    PackedWeightW4A8, or an INT4 weight in the reference uint8 / int32 packing (packed here on
    every call; pack once at load time instead); sw fp32 [N] per-channel scale
    (quantize_weight_int4_channel).  Arguments otherwise as w8a8_matmul; results are
    bit-identical to w8a8_matmul on the unpacked INT4 weight.
    """
    if not isinstance(wq, PackedWeightW4A8):
        wq = PackedWeightW4A8(wq, a_q.shape[1])
    _require_gpu(a_q, sa, sw)
    if a_q.dtype != torch.int8:
        raise RuntimeError("w4a8_matmul expects int8 activations")
    M, K = a_q.shape
    N = wq.N
    if wq.K != K:
        raise RuntimeError(f"w4a8_matmul: K mismatch {tuple(a_q.shape)} vs {wq.shape}")
    a_q = _rowmajor(a_q)
    sa = sa.float().contiguous()
    sw = sw.float().contiguous()
    if out is None:
        out = torch.empty((M, N), device=a_q.device, dtype=torch.float16)
    if out.dtype != torch.float16 or out.stride(-1) != 1:
        raise RuntimeError("w4a8_matmul: out must be fp16 with unit inner stride")
    m_grid = int(grid_m_max) if grid_m_max is not None else M
    bm = int(BLOCK_M) if BLOCK_M else 0  # 0: the library picks the tile (cost model over M, N, K)
    bn = _w8a8_block_n(BLOCK_N)
    nw = int(num_warps) if num_warps else 4
    ws = workspace or _ws.shared(a_q.device)
    need = _lib.lib().specq_w4a8_packed_workspace_size(m_grid, N, K, bm, bn, nw, split_k)
    wptr, wbytes = ws.ensure(need)
    _lib.call("specq_w4a8_packed", a_q.data_ptr(), a_q.stride(0), wq.data.data_ptr(),
              sa.data_ptr(), sw.data_ptr(), out.data_ptr(), out.stride(0),
              M, N, K, int(grid_m_max or 0), _plan_ptr(plan), bm, bn, nw, split_k,
              wptr, wbytes, _stream_ptr(a_q))
    _w8a8_kernel._note(a_q.device.index or 0, (bm, bn, nw, "w4a8"))
    return out, KernelInfo(0, 2 | (16 if plan is not None else 0), m_grid, N, K, bm, bn, nw, split_k)
