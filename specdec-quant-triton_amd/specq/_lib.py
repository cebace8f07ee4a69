"""ctypes binding of libspecq.so (the C ABI declared in include/specq.h).

The library is built in-tree by build.py.  Nothing here falls back to another
implementation: if the library is missing or a call fails, a RuntimeError is raised.
"""
from __future__ import annotations

import ctypes
import os
import threading

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# SPECQ_LIB_PATH names another build of the same library (for example one compiled with
# different tuning); there is no fallback: a missing file raises like a missing libspecq.so.
LIB_PATH = os.environ.get("SPECQ_LIB_PATH") or os.path.join(PKG_DIR, "libspecq.so")

_c_int, _c_i64, _c_size, _c_vp, _c_float = ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_float


class KernelAttrs(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 160),
        ("num_regs", _c_int),
        ("lds_bytes", _c_int),
        ("scratch_bytes", _c_int),
        ("threads", _c_int),
        ("grid", _c_int),
        ("block_m", _c_int),
        ("block_n", _c_int),
        ("num_warps", _c_int),
        ("split_k", _c_int),
    ]


# name -> (restype, argtypes)
SIGNATURES = {
    "specq_version": (_c_int, []),
    "specq_last_error": (ctypes.c_char_p, []),
    "specq_w8a8_workspace_size": (_c_size, [_c_int] * 7),
    "specq_w8a8": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp, _c_vp, _c_i64,
                            _c_int, _c_int, _c_int, _c_int, _c_vp,
                            _c_int, _c_int, _c_int, _c_int, _c_vp, _c_size, _c_vp]),
    "specq_w8a8_packed_bytes": (_c_size, [_c_int, _c_int]),
    "specq_w8a8_pack_weight": (_c_int, [_c_vp, _c_i64, _c_int, _c_int, _c_vp, _c_vp]),
    "specq_w8a8_packed_workspace_size": (_c_size, [_c_int] * 7),
    "specq_w8a8_packed": (_c_int, [_c_vp, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64,
                                   _c_int, _c_int, _c_int, _c_int, _c_vp,
                                   _c_int, _c_int, _c_int, _c_int, _c_vp, _c_size, _c_vp]),
    "specq_w8a8_grouped_workspace_size": (_c_size, [_c_int, _c_int, _c_int, _c_vp, _c_int, _c_int, _c_int, _c_int,
                                                    _c_int]),
    "specq_w8a8_grouped": (_c_int, [_c_int, _c_vp, _c_i64, _c_vp, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                    _c_int, _c_int, _c_int, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_vp, _c_size,
                                    _c_vp]),
    "specq_w8a8_packed_noalloc": (_c_int, [_c_vp, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64,
                                           _c_int, _c_int, _c_int, _c_int, _c_vp,
                                           _c_int, _c_int, _c_int, _c_int, _c_vp]),
    "specq_w4a8_packed_bytes": (_c_size, [_c_int, _c_int]),
    "specq_w4a8_pack_weight": (_c_int, [_c_vp, _c_i64, _c_int, _c_int, _c_int, _c_vp, _c_vp]),
    "specq_w4a8_packed_workspace_size": (_c_size, [_c_int] * 7),
    "specq_w4a8_packed": (_c_int, [_c_vp, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64,
                                   _c_int, _c_int, _c_int, _c_int, _c_vp,
                                   _c_int, _c_int, _c_int, _c_int, _c_vp, _c_size, _c_vp]),
    "specq_set_option": (_c_int, [ctypes.c_char_p, _c_int]),
    "specq_w4a16_workspace_size": (_c_size, [_c_int] * 7),
    "specq_w4a16_packed_bytes": (_c_size, [_c_int, _c_int]),
    "specq_w4a16_pack_weight": (_c_int, [_c_vp, _c_i64, _c_int, _c_int, _c_int, _c_vp, _c_vp]),
    "specq_w4a16": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_int, _c_vp, _c_i64, _c_vp, _c_i64,
                             _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp,
                             _c_int, _c_int, _c_int, _c_int, _c_vp, _c_size, _c_vp]),
    "specq_w4a16_grouped_workspace_size": (_c_size, [_c_int, _c_int, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "specq_w4a16_grouped_split": (_c_int, [_c_int, _c_vp, _c_int, _c_int]),
    "specq_w4a16_grouped": (_c_int, [_c_vp, _c_i64, _c_int, _c_vp, _c_vp, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                     _c_int, _c_int, _c_int, _c_int, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_vp,
                                     _c_size, _c_vp]),
    "specq_paged_attn_workspace_size": (_c_size, [_c_int] * 7),
    "specq_paged_attn": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64,
                                  _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,
                                  _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_int,
                                  _c_vp, _c_i64, _c_int, _c_int, _c_vp,
                                  _c_vp, _c_i64, _c_i64, _c_i64,
                                  _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                  _c_int, _c_int, _c_float, _c_vp, _c_vp, _c_size, _c_vp]),
    "specq_kv_append_int8": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64,
                                      _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,
                                      _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_int,
                                      _c_vp, _c_i64, _c_int, _c_int, _c_vp,
                                      _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp, _c_vp]),
    "specq_silu_mul": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_int, _c_int, _c_int, _c_vp, _c_vp]),
    "specq_quantize_act_int8": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_int, _c_int, _c_int, _c_vp, _c_vp]),
    "specq_silu_mul_quant_int8": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp,
                                           _c_int, _c_int, _c_int, _c_vp, _c_vp]),
    "specq_kernel_attrs_query": (_c_int, [_c_int] * 9 + [ctypes.POINTER(KernelAttrs)]),
}

ERRNAMES = {-5: "EIO", -22: "EINVAL", -28: "ENOSPC", -95: "ENOTSUP"}

_lib = None
_lock = threading.Lock()


DIAG_LIB_PATH = os.path.join(PKG_DIR, "libspecq_diag.so")
# Entry points only the measurement build (libspecq_diag.so) exports.
DIAG_SIGNATURES = {
    "specq_diag_set_timeline": (_c_int, [_c_vp, _c_int]),
    "specq_diag_stream_read": (_c_int, [_c_vp, _c_i64, _c_int, _c_int, _c_int, _c_vp, _c_vp]),
    "specq_diag_xcc_ids": (_c_int, [_c_vp, _c_int, _c_int, _c_vp]),
}


def use_diag() -> None:
    """Load the measurement build (libspecq_diag.so: the same kernels, plus per-workgroup
    timestamps and a streaming-read kernel) instead of libspecq.so.  For specq/profiling.py
    only; must run before the first call into the library."""
    global LIB_PATH
    with _lock:
        if _lib is not None and LIB_PATH != DIAG_LIB_PATH:
            raise RuntimeError("use_diag(): libspecq.so is already loaded in this process")
        LIB_PATH = DIAG_LIB_PATH


def lib() -> ctypes.CDLL:
    """Load libspecq.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(
                        f"{LIB_PATH} is missing: build the HIP kernels first "
                        f"(python {os.path.join(PKG_DIR, 'build.py')})")
                h = ctypes.CDLL(LIB_PATH)
                sigs = dict(SIGNATURES, **(DIAG_SIGNATURES if LIB_PATH == DIAG_LIB_PATH else {}))
                for name, (res, args) in sigs.items():
                    fn = getattr(h, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = h
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().specq_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({ERRNAMES.get(rc, rc)}): {msg}")


def call(name: str, *args) -> int:
    rc = getattr(lib(), name)(*args)
    check(rc, name)
    return rc


_OPTIONS: dict = {}


def set_option(name: str, value: int) -> None:
    call("specq_set_option", name.encode(), int(value))
    _OPTIONS[name] = int(value)


def options_key() -> tuple:
    """The library options set through set_option (they can change which kernel a call runs)."""
    return tuple(sorted(_OPTIONS.items()))


def kernel_attrs(kind: int, variant: int, m_grid: int, N: int, K: int, block_m: int, block_n: int,
                 num_warps: int, split_k: int) -> KernelAttrs:
    out = KernelAttrs()
    rc = lib().specq_kernel_attrs_query(kind, variant, m_grid, N, K, block_m, block_n, num_warps, split_k,
                                        ctypes.byref(out))
    check(rc, "specq_kernel_attrs_query")
    return out
