"""ctypes binding of libhyq.so (the C ABI declared in include/hyq.h).

The library is loaded from this package directory.  If it is missing the
import fails loudly: there is no CPU or eager fallback on the product path.
"""

from __future__ import annotations

import ctypes
import os
import threading
from ctypes import POINTER, Structure, c_float, c_int, c_int32, c_int64, c_size_t, c_uint16, c_void_p, c_int8, c_char_p, c_double

HERE = os.path.dirname(os.path.abspath(__file__))
# HYQ_LIBRARY names another build of the same sources (the phase-trace
# build, libhyq_trace.so); the default is the product library
LIB_PATH = os.environ.get("HYQ_LIBRARY") or os.path.join(HERE, "libhyq.so")

# the hyq_abi_version() these bindings (struct layouts, argument lists) match
ABI_VERSION = 7

HYQ_DT_Q_FP16 = 1
HYQ_DT_SEG_FP16 = 2
HYQ_DT_OUT_FP16 = 4

HYQ_OK = 0
HYQ_EINVAL = -22
HYQ_ENOTSUP = -95
HYQ_EDEVICE = -5
HYQ_ENOSPC = -28

# every symbol declared in include/hyq.h
EXPORTS = (
    "hyq_last_error",
    "hyq_abi_version",
    "hyq_quant_pack",
    "hyq_dequant",
    "hyq_legacy_dequant",
    "hyq_decode_workspace_size",
    "hyq_decode_hybrid",
    "hyq_decode_hybrid_noalloc",
    "hyq_decode_bf16_workspace_size",
    "hyq_decode_bf16",
    "hyq_decode_legacy_workspace_size",
    "hyq_decode_legacy",
    "hyq_vertical_select_workspace_size",
    "hyq_vertical_select",
    "hyq_freeze_workspace_size",
    "hyq_freeze_reorganise",
    "hyq_per_block_int8",
    "hyq_prefill_lists_workspace_size",
    "hyq_prefill_lists",
    "hyq_prefill_workspace_size",
    "hyq_prefill_hybrid",
    "hyq_prefill_unified",
    "hyq_prefill_hybrid_fp8qk",
)


class DecodeParams(Structure):
    """Mirror of `hyq_decode_params` (include/hyq.h)."""
    _fields_ = [
        ("q", c_void_p), ("q_stride", c_int64),
        ("out", c_void_p), ("out_stride", c_int64),
        ("k_packed", c_void_p), ("kp_stride_bh", c_int64), ("kp_stride_n", c_int64),
        ("v_packed", c_void_p), ("vp_stride_bh", c_int64), ("vp_stride_n", c_int64),
        ("k_scale", c_void_p), ("ks_stride_bh", c_int64),
        ("v_scale", c_void_p), ("vs_stride_bh", c_int64),
        ("n_quant", c_int64),
        ("seg_k", c_void_p * 3), ("seg_k_stride_bh", c_int64 * 3), ("seg_k_stride_n", c_int64 * 3),
        ("seg_v", c_void_p * 3), ("seg_v_stride_bh", c_int64 * 3), ("seg_v_stride_n", c_int64 * 3),
        ("seg_n", c_int64 * 3),
        ("bh_kv", c_int32), ("kv_repeat", c_int32), ("head_dim", c_int32),
        ("k_bits", c_int32), ("v_bits", c_int32),
        ("sm_scale", c_float),
        ("split_tokens", c_int32),
        ("seq_lens_quant", c_void_p), ("seq_lens_seg0", c_void_p),
        ("dtype_flags", c_int32),
    ]


class LegacyParams(Structure):
    """Mirror of `hyq_legacy_params` (include/hyq.h)."""
    _fields_ = [
        ("q", c_void_p), ("q_stride", c_int64),
        ("out", c_void_p), ("out_stride", c_int64),
        ("k_codes", c_void_p), ("kc_stride_bh", c_int64), ("kc_stride_n", c_int64),
        ("v_codes", c_void_p), ("vc_stride_bh", c_int64), ("vc_stride_n", c_int64),
        ("k_scale", c_void_p), ("ks_stride_bh", c_int64), ("ks_stride_g", c_int64),
        ("v_scale", c_void_p), ("vs_stride_bh", c_int64), ("vs_stride_g", c_int64),
        ("n", c_int64),
        ("group", c_int32),
        ("k_bits", c_int32), ("v_bits", c_int32),
        ("seg_k", c_void_p * 3), ("seg_k_stride_bh", c_int64 * 3),
        ("seg_v", c_void_p * 3), ("seg_v_stride_bh", c_int64 * 3),
        ("seg_n", c_int64 * 3),
        ("bh_kv", c_int32), ("kv_repeat", c_int32), ("head_dim", c_int32),
        ("sm_scale", c_float),
    ]


class PrefillParams(Structure):
    """Mirror of `hyq_prefill_params` (include/hyq.h)."""
    _fields_ = [
        ("q", c_void_p), ("q_stride_b", c_int64), ("q_stride_h", c_int64), ("q_stride_n", c_int64),
        ("k", c_void_p), ("k_stride_b", c_int64), ("k_stride_h", c_int64), ("k_stride_n", c_int64),
        ("v", c_void_p), ("v_stride_b", c_int64), ("v_stride_h", c_int64), ("v_stride_n", c_int64),
        ("vidx", c_void_p), ("vi_stride_b", c_int64), ("vi_stride_h", c_int64), ("vi_stride_t", c_int64),
        ("out", c_void_p), ("o_stride_b", c_int64), ("o_stride_h", c_int64), ("o_stride_n", c_int64),
        ("batch", c_int32), ("hq", c_int32), ("hkv", c_int32), ("head_dim", c_int32),
        ("n", c_int64), ("t", c_int64),
        ("window", c_int32), ("smooth_k", c_int32), ("pv_mode", c_int32),
        ("sm_scale", c_double),
        ("dtype_fp16", c_int32),
    ]


_lib = None
_lock = threading.Lock()


def _declare(lib):
    lib.hyq_last_error.restype = c_char_p
    lib.hyq_last_error.argtypes = []
    lib.hyq_abi_version.restype = c_int
    lib.hyq_abi_version.argtypes = []
    lib.hyq_quant_pack.restype = c_int
    lib.hyq_quant_pack.argtypes = [c_void_p, c_int32, c_int64, c_int64, c_int32, c_int64, c_int64, c_int32,
                                   c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p]
    lib.hyq_dequant.restype = c_int
    lib.hyq_dequant.argtypes = [c_void_p, c_int64, c_int64, c_int32, c_int64, c_int64, c_int32,
                                c_void_p, c_int64, c_void_p, c_int64, c_int64, c_void_p]
    lib.hyq_legacy_dequant.restype = c_int
    lib.hyq_legacy_dequant.argtypes = [c_void_p, c_int64, c_int64, c_int32, c_int64, c_int64, c_int32,
                                       c_void_p, c_int64, c_int64, c_int32, c_void_p, c_int64, c_int64, c_void_p]
    lib.hyq_decode_workspace_size.restype = c_size_t
    lib.hyq_decode_workspace_size.argtypes = [POINTER(DecodeParams)]
    lib.hyq_decode_hybrid.restype = c_int
    lib.hyq_decode_hybrid.argtypes = [POINTER(DecodeParams), c_void_p, c_size_t, c_void_p]
    lib.hyq_decode_hybrid_noalloc.restype = c_int
    lib.hyq_decode_hybrid_noalloc.argtypes = [POINTER(DecodeParams), c_void_p]
    lib.hyq_decode_bf16_workspace_size.restype = c_size_t
    lib.hyq_decode_bf16_workspace_size.argtypes = [c_int32, c_int32, c_int64, c_int32]
    lib.hyq_decode_bf16.restype = c_int
    lib.hyq_decode_bf16.argtypes = [c_void_p, c_int64, c_void_p, c_int64,
                                    c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64,
                                    c_int64, c_int32, c_int32, c_int32, c_float,
                                    c_void_p, c_size_t, c_void_p]
    lib.hyq_decode_legacy_workspace_size.restype = c_size_t
    lib.hyq_decode_legacy_workspace_size.argtypes = [POINTER(LegacyParams)]
    lib.hyq_decode_legacy.restype = c_int
    lib.hyq_decode_legacy.argtypes = [POINTER(LegacyParams), c_void_p, c_size_t, c_void_p]
    lib.hyq_vertical_select_workspace_size.restype = c_size_t
    lib.hyq_vertical_select_workspace_size.argtypes = [c_int32, c_int32, c_int64, c_int32]
    lib.hyq_vertical_select.restype = c_int
    lib.hyq_vertical_select.argtypes = [c_void_p, c_int64, c_int64, c_int64, c_int32, c_int32, c_int32,
                                        c_void_p, c_int64, c_int64, c_int64, c_int32, c_int64, c_int32,
                                        c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_size_t, c_void_p]
    lib.hyq_freeze_workspace_size.restype = c_size_t
    lib.hyq_freeze_workspace_size.argtypes = [c_int32, c_int64]
    lib.hyq_freeze_reorganise.restype = c_int
    lib.hyq_freeze_reorganise.argtypes = (
        [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_int64, c_int64,
         c_int32, c_int32, c_int64, c_int32, c_int32, c_void_p, c_int32, c_int32, c_int32, c_int32]
        + [c_void_p, c_int64, c_int64] * 2 + [c_void_p, c_int64] * 2 + [c_void_p, c_int64, c_int64] * 4
        + [c_void_p, c_size_t, c_void_p])
    lib.hyq_per_block_int8.restype = c_int
    lib.hyq_per_block_int8.argtypes = ([c_void_p, c_int32, c_int64, c_int64, c_int64, c_int32, c_int32, c_int64,
                                        c_int32, c_float, c_int32, c_void_p, c_int64, c_int64,
                                        c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p])
    lib.hyq_prefill_lists.restype = c_int
    lib.hyq_prefill_lists_workspace_size.restype = c_size_t
    lib.hyq_prefill_lists_workspace_size.argtypes = [c_int32, c_int32, c_int64, c_int64, c_int32]
    lib.hyq_prefill_lists.argtypes = [c_void_p, c_int64, c_int64, c_int64, c_int32, c_int32, c_int64, c_int64,
                                      c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_size_t, c_void_p]
    lib.hyq_prefill_workspace_size.restype = c_size_t
    lib.hyq_prefill_workspace_size.argtypes = [c_int32, c_int32, c_int32, c_int64, c_int64, c_int32, c_int32]
    lib.hyq_prefill_hybrid.restype = c_int
    lib.hyq_prefill_hybrid.argtypes = [POINTER(PrefillParams), c_void_p, c_size_t, c_void_p]
    lib.hyq_prefill_unified.restype = c_int
    lib.hyq_prefill_unified.argtypes = [POINTER(PrefillParams), c_void_p, c_size_t, c_void_p]
    lib.hyq_prefill_hybrid_fp8qk.restype = c_int
    lib.hyq_prefill_hybrid_fp8qk.argtypes = [POINTER(PrefillParams), c_void_p, c_size_t, c_void_p]


def lib():
    """The loaded libhyq.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(
                        f"{LIB_PATH} is missing: build it with `python -m hyquant_amd.build` "
                        "(there is no fallback implementation)")
                l = ctypes.CDLL(LIB_PATH)
                _declare(l)
                if l.hyq_abi_version() != ABI_VERSION:
                    raise RuntimeError(
                        f"{LIB_PATH} reports ABI {l.hyq_abi_version()}, these bindings need {ABI_VERSION}: "
                        "rebuild it with `python -m hyquant_amd.build`")
                _lib = l
    return _lib


def check(status: int, what: str) -> None:
    """Map a libhyq status to the reference's exception types."""
    if status == HYQ_OK:
        return
    msg = lib().hyq_last_error().decode(errors="replace")
    if status in (HYQ_EINVAL, HYQ_ENOTSUP):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed ({status}): {msg}")
