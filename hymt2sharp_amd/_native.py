"""ctypes binding of libhymt_hip.so (include/hymt_hip.h).

The library is built in-tree by hymt2sharp_amd/build.py.  Loading fails
loudly when it is missing: there is no other implementation to fall back to.
"""
from __future__ import annotations

import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
# HYMT_HIP_LIB names another build of the same library (the sanitized one of
# build_san.py, under the CPU tests)
LIB_PATH = os.environ.get("HYMT_HIP_LIB") or os.path.join(PKG, "libhymt_hip.so")
SYNTH_PATH = os.path.join(PKG, "libhymt_synth.so")

HYMT_OK = 0
HYMT_E_ARG = 1
HYMT_E_UNSUPPORTED = 2
HYMT_E_CAPACITY = 3
HYMT_E_NO_DEVICE = 4
HYMT_E_DEVICE = 5
HYMT_E_OOM = 6
HYMT_E_STATE = 7

F32, F16, BF16 = 0, 1, 2
DEVICE_NONE = -1
FLAG_DEVICE_PTRS = 1
PAGE_TOKENS = 64


class HipError(RuntimeError):
    """A failing libhymt_hip call; `status` is the hymt_status code."""

    def __init__(self, status: int, msg: str):
        super().__init__(f"[{status}] {msg}")
        self.status = status


class NotSupportedError(HipError):
    """NotSupportedException in the reference (shape, dtype or capacity)."""


class ArgumentError(HipError, ValueError):
    """ArgumentException in the reference."""


class PlatformNotSupportedError(HipError):
    """PlatformNotSupportedException: no usable device."""


class InvalidOperationError(HipError):
    """InvalidOperationException: driver failure or call out of order."""


_EXC = {
    HYMT_E_ARG: ArgumentError,
    HYMT_E_UNSUPPORTED: NotSupportedError,
    HYMT_E_CAPACITY: NotSupportedError,
    HYMT_E_NO_DEVICE: PlatformNotSupportedError,
    HYMT_E_DEVICE: InvalidOperationError,
    HYMT_E_OOM: MemoryError,
    HYMT_E_STATE: InvalidOperationError,
}

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float

# name -> argtypes (every function returns int)
SIGNATURES = {
    "hymt_abi_version": [],
    "hymt_device_count": [ctypes.POINTER(_i)],
    "hymt_create": [_i, ctypes.POINTER(_vp)],
    "hymt_destroy": [_vp],
    "hymt_set_attn_config": [_vp, _i, _i, _i, _i, _f, _f],
    "hymt_kv_create": [_vp, _i, _i, _i],
    "hymt_kv_info": [_vp, ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_i)],
    "hymt_kv_map": [_vp, _i, _i],
    "hymt_kv_page": [_vp, _i, ctypes.POINTER(_i)],
    "hymt_kv_set_len": [_vp, _i],
    "hymt_kv_harvest": [_vp, _vp, _i, _i],
    "hymt_kv_restore": [_vp, _vp, _i, _i, ctypes.POINTER(_i)],
    "hymt_kv_store_info": [_vp, ctypes.POINTER(_i), ctypes.POINTER(_i)],
    "hymt_kv_upload": [_vp, _i, _i, _i, _vp, _vp],
    "hymt_kv_read": [_vp, _i, _i, _i, _vp, _vp],
    "hymt_attn_decode": [_vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_uint],
    "hymt_attn_decode_noalloc": [_vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp],
    "hymt_attn_prefill": [_vp, _i, _i, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, ctypes.c_uint],
    "hymt_attn_prefill_ld": [_vp, _i, _i, _i, _vp, _i, _vp, _vp, _i, _i, _vp, _vp, _vp, ctypes.c_uint],
    "hymt_sync": [_vp],
    "hymt_timing_get": [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_long), ctypes.POINTER(ctypes.c_double)],
    "hymt_timing_reset": [_vp],
    "hymt_timing_enable": [_vp, _i],
    "hymt_get_stream": [_vp, ctypes.POINTER(_vp)],
    "hymt_dev_alloc": [_vp, ctypes.c_size_t, ctypes.POINTER(_vp)],
    "hymt_dev_free": [_vp, _vp],
    "hymt_memcpy": [_vp, _vp, _vp, ctypes.c_size_t, _i],
    "hymt_graph_begin": [_vp],
    "hymt_graph_end": [_vp, ctypes.POINTER(_vp)],
    "hymt_graph_launch": [_vp, _vp],
    "hymt_graph_destroy": [_vp, _vp],
    "hymt_weight_upload": [_vp, _i, _i, _i, _vp, ctypes.c_size_t, ctypes.POINTER(_vp)],
    "hymt_weight_free": [_vp, _vp],
    "hymt_weight_info": [_vp, ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_i),
                         ctypes.POINTER(ctypes.c_size_t)],
    "hymt_gemv": [_vp, _vp, _vp, _vp, _i, _vp, ctypes.c_float],
    "hymt_embed": [_vp, _vp, _i, _vp],
    "hymt_weight_dense": [_vp, _vp],
    "hymt_gemm": [_vp, _vp, _i, _i, _vp, _i, _vp, _i],
    "hymt_embed_rows": [_vp, _vp, _vp, _i, _vp],
    "hymt_rows_rmsnorm": [_vp, _vp, _i, _i, _vp, ctypes.c_float, _vp],
    "hymt_rows_swiglu": [_vp, _vp, _i, _i, _vp],
    "hymt_rows_swiglu_bf16": [_vp, _vp, _i, _i, _vp],
    "hymt_gemm_swiglu": [_vp, _vp, _vp, _vp, _i, _vp],
    "hymt_to_bf16": [_vp, _vp, ctypes.c_size_t, _vp],
    "hymt_model_create": [_vp, _i, _i, _i, _i, ctypes.c_float, ctypes.POINTER(_vp)],
    "hymt_model_set_layer": [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    "hymt_model_set_io": [_vp, _vp, _vp, _vp],
    "hymt_model_decode": [_vp, _i, _i, _vp],
    "hymt_model_prefill": [_vp, _vp, _i, _i, _vp, ctypes.c_uint],
    "hymt_model_destroy": [_vp],
}

# weight types (GgmlTensorType codes) and gemv flags, as in include/hymt_hip.h
W_F32, W_F16, W_Q8_0, W_Q4_K, W_Q6_K, W_Q2_0C, W_STQ1_0 = 0, 1, 8, 12, 14, 40, 43
GEMV_ACCUMULATE, GEMV_IN_RMSNORM, GEMV_IN_SWIGLU, GEMV_OUT_SWIGLU = 1, 2, 4, 8
GEMM_ACCUMULATE, GEMM_OUT_BF16 = 1, 2
PREFILL_GATE_UP_F32 = 1

_lib = None
_synth = None


def lib() -> ctypes.CDLL:
    """Load libhymt_hip.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built; run python -m hymt2sharp_amd.build")
        L = ctypes.CDLL(LIB_PATH)
        L.hymt_last_error.restype = ctypes.c_char_p
        L.hymt_last_error.argtypes = []
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = _i
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != HYMT_OK:
        msg = lib().hymt_last_error().decode(errors="replace")
        exc = _EXC.get(status, HipError)
        if exc is MemoryError:
            raise MemoryError(msg)
        raise exc(status, msg)


def synth() -> ctypes.CDLL:
    global _synth
    if _synth is None:
        if not os.path.exists(SYNTH_PATH):
            raise ImportError(f"{SYNTH_PATH} is not built; run python -m hymt2sharp_amd.build")
        S = ctypes.CDLL(SYNTH_PATH)
        S.hymt_synth_uniform.argtypes = [ctypes.c_uint64, _vp, ctypes.c_long, _f, _f]
        S.hymt_synth_normal.argtypes = [ctypes.c_uint64, _vp, ctypes.c_long, _f]
        S.hymt_synth_index.argtypes = [ctypes.c_uint64, _vp, ctypes.c_long, ctypes.c_int64]
        for f in (S.hymt_synth_uniform, S.hymt_synth_normal, S.hymt_synth_index):
            f.restype = None
        _synth = S
    return _synth
