"""hymt2sharp_amd -- HyMT2Sharp's attention path on AMD MI355X (gfx950).

RoPE + per-head Q/K RMSNorm, paged KV-cache append, and GQA softmax(QK^T)V
for causal prefill and single-token decode, as hand-written HIP kernels
behind the C ABI in include/hymt_hip.h (libhymt_hip.so).

    from hymt2sharp_amd import HipBackend, create_backend
"""
from ._native import BF16, F16, F32, PAGE_TOKENS  # noqa: F401
from .backend import (ArgumentError, HipBackend, InvalidOperationError,  # noqa: F401
                      NotSupportedError, PlatformNotSupportedError, create_backend,
                      device_count)

__all__ = [
    "HipBackend", "create_backend", "device_count", "F32", "F16", "BF16", "PAGE_TOKENS",
    "ArgumentError", "NotSupportedError", "PlatformNotSupportedError", "InvalidOperationError",
]
