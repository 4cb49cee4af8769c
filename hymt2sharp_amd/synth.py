"""Seeded synthetic inputs of the benchmark configurations.

Generator: xoshiro256** seeded through SplitMix64 (the reference's sampler
RNG, Sampling.cs:375-409), in libhymt_synth.so.  Seed of a tensor is
0x48594D54 + 16*config + tensor_id with ids Q=0, Knew=1, Vnew=2, Kcache=3,
Vcache=4, gamma_q=5, gamma_k=6, outlier positions=7.
"""
from __future__ import annotations

import numpy as np

from . import _native as N

SEED_BASE = 0x48594D54
Q, KNEW, VNEW, KCACHE, VCACHE, GQ, GK, OUTLIERS = range(8)


def seed(config: int, tensor: int, salt: int = 0) -> int:
    return (SEED_BASE + 16 * config + tensor + (salt << 32)) & 0xFFFFFFFFFFFFFFFF


def normal(s: int, shape, scale: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    N.synth().hymt_synth_normal(s, out.ctypes.data, n, scale)
    return out.reshape(shape)


def uniform(s: int, shape, lo: float, hi: float) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    N.synth().hymt_synth_uniform(s, out.ctypes.data, n, lo, hi)
    return out.reshape(shape)


def index(s: int, n: int, modulus: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int64)
    N.synth().hymt_synth_index(s, out.ctypes.data, n, modulus)
    return out


def f32_to_bf16_bits(x) -> np.ndarray:
    """Ops.ConvertToBf16's integer RNE (Ops.cs:664-665), vectorised."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((b + np.uint32(0x7FFF) + ((b >> 16) & np.uint32(1))) >> 16).astype(np.uint16)


def bf16_bits_to_f32(h) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint32) << 16).view(np.float32)
