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


# ---- synthetic quantized weights ---------------------------------------------------
# (block byte counts per format, BlockLayout.cs:9-106; offset of the fp16
# scale fields that must hold a finite, moderate value)
_W_BLOCK = {8: (32, 34, (0,)), 12: (256, 144, (0, 2)), 14: (256, 210, (208,)), 40: (512, 130, (0,)),
            43: (256, 42, (40,))}


def random_weight(s: int, wtype: int, rows: int, cols: int) -> bytes:
    """rows x cols weights as rows of GGUF blocks: uniform random quant bytes,
    fp16 scales drawn from [2^-9, 2^-6) so the values stay O(1)."""
    rng = np.random.default_rng(s)
    if wtype == N.W_F32:
        return (rng.standard_normal(rows * cols) * 0.05).astype(np.float32).tobytes()
    if wtype == N.W_F16:
        return (rng.standard_normal(rows * cols) * 0.05).astype(np.float16).tobytes()
    vals, nbytes, scale_offs = _W_BLOCK[wtype]
    nb = rows * (cols // vals)
    raw = rng.integers(0, 256, (nb, nbytes), dtype=np.uint8)
    for off in scale_offs:
        d = (2.0 ** rng.uniform(-9, -6, nb)).astype(np.float16).view(np.uint16)
        raw[:, off] = d & 0xFF
        raw[:, off + 1] = d >> 8
    return raw.tobytes()
