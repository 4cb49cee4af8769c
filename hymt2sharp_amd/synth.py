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


def random_model(s: int, cfg, types: dict | None = None, tied: bool = False) -> dict:
    """A hunyuan-dense model of the config's shape with seeded random weights:
    GGUF name -> model.Tensor.  `types` maps a role ("attn", "ffn", "embd",
    "out") to a weight type, or to a list of types taken per layer in turn
    (default Q4_K, and Q6_K for the embedding and output, as in the Q4_K_M
    files); norm weights are F32 ~ U(0.9, 1.1)."""
    from .model import Tensor
    t = {"attn": N.W_Q4_K, "ffn": N.W_Q4_K, "embd": N.W_Q6_K, "out": N.W_Q6_K}
    t.update(types or {})

    def ty(role, l=0):
        v = t[role]
        return v[l % len(v)] if isinstance(v, (list, tuple)) else v

    H, F, qd, kd = cfg.hidden_size, cfg.ffn_size, cfg.num_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim
    out, k = {}, [0]

    def m(name, wt, rows, cols):
        k[0] += 1
        out[name] = Tensor(wt, rows, cols, random_weight(s * 1000 + k[0], wt, rows, cols))

    def v(name, n):
        k[0] += 1
        out[name] = Tensor(N.W_F32, 1, n, uniform(s * 1000 + k[0], n, 0.9, 1.1).astype(np.float32).tobytes())

    for l in range(cfg.num_layers):
        p = f"blk.{l}."
        v(p + "attn_norm.weight", H)
        v(p + "ffn_norm.weight", H)
        v(p + "attn_q_norm.weight", cfg.head_dim)
        v(p + "attn_k_norm.weight", cfg.head_dim)
        m(p + "attn_q.weight", ty("attn", l), qd, H)
        m(p + "attn_k.weight", ty("attn", l), kd, H)
        m(p + "attn_v.weight", ty("attn", l), kd, H)
        m(p + "attn_output.weight", ty("attn", l), H, qd)
        m(p + "ffn_gate.weight", ty("ffn", l), F, H)
        m(p + "ffn_up.weight", ty("ffn", l), F, H)
        m(p + "ffn_down.weight", ty("ffn", l), H, F)
    m("token_embd.weight", ty("embd"), cfg.vocab_size, H)
    if not tied:
        m("output.weight", ty("out"), cfg.vocab_size, H)
    v("output_norm.weight", H)
    return out
