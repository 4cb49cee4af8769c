"""Independent fp64 numpy statements of the attention math, from the
definitions (NeoX RoPE, RMSNorm, causal GQA softmax attention), used to pin
the C oracle.  Nothing here is shared with oracle/hymt_oracle.c."""
from __future__ import annotations

import numpy as np


def rope_freqs_f32(half: int, base: float) -> np.ndarray:
    """The reference's fp32 frequency values 1 / base^(i/half) (Ops.cs:176-177),
    computed here in fp64 then rounded once: the same fp32 number up to the
    last-bit rounding of powf, which the tests allow for."""
    i = np.arange(half, dtype=np.float64)
    return (1.0 / np.power(np.float64(np.float32(base)), np.float32(i / half).astype(np.float64))).astype(np.float32)


def rope(x: np.ndarray, start: int, base: float, rope_dim: int | None = None) -> np.ndarray:
    """x [tokens][heads][D] -> rotated copy in fp64 (pairs (i, i+half))."""
    x = np.asarray(x, np.float64)
    tokens, heads, D = x.shape
    rd = D if rope_dim is None else rope_dim
    half = rd // 2
    freqs = rope_freqs_f32(half, base).astype(np.float64)
    pos = np.arange(start, start + tokens, dtype=np.float64)
    # the angle is formed in fp32 (Ops.cs:184): pos * freq rounded to fp32
    ang = (pos[:, None].astype(np.float32) * freqs[None, :].astype(np.float32)).astype(np.float64)
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    y = x.copy()
    x0, x1 = x[..., :half], x[..., half:rd]
    y[..., :half] = x0 * c - x1 * s
    y[..., half:rd] = x0 * s + x1 * c
    return y


def rmsnorm(x: np.ndarray, w, eps: float) -> np.ndarray:
    x = np.asarray(x, np.float64)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    y = x * r
    return y if w is None else y * np.asarray(w, np.float64)


def attention(q, k_cache, v_cache, heads, kv_heads, start, scale):
    """q [seq][heads][D]; caches [L][kv_heads][D]; query row t sees keys
    [0, start + t].  Plain softmax (no floor) in fp64."""
    q = np.asarray(q, np.float64)
    K = np.asarray(k_cache, np.float64)
    V = np.asarray(v_cache, np.float64)
    seq, _, D = q.shape
    G = heads // kv_heads
    out = np.zeros((seq, heads, D))
    for h in range(heads):
        kvh = h // G
        s = (q[:, h, :] @ K[:, kvh, :].T) * scale          # [seq][L]
        L = K.shape[0]
        vis = np.arange(L)[None, :] <= (start + np.arange(seq))[:, None]
        s = np.where(vis, s, -np.inf)
        s = s - s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[:, h, :] = p @ V[:, kvh, :]
    return out
