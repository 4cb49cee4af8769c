"""fp64 model of the prefill kernel's rounding points.

The MFMA prefill (hymt2sharp_amd/csrc/prefill_attn.hip) differs from the
fp32 reference in two roundings only: q after RoPE/norm, scaled by
log2(e)/sqrt(D), is rounded to the MFMA operand type, and each softmax
weight p = 2^(s - m) is rounded to that type before P*V, where m is the
running row maximum after the current 64-position kv tile (online softmax).
The row sum l accumulates the unrounded p.  Work items that split a q
block's kv range keep their own (m, l, O) and are merged with weights
2^(m_i - max m).

This model reproduces those roundings in fp64 so the GPU result can be
checked far tighter than against the fp32 oracle.  Test infrastructure only.
"""
from __future__ import annotations

import numpy as np

from hymt2sharp_amd import BF16, F16
from hymt2sharp_amd import synth as S

LOG2E = 1.4426950408889634
FLOOR2 = np.float32(-80.0 * LOG2E)


def round_to(x, dtype):
    x = np.asarray(x, dtype=np.float32)
    if dtype == BF16:
        return S.bf16_bits_to_f32(S.f32_to_bf16_bits(x)).reshape(x.shape).astype(np.float64)
    if dtype == F16:
        return x.astype(np.float16).astype(np.float64)
    raise ValueError(dtype)


def tiles_of(pos0, qb, seq):
    last = min(pos0 + qb * 32 + 31, pos0 + seq - 1)
    return last // 64 + 1


def split_ranges(pos0, seq, kv_heads, cap=None):
    """Tile ranges per q block, mirroring hymt_attn_prefill's work items."""
    nqb = (seq + 31) // 32
    max_tiles = max(tiles_of(pos0, qb, seq) for qb in range(nqb))
    if cap is None:
        cap = max_tiles
        pairs = nqb * kv_heads
        if pairs < 256:
            per = (256 + pairs - 1) // pairs
            cap = max(4, (max_tiles + per - 1) // per)
    out = []
    for qb in range(nqb):
        nt = tiles_of(pos0, qb, seq)
        ns = (nt + cap - 1) // cap
        out.append([(s * nt // ns, (s + 1) * nt // ns) for s in range(ns)])
    return out


def prefill_model(q_hat, cache_k, cache_v, heads, kv_heads, head_dim, pos0, seq, dtype, cap=None):
    """q_hat [seq][heads*D] (after RoPE/norm, fp32); cache_k/v [L][kv_heads*D]
    as fp32 values of the stored cache.  Returns out [seq][heads*D] (fp64)."""
    D = head_dim
    G = heads // kv_heads
    L = pos0 + seq
    qscale = np.float32(LOG2E / np.sqrt(D))
    qm = round_to(np.asarray(q_hat, np.float32).reshape(seq, heads, D) * qscale, dtype)
    K = np.asarray(cache_k, np.float64)[:L].reshape(L, kv_heads, D)
    V = np.asarray(cache_v, np.float64)[:L].reshape(L, kv_heads, D)
    out = np.zeros((seq, heads, D))
    ranges = split_ranges(pos0, seq, kv_heads, cap)
    for h in range(heads):
        kvh = h // G
        s_all = qm[:, h, :] @ K[:, kvh, :].T                 # [seq][L]
        qpos = pos0 + np.arange(seq)
        vis = np.arange(L)[None, :] <= qpos[:, None]
        for qb, splits in enumerate(ranges):
            rows = np.arange(qb * 32, min(qb * 32 + 32, seq))
            parts = []
            for (t0, t1) in splits:
                m = np.full(len(rows), float(FLOOR2))
                l = np.zeros(len(rows))
                o = np.zeros((len(rows), D))
                for t in range(t0, t1):
                    cols = np.arange(t * 64, min(t * 64 + 64, L))
                    st = s_all[np.ix_(rows, cols)]
                    vv = vis[np.ix_(rows, cols)]
                    mt = np.where(vv, st, -np.inf).max(axis=1)
                    mnew = np.maximum(m, mt)
                    alpha = np.exp2(m - mnew)
                    p = np.where(vv, np.exp2(np.maximum(st - mnew[:, None], float(FLOOR2))), 0.0)
                    l = l * alpha + p.sum(axis=1)
                    o = o * alpha[:, None] + round_to(p, dtype) @ V[cols, kvh, :]
                    m = mnew
                parts.append((m, l, o))
            if len(parts) == 1:
                m, l, o = parts[0]
                out[rows, h, :] = np.where(l[:, None] > 0, o / np.where(l > 0, l, 1)[:, None], 0)
            else:
                M = np.max([p[0] for p in parts], axis=0)
                lt = sum(np.exp2(p[0] - M) * p[1] for p in parts)
                ot = sum(np.exp2(p[0] - M)[:, None] * p[2] for p in parts)
                out[rows, h, :] = ot / lt[:, None]
    return out.reshape(seq, heads * D)
