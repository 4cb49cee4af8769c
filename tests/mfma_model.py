"""fp64 model of the prefill kernel's rounding points.

The MFMA prefill (hymt2sharp_amd/csrc/prefill_attn.hip) differs from the
fp32 reference in its roundings and its order of accumulation only:

* q after RoPE/norm, scaled by log2(e)/sqrt(D), is rounded to the MFMA
  operand type;
* each softmax weight p = 2^(s - m) is rounded to that type before P*V and
  the row sum l adds the rounded weights;
* m is a lazy running reference: it starts at the reference's -80 (natural
  log units) and moves up to the row's tile maximum (if higher) on a wave
  half's first 64-position tile and on any later tile where some row of the
  wave's 32 rows has s - m > 8 (then for every row); otherwise m stays, so p
  may reach 2^8;
* a wave's 32 rows are the 16-row q blocks b and nb-1-b of a block pair
  (the causal work of every pair is then about equal); the pair's kv range
  is that of its long block, the short block taking part in the tiles it
  attends to;
* the tiles of a work item alternate between two wave halves (even and odd
  tile offsets), each with its own (m, l, O), combined with weights
  2^(m_i - max m); work items that split a pair's kv range are combined
  the same way, each split item's O / l rounded to the operand type first
  (the partials are stored in it) and weighted by its l.

This model reproduces those steps in fp64 so the GPU result can be checked
far tighter than against the fp32 oracle.  Test infrastructure only.
"""
from __future__ import annotations

import numpy as np

from hymt2sharp_amd import BF16, F16
from hymt2sharp_amd import synth as S

LOG2E = 1.4426950408889634
ITEM_TILES = 1024  # kItemTiles: kv tiles per work item
FLOOR2 = np.float32(-80.0 * LOG2E)


def round_to(x, dtype):
    x = np.asarray(x, dtype=np.float32)
    if dtype == BF16:
        return S.bf16_bits_to_f32(S.f32_to_bf16_bits(x)).reshape(x.shape).astype(np.float64)
    if dtype == F16:
        return x.astype(np.float16).astype(np.float64)
    raise ValueError(dtype)


def block_tiles(pos0, b, seq):
    """kv tiles the 16-row q block b attends to."""
    last = min(pos0 + b * 16 + 15, pos0 + seq - 1)
    return last // 64 + 1


def pair_items(pos0, seq, kv_heads, cap=None):
    """Per block pair: (rows of the pair, its tile ranges), mirroring
    hymt_attn_prefill's work items.  Pair p holds the short block p and the
    long block nb-1-p (the middle block of an odd count alone)."""
    nb = (seq + 15) // 16
    npairs = (nb + 1) // 2
    max_tiles = max(block_tiles(pos0, nb - 1 - p, seq) for p in range(npairs))
    if cap is None:
        cap = max_tiles
        pairs = npairs * kv_heads
        if pairs < 128:
            per = (256 + pairs - 1) // pairs
            cap = max(4, (max_tiles + per - 1) // per)
    cap = min(cap, ITEM_TILES)
    out = []
    for p in range(npairs):
        a, b = p, nb - 1 - p
        rows = list(range(b * 16, min(b * 16 + 16, seq)))
        if a < b:
            rows += list(range(a * 16, a * 16 + 16))
        nt = block_tiles(pos0, b, seq)
        ns = (nt + cap - 1) // cap
        out.append((np.array(rows), [(s * nt // ns, (s + 1) * nt // ns) for s in range(ns)]))
    return out


LAZY = 8.0


def _half_softmax(s_rows, vis_rows, tiles, L, V, dtype):
    """One wave half: online softmax over `tiles` for the q rows given.
    Returns (m, l, O) with l the sum of the rounded weights."""
    n, D = s_rows.shape[0], V.shape[1]
    m = np.full(n, float(FLOOR2))
    l = np.zeros(n)
    o = np.zeros((n, D))
    for k, t in enumerate(tiles):
        cols = np.arange(t * 64, min(t * 64 + 64, L))
        sm = np.where(vis_rows[:, cols], s_rows[:, cols] - m[:, None], -np.inf)
        mt = sm.max(axis=1)
        if k == 0 or np.any(mt > LAZY):
            d = np.maximum(mt, 0.0)
            m = m + d
            al = np.exp2(-d)
            l = l * al
            o = o * al[:, None]
            sm = sm - d[:, None]
        p = round_to(np.exp2(sm), dtype)
        l = l + p.sum(axis=1)
        o = o + p @ V[cols]
    return m, l, o


def _combine(parts):
    M = np.max([p[0] for p in parts], axis=0)
    w = [np.exp2(p[0] - M) for p in parts]
    lt = sum(wi * p[1] for wi, p in zip(w, parts))
    ot = sum(wi[:, None] * p[2] for wi, p in zip(w, parts))
    return M, lt, ot


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
    pairs = pair_items(pos0, seq, kv_heads, cap)
    qpos = pos0 + np.arange(seq)
    vis = np.arange(L)[None, :] <= qpos[:, None]
    for h in range(heads):
        kvh = h // G
        s_all = qm[:, h, :] @ K[:, kvh, :].T                 # [seq][L]
        for rows, splits in pairs:
            items = []
            for (t0, t1) in splits:
                halves = [_half_softmax(s_all[rows], vis[rows], range(t0 + hp, t1, 2), L,
                                        V[:, kvh, :], dtype) for hp in (0, 1)]
                items.append(_combine(halves))
            if len(items) > 1:  # partials stored as O / l in the operand type
                items = [(mi, li, li[:, None] * round_to(np.where(li[:, None] > 0, oi / np.where(li > 0, li, 1)[:, None], 0),
                                                         dtype)) for mi, li, oi in items]
            m, l, o = items[0] if len(items) == 1 else _combine(items)
            out[rows, h, :] = np.where(l[:, None] > 0, o / np.where(l > 0, l, 1)[:, None], 0)
    return out.reshape(seq, heads * D)
