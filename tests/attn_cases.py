"""Inputs of the benchmark configurations (seeded) and the GPU-vs-oracle
comparison used by the GPU parity tests."""
from __future__ import annotations

import numpy as np

from hymt2sharp_amd import synth as S
from oracle import oracle as O

HQ, HKV, D = 16, 4, 128
KV_STRIDE = HKV * D
BASE, EPS = 10000.0, 1e-6
SCALE = 1.0 / np.sqrt(D)


def cache_rows(config, n, dtype_scale=None, salt=0, outlier_frac=0.0):
    """Existing cache rows [n][KV_STRIDE] as bf16 bit patterns (what UploadKv
    takes) for K and V.  K ~ N(0,1)*dtype_scale with an optional fraction of
    positions scaled x30."""
    ks = SCALE if dtype_scale is None else dtype_scale
    k = S.normal(S.seed(config, S.KCACHE, salt), (n, KV_STRIDE), ks)
    v = S.normal(S.seed(config, S.VCACHE, salt), (n, KV_STRIDE), SCALE)
    if outlier_frac > 0 and n > 0:
        cnt = max(1, int(outlier_frac * n))
        idx = S.index(S.seed(config, S.OUTLIERS, salt), cnt, n)
        k[idx] *= 30.0
    return S.f32_to_bf16_bits(k), S.f32_to_bf16_bits(v)


def new_token(config, salt=0, norm=False, seq=1):
    q = S.normal(S.seed(config, S.Q, salt), (seq, HQ * D), SCALE)
    k = S.normal(S.seed(config, S.KNEW, salt), (seq, KV_STRIDE), SCALE)
    v = S.normal(S.seed(config, S.VNEW, salt), (seq, KV_STRIDE), SCALE)
    qnw = knw = None
    if norm == "gamma":
        qnw = S.uniform(S.seed(config, S.GQ, salt), (D,), 0.9, 1.1)
        knw = S.uniform(S.seed(config, S.GK, salt), (D,), 0.9, 1.1)
    elif norm == "ones":
        qnw = np.ones(D, np.float32)
        knw = np.ones(D, np.float32)
    return q, k, v, qnw, knw


def oracle_cache(kbits, vbits, cap, dtype):
    """Oracle cache of `cap` rows holding the uploaded rows, converted to the
    cache dtype exactly as the device does (bf16 -> f32 -> dtype)."""
    ck = O.new_cache(cap, HKV, D, dtype)
    cv = O.new_cache(cap, HKV, D, dtype)
    n = kbits.shape[0]
    if n:
        ck[:n] = O.to_storage(S.bf16_bits_to_f32(kbits), dtype)
        cv[:n] = O.to_storage(S.bf16_bits_to_f32(vbits), dtype)
    return ck, cv


def max_rel(a, b):
    return O.rel_err(a, b)
