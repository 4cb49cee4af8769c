"""Decode attention on the GPU vs the CPU oracle (HunyuanDenseModel.DecodeAttention
restated in oracle/hymt_oracle.c).

Tolerance: the north star's fp32 bound, max rel <= 1e-3 with the reference's
own metric (AttentionTests.cs:151-164), for every KV dtype: the oracle stores
K/V in the same dtype with the same RNE rounding, so only fp32 arithmetic
order differs.
"""
import numpy as np
import pytest

from hymt2sharp_amd import BF16, F16, F32, HipBackend
from hymt2sharp_amd import synth as S
from tests.attn_cases import (BASE, D, EPS, HKV, HQ, SCALE, cache_rows, max_rel, new_token,
                              oracle_cache)

pytestmark = pytest.mark.gpu

TOL = 1e-3
DT = {"f32": F32, "f16": F16, "bf16": BF16}


def make_backend(layers, cap, dtype, rope_dim=D):
    return HipBackend(0).configure(HQ, HKV, D, rope_dim, BASE, EPS).create_cache(layers, cap, dtype)


def run_case(oracle, dtype, pos, norm, config=1, salt=0, outlier_frac=0.0, kscale=None, layer=0,
             layers=1, rope_dim=D):
    cap = pos + 1
    kb, vb = cache_rows(config, pos, dtype_scale=kscale, salt=salt, outlier_frac=outlier_frac)
    q, k, v, qnw, knw = new_token(config, salt, norm)
    be = make_backend(layers, cap, dtype, rope_dim)
    try:
        if pos:
            be.UploadKv(layer, 0, pos, kb, vb)
        got = be.DecodeAttention(layer, pos, q[0], k[0], v[0], qnw, knw)
        krow, vrow = be.ReadKv(layer, pos, 1)
    finally:
        be.Dispose()
    ck, cv = oracle_cache(kb, vb, cap, dtype)
    ref = oracle.decode_attention(q[0], k[0], v[0], qnw, knw, ck, cv, dtype, HQ, HKV, D, BASE,
                                  EPS, pos, rope_dim=rope_dim)
    return got, ref, (krow[0], vrow[0]), (oracle.from_storage(ck[pos], dtype),
                                          oracle.from_storage(cv[pos], dtype))


def ulp_close(a, b, dtype):
    """Appended rows.  f16/bf16: equal up to one unit in the last place of the
    storage dtype (the fp32 RoPE/norm values may straddle a rounding boundary).
    f32: within 8 fp32 ulps of the row's largest element, the cancellation
    error of x0*c - x1*s computed in a different association order."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    if dtype == F32:
        return bool(np.max(np.abs(a - b)) <= 8 * 2.0 ** -24 * np.max(np.abs(b)))
    mant = {F16: 10, BF16: 7}[dtype]
    ulp = np.maximum(np.abs(b), 6.1e-5 if dtype == F16 else 1e-30) * 2.0 ** -mant
    return bool(np.all(np.abs(a - b) <= ulp * 1.0001))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("norm", [None, "ones"])
def test_config1_decode_513(oracle, hip_available, dtype, norm):
    """Config 1: one layer, cache of 512 + token at 512, fp32 (literal) and bf16 (reference)."""
    dt = DT[dtype]
    got, ref, (kr, vr), (kr_ref, vr_ref) = run_case(oracle, dt, 512, norm, config=1)
    assert max_rel(got, ref) <= TOL, max_rel(got, ref)
    assert ulp_close(kr, kr_ref, dt) and ulp_close(vr, vr_ref, dt)


@pytest.mark.parametrize("layer", [0, 31])
def test_config2_decode_4097_fp16(oracle, hip_available, layer):
    """Config 2 layer: fp16 KV, pos 4096, QK RMSNorm with gamma ~ U(0.9, 1.1)."""
    got, ref, (kr, vr), (kr_ref, vr_ref) = run_case(oracle, F16, 4096, "gamma", config=2,
                                                    salt=layer, layer=layer, layers=32)
    assert max_rel(got, ref) <= TOL, max_rel(got, ref)
    assert ulp_close(kr, kr_ref, F16) and ulp_close(vr, vr_ref, F16)


@pytest.mark.parametrize("L", [1024, 4096, 16384, 32768])
def test_config5_long_context_outliers(oracle, hip_available, L):
    """Config 5: K ~ N(0,1) with 0.1% of positions x30 (peaked logits), fp16 KV."""
    got, ref, _, _ = run_case(oracle, F16, L - 1, None, config=5, kscale=1.0, outlier_frac=0.001)
    assert max_rel(got, ref) <= TOL, max_rel(got, ref)


@pytest.mark.parametrize("dtype,pos", [("f16", 20480), ("bf16", 24639), ("f32", 40000), ("f16", 65600),
                                       ("bf16", 16448), ("f32", 32000)])
def test_decode_page_runs(oracle, hip_available, dtype, pos):
    """Past 256 cached pages each split takes its pages in runs: 2 at a time
    for an even count per split (24639 -> 385 pages, 4 per split, the last
    split holding one), 1 at a time for an odd one (20480 -> 3 per split,
    65600 -> 9, the last split holding 8); 16448 (257 pages) is the first
    context past the 2-page splits.  fp32 caches always take runs of one
    (32000 -> 500 pages, 4 per split)."""
    dt = DT[dtype]
    got, ref, (kd, vd), (kr, vr) = run_case(oracle, dt, pos, "gamma", salt=pos)
    assert max_rel(got, ref) <= TOL, max_rel(got, ref)
    assert ulp_close(kd, kr, dt) and ulp_close(vd, vr, dt)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("pos", [0, 1, 62, 63, 64, 65, 127, 128, 200, 8191, 8192, 8250])
def test_decode_edges(oracle, hip_available, dtype, pos):
    """Page boundaries, a single position, and the multi-page splits past 8192."""
    dt = DT[dtype]
    got, ref, (kr, vr), (kr_ref, vr_ref) = run_case(oracle, dt, pos, "gamma", config=7, salt=pos)
    assert max_rel(got, ref) <= TOL, max_rel(got, ref)
    assert ulp_close(kr, kr_ref, dt) and ulp_close(vr, vr_ref, dt)


def test_decode_chain_matches_oracle(oracle, hip_available):
    """Decode steps appending one token each (the Forward([token]) loop):
    every step's output and the whole cache match the oracle run step by step."""
    steps = 70
    be = make_backend(1, steps, F32)
    ck, cv = oracle_cache(np.zeros((0, HKV * D), np.uint16), np.zeros((0, HKV * D), np.uint16),
                          steps, F32)
    worst = 0.0
    try:
        for p in range(steps):
            q, k, v, qnw, knw = new_token(8, p, "gamma")
            got = be.DecodeAttention(0, p, q[0], k[0], v[0], qnw, knw)
            ref = oracle.decode_attention(q[0], k[0], v[0], qnw, knw, ck, cv, F32, HQ, HKV, D,
                                          BASE, EPS, p)
            worst = max(worst, max_rel(got, ref))
        kd, vd = be.ReadKv(0, 0, steps)
    finally:
        be.Dispose()
    assert worst <= TOL, worst
    assert all(ulp_close(kd[p], ck[p], F32) for p in range(steps))
    assert np.array_equal(vd, cv)


def test_decode_repeat_is_deterministic(hip_available):
    """Re-running the same step (same pos) rewrites the same row and gives
    the same output bit for bit (the split merge order is fixed)."""
    kb, vb = cache_rows(9, 3000)
    q, k, v, qnw, knw = new_token(9, 0, "gamma")
    be = make_backend(1, 3001, F16)
    try:
        be.UploadKv(0, 0, 3000, kb, vb)
        a = be.DecodeAttention(0, 3000, q[0], k[0], v[0], qnw, knw)
        b = be.DecodeAttention(0, 3000, q[0], k[0], v[0], qnw, knw)
    finally:
        be.Dispose()
    assert np.array_equal(a, b)


@pytest.mark.parametrize("rope_dim", [64, 32, 2, 0])
@pytest.mark.parametrize("dtype,pos", [("f16", 4096), ("bf16", 700), ("f32", 513), ("f16", 9000)])
def test_decode_partial_rotary(oracle, hip_available, rope_dim, dtype, pos):
    """rope_dim < head_dim (ModelConfig.RopeDim, ModelConfig.cs:30): dims at
    or past rope_dim pass through the rotation (Ops.cs:100, 157); rope_dim 0
    rotates nothing.  These run the kernels' partial-rotary path (partner and
    table index per element), single- and multi-page splits."""
    dt = DT[dtype]
    got, ref, (kr, vr), (kr_ref, vr_ref) = run_case(oracle, dt, pos, "gamma", config=9,
                                                    salt=rope_dim + pos, rope_dim=rope_dim)
    assert max_rel(got, ref) <= TOL, max_rel(got, ref)
    assert ulp_close(kr, kr_ref, dt) and ulp_close(vr, vr_ref, dt)


def _appended_rows(oracle, k, v, knw, dtype, rope_dim=D):
    """The rows DecodeAttention appends for new k/v rows k[t], v[t] at
    positions t = 0..n-1: K after RoPE at t (Ops.cs:98-168) and, with a gamma,
    RMSNorm (Ops.cs:12-90), both rounded to the cache dtype; V raw, rounded."""
    n = k.shape[0]
    kr = oracle.neox_rope(k.reshape(n, HKV, D), 0, BASE, rope_dim)
    if knw is not None:
        kr = oracle.rmsnorm(kr, knw, EPS)
    return oracle.to_storage(kr.reshape(n, HKV * D), dtype), oracle.to_storage(v, dtype)


def _not_bf16(a):
    """Fraction of fp32 elements with a nonzero low half (not bf16-representable)."""
    bits = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return float(np.mean((bits & 0xFFFF) != 0))


@pytest.mark.parametrize("norm", [None, "ones"])
def test_config1_fp32_cache_filled_by_appends(oracle, hip_available, norm):
    """Config 1 with a genuinely fp32 cache: the 512 cached rows come from 512
    decode appends (the Forward([token]) loop), so K and V hold fp32 values
    whose low halves are not zero and the kernel's bf16 hi + lo split of the
    cached operands carries both halves.  Every step, and the config-1 step at
    position 512 (L = 513, one split of 8 pages), within max rel 1e-3 of the
    oracle run step by step over its own fp32 cache."""
    steps = 512
    be = make_backend(1, steps + 1, F32)
    ck, cv = oracle_cache(np.zeros((0, HKV * D), np.uint16), np.zeros((0, HKV * D), np.uint16),
                          steps + 1, F32)
    worst = 0.0
    try:
        for p in range(steps):
            q, k, v, qnw, knw = new_token(11, p, norm)
            got = be.DecodeAttention(0, p, q[0], k[0], v[0], qnw, knw)
            ref = oracle.decode_attention(q[0], k[0], v[0], qnw, knw, ck, cv, F32, HQ, HKV, D,
                                          BASE, EPS, p)
            worst = max(worst, max_rel(got, ref))
        kd, vd = be.ReadKv(0, 0, steps)
        assert _not_bf16(kd) > 0.99 and _not_bf16(vd) > 0.99, (_not_bf16(kd), _not_bf16(vd))
        q, k, v, qnw, knw = new_token(1, 0, norm)
        got = be.DecodeAttention(0, steps, q[0], k[0], v[0], qnw, knw)
    finally:
        be.Dispose()
    ref = oracle.decode_attention(q[0], k[0], v[0], qnw, knw, ck, cv, F32, HQ, HKV, D, BASE, EPS, steps)
    assert worst <= TOL, worst
    assert max_rel(got, ref) <= TOL, max_rel(got, ref)
    assert all(ulp_close(kd[p], ck[p], F32) for p in range(steps))
    assert np.array_equal(vd, cv[:steps])


@pytest.mark.parametrize("pos", [16500, 20551])
def test_fp32_cache_runs_filled_by_appends(oracle, hip_available, pos):
    """The fp32 run path (past 256 cached pages every split takes its pages
    one at a time: 16500 -> 258 pages, 3 per split; 20551 -> 322 pages, 3 per
    split, the last holding one) over a cache written only by decode appends,
    so every cached K and V row holds fp32 values with nonzero low halves.
    The device cache is checked row by row against the oracle's appended rows
    and the step at `pos` against the oracle's decode over its own cache."""
    salt = pos
    be = make_backend(1, pos + 1, F32)
    kin = S.normal(S.seed(12, S.KNEW, salt), (pos, HKV * D), SCALE)
    vin = S.normal(S.seed(12, S.VNEW, salt), (pos, HKV * D), SCALE)
    _, _, _, qnw, knw = new_token(12, salt, "gamma")
    qfill = S.normal(S.seed(12, S.Q, salt), (HQ * D,), SCALE)
    try:
        dq, dk, dv = be.alloc(qfill.nbytes), be.alloc(kin.nbytes), be.alloc(vin.nbytes)
        dg, dout = be.alloc(2 * D * 4), be.alloc(HQ * D * 4)
        be.upload(dq, qfill)
        be.upload(dk, kin)
        be.upload(dv, vin)
        be.upload(dg, np.concatenate([qnw, knw]).astype(np.float32))
        row = HKV * D * 4
        for p in range(pos):  # enqueued back to back; one output buffer
            be.decode_dev(0, p, dq, dk + p * row, dv + p * row, dg, dg + D * 4, dout)
        be.sync()
        kd, vd = be.ReadKv(0, 0, pos)
        q, k, v, _, _ = new_token(12, salt + 1, None)
        got = be.DecodeAttention(0, pos, q[0], k[0], v[0], qnw, knw)
    finally:
        be.Dispose()
    kref, vref = _appended_rows(oracle, kin, vin, knw, F32)
    assert _not_bf16(kd) > 0.99 and _not_bf16(vd) > 0.99, (_not_bf16(kd), _not_bf16(vd))
    assert np.array_equal(vd, vref)
    kerr = np.max(np.abs(kd.astype(np.float64) - kref) / np.max(np.abs(kref), axis=1, keepdims=True))
    assert kerr <= 8 * 2.0 ** -24, kerr
    ck = oracle.new_cache(pos + 1, HKV, D, F32)
    cv = oracle.new_cache(pos + 1, HKV, D, F32)
    ck[:pos] = kref
    cv[:pos] = vref
    ref = oracle.decode_attention(q[0], k[0], v[0], qnw, knw, ck, cv, F32, HQ, HKV, D, BASE, EPS, pos)
    assert max_rel(got, ref) <= TOL, max_rel(got, ref)
