"""The CPU oracle (oracle/hymt_oracle.c) pinned against the reference's own
test cases and tolerances, independent fp64 statements (tests/np_ref.py),
closed forms, invariants and committed fixtures (tests/golden/).

The reference ships no golden vectors for this path (its attention tests
compare against inline scalar loops, AttentionTests.cs:8-132); each check
below is chosen so that a plausible slip (sign, index, dropped term,
transposed operand, wrong floor) fails at least one of them.
"""
import math
import os

import numpy as np
import pytest

from hymt2sharp_amd import synth as S
from tests import np_ref

HERE = os.path.dirname(os.path.abspath(__file__))


# ------------------------------------------------------------------ conversions
def test_bf16_round_trip_all_patterns(oracle):
    """Every finite bf16 pattern widens and narrows back to itself."""
    h = np.arange(65536, dtype=np.uint16)
    f = oracle.from_storage(h, oracle.BF16)
    back = oracle.to_storage(f, oracle.BF16)
    finite = np.isfinite(f)
    assert np.array_equal(back[finite], h[finite])


def test_bf16_rne_matches_nearest_even(oracle):
    """Ops.cs:664-665 equals round-to-nearest-even for finite inputs: checked
    against an fp64 nearest-with-ties-to-even model on random and tie bits."""
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2 ** 32, size=400000, dtype=np.uint64).astype(np.uint32)
    ties = (rng.integers(0, 2 ** 16, size=20000, dtype=np.uint64).astype(np.uint32) << 16) | 0x8000
    bits = np.concatenate([bits, ties])
    f = bits.view(np.float32)
    bits = bits[np.isfinite(f) & (np.abs(f) < 3.0e38)]
    f = bits.view(np.float32)
    got = oracle.to_storage(f, oracle.BF16)
    lo = (bits >> 16).astype(np.uint32)
    hi = lo + 1
    flo = (lo << 16).view(np.float32).astype(np.float64)
    fhi = (hi << 16).view(np.float32).astype(np.float64)
    x = f.astype(np.float64)
    dlo, dhi = np.abs(x - flo), np.abs(fhi - x)
    want = np.where(dlo < dhi, lo, np.where(dhi < dlo, hi, np.where(lo % 2 == 0, lo, hi)))
    assert np.array_equal(got.astype(np.uint32), want.astype(np.uint32))


def test_f16_matches_numpy_rne(oracle):
    """fp32 -> fp16 equals numpy's IEEE RNE cast: all 2^16 halves round-trip,
    random finite floats, overflow, subnormals and exact ties."""
    h = np.arange(65536, dtype=np.uint16)
    hf = h.view(np.float16).astype(np.float32)
    ok = np.isfinite(hf)
    assert np.array_equal(oracle.to_storage(hf[ok], oracle.F16), h[ok])
    rng = np.random.default_rng(2)
    f = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 200000),
        np.array([65504, 65519.99, 65520, 1e6, -1e6, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                  2.0 ** -14, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, 0.0, -0.0], np.float32)]
    ).astype(np.float32)
    with np.errstate(over="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.to_storage(f, oracle.F16), want)


# ------------------------------------------------------------------ FastExp
def test_fast_exp_tracks_libm(oracle):
    """FastExpTests.ExpAvx2_TracksMathF (FastExpTests.cs:10-27): rel 2e-5 on
    x = (i-3)*1.25, extended over the softmax argument range [-80, 0]."""
    xs = [np.array([(i - 3) * 1.25 for i in range(8)], np.float32)]
    xs += [np.linspace(-80, 0, 8 * 64, dtype=np.float32).reshape(-1, 8)[j] for j in range(64)]
    for x in xs:
        got = oracle.fast_exp8(x).astype(np.float64)
        want = np.exp(x.astype(np.float64))
        assert np.max(np.abs(got - want) / np.maximum(1e-5, np.abs(want))) < 2e-5


# ------------------------------------------------------------------ RoPE / norm
def test_rope_table_closed_form(oracle):
    """Table rows equal cos/sin(pos * base^(-i/half)) up to the fp32 rounding
    of the frequency and of the angle (Ops.cs:176-186)."""
    half, base, cap = 64, 10000.0, 40000
    c, s = oracle.rope_table(half, base, cap)
    pos = np.arange(cap, dtype=np.float64)[:, None]
    freq = base ** (-np.arange(half, dtype=np.float64) / half)[None, :]
    ang = pos * freq
    tol = 4 * pos * freq * 2.0 ** -24 + 2 * np.abs(ang) * 2.0 ** -24 + 2e-7
    assert np.all(np.abs(c - np.cos(ang)) <= tol)
    assert np.all(np.abs(s - np.sin(ang)) <= tol)
    assert np.all(c[0] == 1) and np.all(s[0] == 0)


def test_neox_rope_against_fp64(oracle):
    x = S.normal(11, (5, 16, 128))
    freq = 10000.0 ** (-np.arange(64) / 64.0)
    amp = np.abs(x[..., :64]) + np.abs(x[..., 64:])
    for start in (0, 1, 511, 4096, 32760):
        got = oracle.neox_rope(x, start, 10000.0)
        want = np_ref.rope(x, start, 10000.0)
        # both sides form the angle pos*freq in fp32 from an fp32 freq that may
        # differ in its last bit (powf vs fp64 pow): |d angle| <= pos*freq*2^-22
        pos = (start + np.arange(5))[:, None, None]
        tol = amp * (pos * freq * 2.0 ** -22 + 2.0 ** -22) + 1e-6
        err = np.abs(got - want)
        assert np.all(err[..., :64] <= tol) and np.all(err[..., 64:] <= tol), start
        # rotation: each (i, i+64) pair keeps its length
        n0 = np.hypot(x[..., :64], x[..., 64:])
        n1 = np.hypot(got[..., :64], got[..., 64:])
        assert np.max(np.abs(n0 - n1)) < 1e-5
    assert np.array_equal(oracle.neox_rope(x, 0, 10000.0)[0], x[0])  # position 0 is the identity


def test_rope_partial_rotary_dims(oracle):
    """rope_dim < head_dim: dims >= rope_dim pass through (Ops.cs:100, 157)."""
    x = S.normal(12, (3, 4, 128))
    got = oracle.neox_rope(x, 17, 10000.0, rope_dim=64)
    want = np_ref.rope(x, 17, 10000.0, rope_dim=64)
    assert np.max(np.abs(got - want)) < 1e-5
    assert np.array_equal(got[..., 64:], x[..., 64:])
    # rope_dim 0 (a GGUF rope.dimension_count of 0, ModelConfig.cs:30): no rotation
    assert np.array_equal(oracle.neox_rope(x, 17, 10000.0, rope_dim=0), x)
    # rope_dim 2: one rotated pair per head
    got = oracle.neox_rope(x, 17, 10000.0, rope_dim=2)
    want = np_ref.rope(x, 17, 10000.0, rope_dim=2)
    assert np.max(np.abs(got - want)) < 1e-5 and np.array_equal(got[..., 2:], x[..., 2:])


def test_rmsnorm_closed_form(oracle):
    x = S.normal(13, (40, 128), 3.0)
    w = S.uniform(14, (128,), 0.9, 1.1)
    for eps in (1e-6, 1e-5):
        got = oracle.rmsnorm(x, w, eps)
        assert np.max(np.abs(got - np_ref.rmsnorm(x, w, eps))) < 2e-6
        unit = got / w
        assert np.max(np.abs(np.sqrt(np.mean(unit.astype(np.float64) ** 2, axis=1)) - 1)) < 1e-5
    assert np.max(np.abs(oracle.rmsnorm(x, None, 1e-6) - np_ref.rmsnorm(x, None, 1e-6))) < 2e-6


# ------------------------------------------------------------------ softmax
def test_softmax_causal_reference_case(oracle):
    """AttentionTests.SoftmaxCausal_MatchesScalarExp (AttentionTests.cs:75-116):
    heads 2, qLen 5, kvLen 8, uniform[-1,1) scores, metric rel 2e-3."""
    sc = S.uniform(8, (2, 5, 8), -1.0, 1.0)
    got = oracle.softmax_causal(sc, 0)
    want = np.zeros_like(sc, dtype=np.float64)
    for q in range(5):
        r = sc[:, q, :q + 1].astype(np.float64)
        e = np.exp(r - r.max(axis=1, keepdims=True))
        want[:, q, :q + 1] = e / e.sum(axis=1, keepdims=True)
    assert oracle.rel_err(got, want) < 2e-3
    for q in range(5):  # masked tail is exactly zero, visible part sums to 1
        assert np.all(got[:, q, q + 1:] == 0)
        assert np.allclose(got[:, q, :q + 1].sum(axis=1), 1, atol=1e-6)


def test_softmax_floor_semantics(oracle):
    """The -80 floor of Ops.SoftmaxRow: exp(max(x - max, -80)) with the max
    starting at -80 (Ops.cs:231, 245, 295)."""
    e80 = math.exp(-80.0)
    r = oracle.softmax_row(np.array([0.0, -200.0], np.float32))
    assert abs(r[1] - e80 / (1 + e80)) < 1e-40 and r[1] > 0   # floored, not 0
    # every logit below -80: the max stays -80, all weights floor to e^-80 -> uniform
    r = oracle.softmax_row(np.array([-200.0, -300.0, -250.0], np.float32))
    assert np.allclose(r, 1 / 3, atol=1e-7)
    r = oracle.softmax_row(np.full(11, -500.0, np.float32))      # >= 8: vector path
    assert np.allclose(r, 1 / 11, atol=1e-7)
    # shift invariance above the floor
    x = S.uniform(15, (37,), -5.0, 5.0)
    assert np.allclose(oracle.softmax_row(x), oracle.softmax_row(x + 7.0), atol=2e-7)


# ------------------------------------------------------------------ attention ops
def _reference_shapes():
    heads, kv_heads, dim, q_len, kv_len = 4, 2, 32, 3, 5
    q = S.uniform(1, (q_len, heads * dim), -1.0, 1.0)
    kb = S.f32_to_bf16_bits(S.uniform(2, (kv_len, kv_heads * dim), -1.0, 1.0))
    vb = S.f32_to_bf16_bits(S.uniform(3, (kv_len, kv_heads * dim), -1.0, 1.0))
    return heads, kv_heads, dim, q_len, kv_len, q, kb, vb


def test_scores_and_combine_reference_case(oracle):
    """AttentionTests.ScoresAndCombine_MatchScalar (AttentionTests.cs:8-72):
    heads 4 / kv 2, dim 32, qLen 3, kvLen 5, bf16 cache; scores rel 5e-5,
    combine rel 5e-4, checked here against fp64 products."""
    heads, kvh, dim, ql, kl, q, kb, vb = _reference_shapes()
    scale = 1.0 / math.sqrt(dim)
    sc = oracle.attention_scores(q, kb, oracle.BF16, heads, kvh, dim, ql, kl, scale, kl)
    K = S.bf16_bits_to_f32(kb).reshape(kl, kvh, dim).astype(np.float64)
    V = S.bf16_bits_to_f32(vb).reshape(kl, kvh, dim).astype(np.float64)
    Q = q.reshape(ql, heads, dim).astype(np.float64)
    want = np.einsum("qhd,khd->hqk", Q, K[:, np.arange(heads) // 2, :]) * scale
    assert oracle.rel_err(sc, want) < 5e-5
    out = oracle.attention_combine(vb, oracle.BF16, want.astype(np.float32), heads, kvh, dim, ql,
                                   kl, kl)
    want_o = np.einsum("hqk,khd->qhd", want, V[:, np.arange(heads) // 2, :]).reshape(ql, -1)
    assert oracle.rel_err(out, want_o) < 5e-4


@pytest.mark.parametrize("dtype", [0, 1, 2])
@pytest.mark.parametrize("kv_len", [1, 3, 4, 7, 64, 513])
def test_attention_decode_fp64(oracle, dtype, kv_len):
    """Ops.AttentionDecode vs fp64 softmax attention on the same stored cache."""
    heads, kvh, dim = 16, 4, 128
    q = S.normal(20 + kv_len, (heads * dim,), 1 / math.sqrt(dim))
    ck = oracle.to_storage(S.normal(21 + kv_len, (kv_len, kvh * dim), 1 / math.sqrt(dim)), dtype)
    cv = oracle.to_storage(S.normal(22 + kv_len, (kv_len, kvh * dim), 1 / math.sqrt(dim)), dtype)
    scale = 1 / math.sqrt(dim)
    got = oracle.attention_decode(q, ck, cv, dtype, heads, kvh, dim, kv_len, scale, kv_len - 1)
    want = np_ref.attention(q.reshape(1, heads, dim),
                            oracle.from_storage(ck, dtype).reshape(kv_len, kvh, dim),
                            oracle.from_storage(cv, dtype).reshape(kv_len, kvh, dim),
                            heads, kvh, kv_len - 1, scale)
    assert oracle.rel_err(got, want.reshape(-1)) < 1e-4


def test_attention_special_cases(oracle):
    heads, kvh, dim, L = 16, 4, 128, 40
    q = S.normal(30, (heads * dim,))
    v = S.normal(31, (L, kvh * dim))
    cv = oracle.to_storage(v, oracle.F32)
    # all keys equal -> uniform weights -> mean of the visible V rows
    ck = np.tile(S.normal(32, (1, kvh * dim)), (L, 1)).astype(np.float32)
    got = oracle.attention_decode(q, ck, cv, oracle.F32, heads, kvh, dim, L, 0.1, L - 1)
    mean = v.reshape(L, kvh, dim).mean(axis=0)[np.arange(heads) // 4]
    assert np.max(np.abs(got.reshape(heads, dim) - mean)) < 1e-5
    # one key aligned with q and huge -> that V row
    ck2 = np.zeros((L, kvh * dim), np.float32)
    for g in range(kvh):
        ck2[17, g * dim:(g + 1) * dim] = 50.0 * q.reshape(heads, dim)[4 * g]
    got = oracle.attention_decode(q, ck2, cv, oracle.F32, heads, kvh, dim, L, 1.0, L - 1)
    for h in range(0, heads, 4):
        assert np.max(np.abs(got.reshape(heads, dim)[h] - v.reshape(L, kvh, dim)[17, h // 4])) < 1e-5
    # rows past the causal bound do not matter
    a = oracle.attention_decode(q, ck, cv, oracle.F32, heads, kvh, dim, L, 0.1, 20)
    ck3, cv3 = ck.copy(), cv.copy()
    ck3[21:] = 99.0
    cv3[21:] = -7.0
    b = oracle.attention_decode(q, ck3, cv3, oracle.F32, heads, kvh, dim, L, 0.1, 20)
    assert np.array_equal(a, b)


# ------------------------------------------------------------------ layer orchestration
def _layer_inputs(seed, seq, norm=True):
    from tests.attn_cases import new_token
    return new_token(seed, 0, "gamma" if norm else None, seq=seq)


def test_decode_layer_against_fp64(oracle):
    """DecodeAttention order (RoPE -> norm -> append -> attend) against the
    fp64 statement with the same stored cache."""
    from tests.attn_cases import BASE, D, EPS, HKV, HQ, cache_rows, oracle_cache
    pos = 300
    kb, vb = cache_rows(40, pos)
    q, k, v, qnw, knw = _layer_inputs(41, 1)
    for dtype in (0, 1, 2):
        ck, cv = oracle_cache(kb, vb, pos + 1, dtype)
        got = oracle.decode_attention(q[0], k[0], v[0], qnw, knw, ck, cv, dtype, HQ, HKV, D, BASE,
                                      EPS, pos)
        qh = np_ref.rmsnorm(np_ref.rope(q.reshape(1, HQ, D), pos, BASE), qnw, EPS)
        kh = np_ref.rmsnorm(np_ref.rope(k.reshape(1, HKV, D), pos, BASE), knw, EPS)
        # the appended row is the rounded RoPE+norm k and the rounded raw v
        k_row = oracle.from_storage(ck[pos], dtype).astype(np.float64)
        assert np.max(np.abs(k_row - kh.reshape(-1))) <= 2.0 ** -7 * np.max(np.abs(kh)) + 1e-6
        assert np.array_equal(oracle.from_storage(cv[pos], dtype),
                              oracle.from_storage(oracle.to_storage(v[0], dtype), dtype))
        Kf = oracle.from_storage(ck, dtype).reshape(pos + 1, HKV, D)
        Vf = oracle.from_storage(cv, dtype).reshape(pos + 1, HKV, D)
        want = np_ref.attention(qh, Kf, Vf, HQ, HKV, pos, 1 / math.sqrt(D))
        assert oracle.rel_err(got, want.reshape(-1)) < 1e-4, dtype


def test_decode_equals_prefill_row_oracle(oracle):
    """Benchmark --verify-prefill invariant on the oracle itself."""
    from tests.attn_cases import BASE, D, EPS, HKV, HQ, oracle_cache
    seq = 70
    q, k, v, qnw, knw = _layer_inputs(42, seq)
    empty = np.zeros((0, HKV * D), np.uint16)
    ck, cv = oracle_cache(empty, empty, seq, oracle.BF16)
    pf = oracle.prefill_attention(q, k, v, qnw, knw, ck, cv, oracle.BF16, HQ, HKV, D, BASE, EPS, 0)
    ck2, cv2 = oracle_cache(empty, empty, seq, oracle.BF16)
    for p in range(seq):
        d = oracle.decode_attention(q[p], k[p], v[p], qnw, knw, ck2, cv2, oracle.BF16, HQ, HKV, D,
                                    BASE, EPS, p)
        assert oracle.rel_err(d, pf[p]) < 1e-4
    assert np.array_equal(ck, ck2) and np.array_equal(cv, cv2)


def test_forward_chunking_equals_monolithic(oracle):
    """Forward's 1024-token chunks (HunyuanDenseModel.cs:344-355) give the
    monolithic result up to summation order."""
    from tests.attn_cases import BASE, D, EPS, HKV, HQ, oracle_cache
    seq = 1100
    q, k, v, qnw, knw = _layer_inputs(43, seq)
    empty = np.zeros((0, HKV * D), np.uint16)
    c1 = oracle_cache(empty, empty, seq, oracle.F16)
    c2 = oracle_cache(empty, empty, seq, oracle.F16)
    a = oracle.prefill_attention(q, k, v, qnw, knw, *c1, oracle.F16, HQ, HKV, D, BASE, EPS, 0,
                                 threads=8, chunked=True)
    b = oracle.prefill_attention(q, k, v, qnw, knw, *c2, oracle.F16, HQ, HKV, D, BASE, EPS, 0,
                                 threads=8, chunked=False)
    assert oracle.rel_err(a, b) < 1e-5
    assert np.array_equal(c1[0], c2[0])


# ------------------------------------------------------------------ fixtures
def test_golden_fixtures(oracle):
    """Committed numpy-fp64 fixtures (tests/golden/make_golden.py)."""
    path = os.path.join(HERE, "golden", "attention_golden.npz")
    g = np.load(path, allow_pickle=False)
    names = sorted({k.split("__")[0] for k in g.files})
    assert names
    for n in names:
        f = {k.split("__")[1]: g[k] for k in g.files if k.startswith(n + "__")}
        heads, kvh, D, pos, seq, dtype = (int(x) for x in f["meta"])
        qnw = f["qnw"] if f["qnw"].size else None
        knw = f["knw"] if f["knw"].size else None
        ck = oracle.new_cache(pos + seq, kvh, D, dtype)
        cv = oracle.new_cache(pos + seq, kvh, D, dtype)
        if pos:
            ck[:pos] = oracle.to_storage(f["kcache"], dtype)
            cv[:pos] = oracle.to_storage(f["vcache"], dtype)
        if seq == 1:
            got = oracle.decode_attention(f["q"][0], f["k"][0], f["v"][0], qnw, knw, ck, cv, dtype,
                                          heads, kvh, D, 10000.0, 1e-6, pos)[None, :]
        else:
            got = oracle.prefill_attention(f["q"], f["k"], f["v"], qnw, knw, ck, cv, dtype, heads,
                                           kvh, D, 10000.0, 1e-6, pos)
        assert oracle.rel_err(got, f["out"]) < 2e-4, n
