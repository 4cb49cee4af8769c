"""Prefill side of ForwardStep on the GPU through the C ABI: the row kernels
(RMSNorm, SwiGLU and rounding into bf16), the dense bf16 weight copies, the
bf16 GEMMs (hipBLASLt) and the whole multi-token ForwardStep against the
oracle's decode steps over the same tokens (oracle/model.py).

Bounds: row kernels within one bf16 ulp of the oracle's fp32/double value
rounded to bf16 (the fp32 sums may fall either side of a rounding edge);
rounding of fp32 input bit-exact; dense copies bit-exact for all but a few
values at rounding edges; GEMMs within 1e-5 of sum |x w| per output against
a double product of the same bf16 operands.  Prefill logits: the weights and
activations enter the GEMMs as bf16 (relative error 2^-9 each), so the
logits carry a stated bound of 1.5e-2 of the largest logit after two layers
(measured 1e-3 to 5e-3), against 1e-4 for the fp32 decode path."""
import numpy as np
import pytest

from hymt2sharp_amd import HipBackend
from hymt2sharp_amd import _native as N
from hymt2sharp_amd import synth as S
from hymt2sharp_amd.model import DeviceModel, ModelConfig, Tensor
from oracle import oracle as O
from oracle.model import OracleModel

pytestmark = pytest.mark.gpu


def bf16_bits(x):
    return S.f32_to_bf16_bits(np.asarray(x, np.float32))


def bf16_val(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def ulp_diff(a_bits, b_bits):
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    return np.abs(a - b)  # same-sign values: one bit pattern step = one ulp


@pytest.fixture
def be(hip_available):
    b = HipBackend(0)
    yield b
    b.Dispose()


def dev(be, arr):
    p = be.alloc(max(arr.nbytes, 4))
    be.upload(p, arr)
    return p


def test_rows_rmsnorm_swiglu_and_rounding(be):
    rng = np.random.default_rng(3)
    m, n = 37, 2048
    x = (rng.standard_normal((m, n)) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    dx, dw, do = dev(be, x), dev(be, w), be.alloc(m * n * 2)
    be.rows_rmsnorm(dx, m, n, dw, 1e-5, do)
    be.sync()
    got = be.download(np.empty((m, n), np.uint16), do)
    ref = bf16_bits(O.rmsnorm(x, w, 1e-5))
    assert ulp_diff(got, ref).max() <= 1 and np.mean(got == ref) > 0.99
    # SwiGLU: gate then up per row
    F = 6144
    gu = (rng.standard_normal((m, 2 * F)) * 4).astype(np.float32)
    dgu, dact = dev(be, gu), be.alloc(m * F * 2)
    be.rows_swiglu(dgu, m, F, dact)
    be.sync()
    got = be.download(np.empty((m, F), np.uint16), dact)
    g, u = gu[:, :F].astype(np.float64), gu[:, F:].astype(np.float64)
    ref = bf16_bits((g / (1 + np.exp(-g)) * u).astype(np.float32))
    assert ulp_diff(got, ref).max() <= 1 and np.mean(got == ref) > 0.99
    # the same over a bf16 gate/up (a bf16 GEMM output)
    gub = bf16_bits(gu)
    dgub = dev(be, gub)
    be.rows_swiglu_bf16(dgub, m, F, dact)
    be.sync()
    got = be.download(np.empty((m, F), np.uint16), dact)
    gv = bf16_val(gub).astype(np.float64)
    g, u = gv[:, :F], gv[:, F:]
    ref = bf16_bits((g / (1 + np.exp(-g)) * u).astype(np.float32))
    assert ulp_diff(got, ref).max() <= 1 and np.mean(got == ref) > 0.99
    be.free(dgub)
    # rounding: bit-exact RNE (Ops.cs:664-665)
    be.to_bf16(dx, m * n, do)
    be.sync()
    got = be.download(np.empty((m, n), np.uint16), do)
    assert np.array_equal(got, bf16_bits(x))
    for p in (dx, dw, do, dgu, dact):
        be.free(p)


@pytest.mark.parametrize("m,n", [
    (1, 4),        # one float4: a wave per row, lanes past the row reload it
    (9, 1000),     # 250 float4s: the last wave column partly empty; ragged row count
    (37, 2048),    # the model's rows
    (8, 4096),     # a wave per row, 16 float4s per lane
    (5, 4100),     # past 4096: a workgroup per row
    (3, 8192),
])
def test_rows_rmsnorm_shapes(be, m, n):
    """Every row-length class of hymt_rows_rmsnorm against the oracle's
    RMSNorm, rounded to bf16: within one bf16 ulp (the sum order differs)."""
    rng = np.random.default_rng(m * 10007 + n)
    x = (rng.standard_normal((m, n)) * 2).astype(np.float32)
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    dx, dw, do = dev(be, x), dev(be, w), be.alloc(m * n * 2 + 64)
    be.upload(do, np.full(m * n + 32, 0x7FC1, np.uint16))  # a canary past the rows
    be.rows_rmsnorm(dx, m, n, dw, 1e-5, do)
    be.sync()
    got = be.download(np.empty(m * n + 32, np.uint16), do)
    ref = bf16_bits(O.rmsnorm(x, w, 1e-5)).reshape(m, n)
    assert ulp_diff(got[:m * n].reshape(m, n), ref).max() <= 1
    assert np.all(got[m * n:] == 0x7FC1)
    for p in (dx, dw, do):
        be.free(p)


@pytest.mark.parametrize("m,F,offset,scale", [
    (37, 6144, 0, 4.0),   # 16-byte path, the model's width
    (3, 520, 0, 4.0),     # 16-byte path, rows that end mid-workgroup
    (6, 1024, 0, 12.0),   # 16-byte path, gates to about +-50, plus the extremes below
    (5, 1004, 0, 4.0),    # F not a multiple of 8: the 8-byte kernel
    (4, 6144, 8, 4.0),    # input 8 bytes off 16-byte alignment: the 8-byte kernel
])
def test_rows_swiglu_bf16_paths(be, m, F, offset, scale):
    """Both SwiGLU kernels over a bf16 gate/up against the float64 form
    rounded to bf16: within one bf16 ulp."""
    rng = np.random.default_rng(F + m)
    gu = (rng.standard_normal((m, 2 * F)) * scale).astype(np.float32)
    # gates where e^-g overflows fp32 (result -0 * u) or vanishes (result g u)
    gu[0, :6] = [-200.0, -100.0, -90.0, 90.0, 100.0, 200.0]
    gu[0, F:F + 6] = 1.0
    gub = bf16_bits(gu).reshape(m, 2 * F)
    base = be.alloc(gub.nbytes + 64)
    be.upload(base + offset, gub)
    dact = be.alloc(m * F * 2 + 64)
    be.upload(dact, np.full(m * F + 32, 0x7FC1, np.uint16))
    be.rows_swiglu_bf16(base + offset, m, F, dact)
    be.sync()
    got = be.download(np.empty(m * F + 32, np.uint16), dact)
    gv = bf16_val(gub)
    g, u = gv[:, :F], gv[:, F:]
    with np.errstate(over="ignore"):  # fp32 semantics: e^-g = inf gives -0
        ref = bf16_bits(g / (np.float32(1) + np.exp(-g)) * u).reshape(m, F)
    assert ulp_diff(got[:m * F].reshape(m, F), ref).max() <= 1
    assert np.all(got[m * F:] == 0x7FC1)
    be.free(base)
    be.free(dact)


@pytest.mark.parametrize("wtype", [N.W_Q4_K, N.W_Q6_K, N.W_Q8_0, N.W_Q2_0C, N.W_STQ1_0, N.W_F16])
def test_dense_copy_and_embed_rows(be, wtype):
    rows, cols = 300, 2048
    raw = S.random_weight(500 + wtype, wtype, rows, cols)
    full = O.dequant(wtype, raw, rows, cols)
    w = be.weight_upload(wtype, rows, cols, raw)
    try:
        be.weight_dense(w)
        be.weight_dense(w)  # a second call keeps the copy
        info = be.weight_info(w)
        assert info["device_bytes"] >= rows * cols * 2
        ids = np.array([0, 299, 7, 7, 150], np.int32)
        out = be.alloc(ids.size * cols * 4)
        be.embed_rows(w, ids, out)
        got = be.download(np.empty((ids.size, cols), np.float32), out)
        assert np.all(np.abs(got - full[ids]) <= 2e-7 * np.abs(full[ids]).max(axis=1, keepdims=True))
        with pytest.raises(N.ArgumentError):
            be.embed_rows(w, np.array([rows], np.int32), out)
        be.free(out)
    finally:
        be.weight_free(w)


@pytest.mark.parametrize("m", [1, 37, 256])
def test_gemm_matches_double_product(be, m):
    rows, cols = 640, 2048
    raw = S.random_weight(900 + m, N.W_Q4_K, rows, cols)
    wd = bf16_val(bf16_bits(O.dequant(N.W_Q4_K, raw, rows, cols))).astype(np.float64)
    rng = np.random.default_rng(m)
    xb = bf16_bits(rng.standard_normal((m, cols)).astype(np.float32))
    x = bf16_val(xb).astype(np.float64)
    y0 = rng.standard_normal((m, rows)).astype(np.float32)
    w = be.weight_upload(N.W_Q4_K, rows, cols, raw)
    be.weight_dense(w)
    dxb, dy, dy16 = dev(be, xb), dev(be, y0), be.alloc(m * rows * 2)
    try:
        mag = np.abs(x) @ np.abs(wd).T
        ref = x @ wd.T
        # fp32 out, all rows
        be.gemm(w, dxb, m, dy)
        be.sync()
        got = be.download(np.empty((m, rows), np.float32), dy)
        assert np.all(np.abs(got - ref) <= 1e-5 * mag + 1e-6)
        # accumulate into y
        be.upload(dy, y0)
        be.gemm(w, dxb, m, dy, accumulate=True)
        be.sync()
        got = be.download(np.empty((m, rows), np.float32), dy)
        assert np.all(np.abs(got - (ref + y0)) <= 1e-5 * (mag + np.abs(y0)) + 1e-6)
        # a row range, bf16 out
        be.gemm(w, dxb, m, dy16, row0=128, nrows=256, out_bf16=True)
        be.sync()
        got = bf16_val(be.download(np.empty((m, 256), np.uint16), dy16)).astype(np.float64)
        sub, smag = ref[:, 128:384], mag[:, 128:384]
        assert np.all(np.abs(got - sub) <= 2.0 ** -8 * np.abs(sub) + 1e-5 * smag + 1e-6)
        with pytest.raises(N.ArgumentError):
            be.gemm(w, dxb, m, dy, row0=600, nrows=64)
        with pytest.raises(N.ArgumentError):
            be.gemm(w, dxb, m, dy, accumulate=True, out_bf16=True)
    finally:
        for p in (dxb, dy, dy16):
            be.free(p)
        be.weight_free(w)


def test_gemm_needs_dense_copy(be):
    raw = S.random_weight(1, N.W_Q8_0, 64, 2048)
    w = be.weight_upload(N.W_Q8_0, 64, 2048, raw)
    d = be.alloc(64 * 2048 * 4)
    try:
        with pytest.raises(N.InvalidOperationError):
            be.gemm(w, d, 1, d)
    finally:
        be.free(d)
        be.weight_free(w)


CFG = ModelConfig(num_layers=2, hidden_size=2048, ffn_size=6144, num_heads=16, num_kv_heads=4,
                  head_dim=128, vocab_size=512, rope_base=10000.0, rope_dim=128, eps=1e-5)
PREFILL_BOUND = 1.5e-2


@pytest.mark.parametrize("case", [
    dict(seed=3, types={"attn": [N.W_Q4_K, N.W_Q8_0], "ffn": [N.W_Q6_K, N.W_Q2_0C],
                        "embd": N.W_Q6_K, "out": N.W_STQ1_0}, kv=N.BF16, m=40, chunk=16,
         v_override=N.W_F16),
    dict(seed=4, types={"attn": N.W_STQ1_0, "ffn": N.W_Q4_K, "embd": N.W_Q8_0}, kv=N.F16, m=70,
         chunk=1024, tied=True),
])
def test_prefill_forward_matches_oracle(be, monkeypatch, case):
    monkeypatch.setattr(DeviceModel, "PREFILL_CHUNK", case["chunk"])
    t = S.random_model(case["seed"], CFG, case["types"], tied=case.get("tied", False))
    if "v_override" in case:  # layer 1's q/k/v types differ: three GEMMs, packed prefill
        name = "blk.1.attn_v.weight"
        r, c = t[name].rows, t[name].cols
        t[name] = Tensor(case["v_override"], r, c, S.random_weight(77, case["v_override"], r, c))
    om = OracleModel(CFG, t, 128, case["kv"])
    be.LoadModel(t, CFG, max_tokens=128, kv_dtype=case["kv"])
    toks = list(np.random.default_rng(case["seed"]).integers(0, CFG.vocab_size, case["m"]))
    got = be.ForwardStep(toks, 0)
    ref = om.forward(toks, 0)
    err = np.max(np.abs(got - ref)) / np.max(np.abs(ref))
    print(f"prefill m={case['m']} rel {err:.2e}", flush=True)
    assert err <= PREFILL_BOUND
    # the K/V rows the prefill wrote: the next decode step reads all of them
    got = be.ForwardStep([11], case["m"])
    ref = om.step(11, case["m"])
    err = np.max(np.abs(got - ref)) / np.max(np.abs(ref))
    print(f"decode after prefill rel {err:.2e}", flush=True)
    assert err <= PREFILL_BOUND


def test_strided_prefill_equals_packed(be):
    """q, k, v as column ranges of one [seq][q|k|v] buffer give the same
    outputs and cache rows as packed arrays."""
    H, KV, D, seq = 16, 4, 128, 70
    ld = (H + 2 * KV) * D
    rng = np.random.default_rng(5)
    qkv = bf16_bits((rng.standard_normal((seq, ld)) / np.sqrt(D)).astype(np.float32))
    q = np.ascontiguousarray(qkv[:, :H * D])
    k = np.ascontiguousarray(qkv[:, H * D:(H + KV) * D])
    v = np.ascontiguousarray(qkv[:, (H + KV) * D:])
    g = rng.uniform(0.9, 1.1, D).astype(np.float32)
    be.configure(H, KV, D, D, 10000.0, 1e-6).create_cache(2, 128, N.BF16)
    dq, dk, dv, dqkv, dg = dev(be, q), dev(be, k), dev(be, v), dev(be, qkv), dev(be, g)
    o1, o2 = be.alloc(seq * H * D * 4), be.alloc(seq * H * D * 4)
    try:
        be.prefill_dev(0, 0, seq, dq, dk, dv, N.BF16, dg, dg, o1)
        be.prefill_dev_ld(1, 0, seq, dqkv, ld, dqkv + 2 * H * D, dqkv + 2 * (H + KV) * D, ld, N.BF16,
                          dg, dg, o2)
        be.sync()
        a = be.download(np.empty((seq, H * D), np.float32), o1)
        b = be.download(np.empty((seq, H * D), np.float32), o2)
        assert np.array_equal(a, b)
        k0, v0 = be.ReadKv(0, 0, seq)
        k1, v1 = be.ReadKv(1, 0, seq)
        assert np.array_equal(k0, k1) and np.array_equal(v0, v1)
        with pytest.raises(N.ArgumentError):
            be.prefill_dev_ld(1, 0, seq, dqkv, H * D - 8, dqkv, dqkv, ld, N.BF16, None, None, o2)
        with pytest.raises(N.ArgumentError):
            N.check(be._lib.hymt_attn_prefill_ld(be._h, 1, 0, seq, dqkv, ld, dqkv, dqkv, ld, N.BF16,
                                                 None, None, o2, 0))
    finally:
        for p in (dq, dk, dv, dqkv, dg, o1, o2):
            be.free(p)


def _read_logits(be, m):
    return be.download(np.empty(CFG.vocab_size, np.float32), m.logits)


@pytest.mark.parametrize("n", [70, 2100])
def test_native_prefill_equals_composed_calls(be, n):
    """hymt_model_prefill (one C ABI call, 2048-row chunks) gives the same
    logits and cache rows, bit for bit, as the same sequence issued as
    separate C ABI calls (DeviceModel.prefill_composed), on one context (so
    both use the same GEMM algorithms).  n = 2100 runs two chunks."""
    cfg = ModelConfig(num_layers=2, vocab_size=512)
    t = S.random_model(8, cfg, {"attn": N.W_Q4_K, "ffn": N.W_Q8_0, "embd": N.W_Q6_K, "out": N.W_Q6_K})
    be.LoadModel(t, cfg, max_tokens=n + 64, kv_dtype=N.BF16)
    m = be._model
    toks = [int(x) for x in np.random.default_rng(n).integers(0, cfg.vocab_size, n)]
    m.prefill(toks, 0)
    be.sync()
    native = _read_logits(be, m)
    kv_native = [be.ReadKv(l, 0, n) for l in range(cfg.num_layers)]
    for i in range(0, n, DeviceModel.PREFILL_CHUNK):
        m.prefill_composed(toks[i:i + DeviceModel.PREFILL_CHUNK], i)
    be.sync()
    composed = _read_logits(be, m)
    assert np.array_equal(native, composed)
    for l in range(cfg.num_layers):
        k, v = be.ReadKv(l, 0, n)
        assert np.array_equal(k, kv_native[l][0]) and np.array_equal(v, kv_native[l][1]), l
    # an argument error enqueues nothing
    with pytest.raises(N.ArgumentError):
        m.prefill([0, cfg.vocab_size], n)
    with pytest.raises(N.NotSupportedError):
        m.prefill([1] * 200, n)  # past the capacity


@pytest.mark.parametrize("fused", [True, False])
def test_deep_prefill_gate_up_rounding(be, fused):
    """The bf16 gate/up GEMM output (two extra bf16 roundings per FFN element
    against the reference's fp32 _pfGu, VulkanBackend.cs:595,604) and the
    fp32 one over a 6-layer model, with gate and up as one [gate; up] weight
    (one GEMM) or, of different types, as two: logits of both forms within
    the prefill bound of the oracle's fp32/double decode steps; their
    distances are printed."""
    cfg = ModelConfig(num_layers=6, vocab_size=512)
    t = S.random_model(12, cfg, {"attn": N.W_Q4_K, "ffn": N.W_Q4_K, "embd": N.W_Q6_K, "out": N.W_Q6_K})
    if not fused:
        for l in range(cfg.num_layers):
            name = f"blk.{l}.ffn_up.weight"
            r, c = t[name].rows, t[name].cols
            t[name] = Tensor(N.W_Q8_0, r, c, S.random_weight(300 + l, N.W_Q8_0, r, c))
    toks = [int(x) for x in np.random.default_rng(12).integers(0, cfg.vocab_size, 24)]
    om = OracleModel(cfg, t, 64, N.BF16)
    ref = om.forward(toks, 0)
    be.LoadModel(t, cfg, max_tokens=64, kv_dtype=N.BF16)
    m = be._model
    errs = {}
    for f32 in (False, True):
        m.prefill(toks, 0, gate_up_f32=f32)
        be.sync()
        got = _read_logits(be, m)
        errs[f32] = np.max(np.abs(got - ref)) / np.max(np.abs(ref))
    print(f"6-layer prefill logits rel (fused {fused}): flag off {errs[False]:.2e}, flag on {errs[True]:.2e}",
          flush=True)
    assert errs[False] <= PREFILL_BOUND and errs[True] <= PREFILL_BOUND
