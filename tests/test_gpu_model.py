"""The decode step on the GPU through the C ABI: the GEMV input modes
(RMSNorm and SwiGLU), the embedding row, and the whole hunyuan-dense layer
stack (HipBackend.LoadModel / ForwardStep, hymt2sharp_amd/model.py) against
the oracle's decode step (oracle/model.py) on seeded synthetic models with
mixed weight formats.

Bounds: GEMV results within 1e-5 of sum |w x| of the row (fp32 sums and
expf against double); embedding rows within 2e-7 of the row's largest value
(fp32 products, with or without contraction); logits within 1e-4 of the
largest logit after two layers (measured 1e-6 to 1e-5), where the K/V rows are rounded to bf16/fp16
from fp32 on the GPU and from double-accumulated sums in the oracle."""
import numpy as np
import pytest

from hymt2sharp_amd import HipBackend
from hymt2sharp_amd import _native as N
from hymt2sharp_amd import synth as S
from hymt2sharp_amd.model import ModelConfig, Tensor
from oracle import oracle as O
from oracle.model import OracleModel

pytestmark = pytest.mark.gpu

TYPES = [N.W_F32, N.W_F16, N.W_Q8_0, N.W_Q4_K, N.W_Q6_K, N.W_Q2_0C, N.W_STQ1_0]


def _with(be, arrays, fn):
    ptrs = [be.alloc(a.nbytes) for a in arrays]
    try:
        for p, a in zip(ptrs, arrays):
            be.upload(p, a)
        return fn(*ptrs)
    finally:
        for p in ptrs:
            be.free(p)


@pytest.mark.parametrize("wtype", [N.W_Q4_K, N.W_Q8_0, N.W_STQ1_0, N.W_F32])
@pytest.mark.parametrize("cols", [2048, 6144])
def test_gemv_rmsnorm_input(hip_available, wtype, cols):
    rows, eps = 300, 1e-5
    raw = S.random_weight(40 + wtype + cols, wtype, rows, cols)
    rng = np.random.default_rng(wtype + cols)
    x = (rng.standard_normal(cols) * 3).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    be = HipBackend(0)
    try:
        w = be.weight_upload(wtype, rows, cols, raw)
        y = np.zeros(rows, np.float32)

        def run(dx, dnw, dy):
            be.gemv(w, dx, dy, rmsnorm=dnw, eps=eps)
            be.sync()
            return be.download(np.empty(rows, np.float32), dy)
        got = _with(be, [x, nw, y], run)
        be.weight_free(w)
    finally:
        be.Dispose()
    n = O.rmsnorm(x[None, :], nw, eps)[0]
    ref = O.gemv(wtype, raw, rows, cols, n)
    mag = np.abs(O.dequant(wtype, raw, rows, cols).astype(np.float64)) @ np.abs(n.astype(np.float64))
    assert np.all(np.abs(got - ref) <= 1e-5 * mag + 1e-6), np.max(np.abs(got - ref) / mag)


@pytest.mark.parametrize("wtype", [N.W_Q4_K, N.W_Q6_K, N.W_Q2_0C, N.W_F16])
def test_gemv_swiglu_input_accumulates(hip_available, wtype):
    rows, cols = 2048, 6144
    raw = S.random_weight(90 + wtype, wtype, rows, cols)
    rng = np.random.default_rng(wtype)
    gu = (rng.standard_normal(2 * cols) * 4).astype(np.float32)
    y0 = rng.standard_normal(rows).astype(np.float32)
    be = HipBackend(0)
    try:
        w = be.weight_upload(wtype, rows, cols, raw)

        def run(dx, dy):
            be.gemv(w, dx, dy, accumulate=True, swiglu=True)
            be.sync()
            return be.download(np.empty(rows, np.float32), dy)
        got = _with(be, [gu, y0], run)
        be.weight_free(w)
    finally:
        be.Dispose()
    g, u = gu[:cols].astype(np.float64), gu[cols:].astype(np.float64)
    act = (g / (1 + np.exp(-g)) * u).astype(np.float32)
    ref = O.gemv(wtype, raw, rows, cols, act, y=y0)
    mag = np.abs(O.dequant(wtype, raw, rows, cols).astype(np.float64)) @ np.abs(act) + np.abs(y0)
    assert np.all(np.abs(got - ref) <= 1e-5 * mag + 1e-6), np.max(np.abs(got - ref) / mag)


@pytest.mark.parametrize("wtype,F,cols,rms", [
    (N.W_Q4_K, 6145, 2048, True),   # 16 lanes a row: gate/up pairs swap by lane shuffle; a ragged last workgroup
    (N.W_Q4_K, 301, 2048, False),   # 64 lanes a row: pairs swap through LDS
    (N.W_Q6_K, 1000, 2048, True),
    (N.W_Q8_0, 301, 6144, True),
    (N.W_F32, 64, 2048, False),
])
def test_gemv_swiglu_output(hip_available, wtype, F, cols, rms):
    """HYMT_GEMV_OUT_SWIGLU: W = [gate; up] (2F rows), y[F] = silu(gate x') * (up x')."""
    rows, eps = 2 * F, 1e-5
    raw = S.random_weight(70 + wtype + F, wtype, rows, cols)
    rng = np.random.default_rng(F + cols)
    x = (rng.standard_normal(cols) * 2).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    be = HipBackend(0)
    try:
        w = be.weight_upload(wtype, rows, cols, raw)
        y = np.full(F + 7, 123.0, np.float32)

        def run(dx, dnw, dy):
            be.gemv(w, dx, dy, rmsnorm=dnw if rms else None, eps=eps, swiglu_out=True)
            be.sync()
            out = be.download(np.empty(F + 7, np.float32), dy)
            with pytest.raises(N.ArgumentError):
                be.gemv(w, dx, dy, accumulate=True, swiglu_out=True)
            return out
        got = _with(be, [x, nw, y], run)
        be.weight_free(w)
    finally:
        be.Dispose()
    assert np.all(got[F:] == 123.0), "wrote past the F outputs"
    got = got[:F]
    xn = O.rmsnorm(x[None, :], nw, eps)[0] if rms else x
    full = O.dequant(wtype, raw, rows, cols).astype(np.float64)
    ref = full @ xn.astype(np.float64)
    mag = np.abs(full) @ np.abs(xn.astype(np.float64))
    g, u = ref[:F], ref[F:]
    with np.errstate(over="ignore"):  # exp(-g) = inf for g << 0: silu(g) = -0
        act = g / (1 + np.exp(-g)) * u
    # the fp32 sums' errors (1e-5 of sum |w x| each) carried through silu (slope <= 1.1) and the product
    tol = 1.1 * np.abs(u) * 1e-5 * mag[:F] + np.abs(g) * 1e-5 * mag[F:] + 1e-6 * np.abs(act) + 1e-6
    assert np.all(np.abs(got - act) <= tol), np.max(np.abs(got - act) / tol)


def test_gemv_swiglu_output_needs_pairs(hip_available):
    be = HipBackend(0)
    try:
        w = be.weight_upload(N.W_F32, 3, 2048, np.zeros(3 * 2048, np.float32).tobytes())
        dx, dy = be.alloc(4 * 2048), be.alloc(16)
        with pytest.raises(N.ArgumentError):
            be.gemv(w, dx, dy, swiglu_out=True)
        be.free(dx)
        be.free(dy)
        be.weight_free(w)
    finally:
        be.Dispose()


@pytest.mark.parametrize("wtype", TYPES)
def test_embed_rows(hip_available, wtype):
    rows, cols = 97, 2048
    raw = S.random_weight(7 + wtype, wtype, rows, cols)
    full = O.dequant(wtype, raw, rows, cols)
    be = HipBackend(0)
    try:
        w = be.weight_upload(wtype, rows, cols, raw)
        out = be.alloc(4 * cols)
        try:
            for r in (0, 1, 50, rows - 1):
                be.embed(w, r, out)
                be.sync()
                got = be.download(np.empty(cols, np.float32), out)
                assert np.all(np.abs(got - full[r]) <= 2e-7 * np.max(np.abs(full[r]))), (wtype, r)
            with pytest.raises(N.ArgumentError):
                be.embed(w, rows, out)
        finally:
            be.free(out)
            be.weight_free(w)
    finally:
        be.Dispose()


CFG = ModelConfig(num_layers=2, hidden_size=2048, ffn_size=6144, num_heads=16, num_kv_heads=4,
                  head_dim=128, vocab_size=512, rope_base=10000.0, rope_dim=128, eps=1e-5)


def _model(seed, types, tied=False, v_override=None):
    t = S.random_model(seed, CFG, types, tied=tied)
    if v_override is not None:  # a layer whose q/k/v types differ: three GEMVs
        name = "blk.1.attn_v.weight"
        r, c = t[name].rows, t[name].cols
        t[name] = Tensor(v_override, r, c, S.random_weight(seed + 77, v_override, r, c))
    return t


@pytest.mark.parametrize("case", [
    dict(seed=1, types={"attn": [N.W_Q4_K, N.W_Q8_0], "ffn": [N.W_Q6_K, N.W_Q2_0C],
                        "embd": N.W_Q6_K, "out": N.W_STQ1_0}, kv=N.BF16, v_override=N.W_F16),
    dict(seed=2, types={"attn": N.W_Q2_0C, "ffn": [N.W_STQ1_0, N.W_Q4_K], "embd": N.W_Q8_0},
         kv=N.F16, tied=True),
])
def test_decode_steps_match_oracle(hip_available, case):
    t = _model(case["seed"], case["types"], case.get("tied", False), case.get("v_override"))
    om = OracleModel(CFG, t, 64, case["kv"])
    be = HipBackend(0)
    try:
        # without dense copies several tokens in one call run as decode steps
        be.LoadModel(t, CFG, max_tokens=64, kv_dtype=case["kv"], prefill=False)
        toks = [5, 300, 17, 511, 0, 42]
        for pos, tok in enumerate(toks):
            got = be.ForwardStep([tok], pos)
            ref = om.step(tok, pos)
            err = np.max(np.abs(got - ref)) / np.max(np.abs(ref))
            print(f"pos {pos} rel {err:.2e}", flush=True)
            assert err <= 1e-4, (pos, err)
        # several tokens in one call: the logits of the last one
        got = be.ForwardStep([9, 10, 11], len(toks))
        ref = om.forward([9, 10, 11], len(toks))
        assert np.max(np.abs(got - ref)) <= 1e-4 * np.max(np.abs(ref))
    finally:
        be.Dispose()


def test_forward_step_requires_model(hip_available):
    be = HipBackend(0)
    try:
        with pytest.raises(N.InvalidOperationError):
            be.ForwardStep([1], 0)
    finally:
        be.Dispose()


def test_misaligned_vectors_are_refused(hip_available):
    be = HipBackend(0)
    try:
        raw = S.random_weight(3, N.W_Q8_0, 16, 2048)
        w = be.weight_upload(N.W_Q8_0, 16, 2048, raw)
        d = be.alloc(4 * 4096)
        try:
            with pytest.raises(N.ArgumentError):
                be.gemv(w, d + 4, d)
            with pytest.raises(N.ArgumentError):
                be.gemv(w, d, d, rmsnorm=d + 8)
            with pytest.raises(N.ArgumentError):
                be.rows_rmsnorm(d + 4, 1, 2048, d, 1e-5, d)
            with pytest.raises(N.ArgumentError):
                be.to_bf16(d, 8, d + 2)
        finally:
            be.free(d)
            be.weight_free(w)
    finally:
        be.Dispose()


def test_native_step_equals_composed_calls(hip_available):
    """hymt_model_decode enqueues exactly the composed sequence of C ABI calls."""
    t = _model(5, {"attn": N.W_Q4_K, "ffn": [N.W_Q8_0, N.W_Q6_K], "embd": N.W_Q6_K}, tied=True,
               v_override=N.W_Q8_0)
    be = HipBackend(0)
    try:
        be.LoadModel(t, CFG, max_tokens=16, kv_dtype=N.BF16, prefill=False)
        m = be._model
        for pos, tok in enumerate([1, 400, 22, 3]):
            m.step_composed(tok, pos)
            a = be.download(np.empty(CFG.vocab_size, np.float32), m.logits)
            m.step(tok, pos)  # rewrites the same cache row with the same values
            b = be.download(np.empty(CFG.vocab_size, np.float32), m.logits)
            assert np.array_equal(a, b), pos
        with pytest.raises(N.ArgumentError):
            N.check(be._lib.hymt_model_decode(m._native, CFG.vocab_size, 4, m.logits))
        with pytest.raises(N.NotSupportedError):  # beyond the cache's capacity
            N.check(be._lib.hymt_model_decode(m._native, 1, 1000, m.logits))
        with pytest.raises(N.ArgumentError):
            N.check(be._lib.hymt_model_decode(m._native, 1, -1, m.logits))
        m.step(2, 4)  # the model still steps after the refusals
        be.sync()
    finally:
        be.Dispose()
