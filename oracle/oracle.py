"""ctypes binding of the CPU oracle (libhymt_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker of the HIP path.  The product
(hymt2sharp_amd) never imports this module.

Each wrapper names the reference function it restates; the C file cites the
reference lines.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# HYMT_ORACLE_LIB names another build of the same checker (the sanitized one of
# hymt2sharp_amd/build_san.py, under the CPU tests)
LIB_PATH = os.environ.get("HYMT_ORACLE_LIB") or os.path.join(HERE, "libhymt_oracle.so")

F32, F16, BF16 = 0, 1, 2
DTYPE_NAMES = {F32: "f32", F16: "f16", BF16: "bf16"}
_NP_STORAGE = {F32: np.float32, F16: np.uint16, BF16: np.uint16}

_lib = None


def build() -> None:
    """Compile libhymt_oracle.so with the Makefile beside this file."""
    subprocess.run(["make", "-s", "-C", HERE, "-B"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_fp = ctypes.POINTER(ctypes.c_float)
_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float


def _declare(L):
    L.orc_f32_to_bf16.restype = ctypes.c_uint16
    L.orc_f32_to_bf16.argtypes = [_f]
    L.orc_bf16_to_f32.restype = _f
    L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_f32_to_f16.restype = ctypes.c_uint16
    L.orc_f32_to_f16.argtypes = [_f]
    L.orc_f16_to_f32.restype = _f
    L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_convert.argtypes = [_vp, _vp, ctypes.c_long, _i]
    L.orc_fast_exp8.argtypes = [_vp, _vp]
    L.orc_rmsnorm.argtypes = [_vp, _vp, _vp, _i, _i, _f]
    L.orc_rope_table.argtypes = [_i, _f, _i, _vp, _vp]
    L.orc_neox_rope.argtypes = [_vp, _i, _i, _i, _i, _i, _f]
    L.orc_softmax_row.argtypes = [_vp, _i]
    L.orc_softmax_causal.argtypes = [_vp, _i, _i, _i, _i, _i]
    L.orc_attention_scores.argtypes = [_vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _i, _i, _f, _i, _i]
    L.orc_attention_decode.argtypes = [_vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _i, _i, _f, _i, _i]
    L.orc_attention_combine.argtypes = [_vp, _i, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _i]
    layer = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _f, _i]
    L.orc_decode_attention.argtypes = layer + [_vp, _i]
    L.orc_prefill_attention.argtypes = layer + [_i, _vp, _i]
    L.orc_forward_prefill_attention.argtypes = layer + [_i, _vp, _i]
    L.orc_attention_f64.argtypes = [_vp, _vp, _vp, _i, _i, _i, _i, _i, ctypes.c_double, _vp]
    L.orc_row_bytes.restype = ctypes.c_long
    L.orc_row_bytes.argtypes = [_i, _i]
    L.orc_dequant_row.argtypes = [_i, _vp, _i, _vp]
    L.orc_gemv.argtypes = [_i, _vp, _i, _i, _vp, _vp, _i]
    L.orc_cpu_q8k_gemv.argtypes = [_i, _vp, _i, _i, _vp, _vp, _i, _i]
    L.orc_cpu_decode_step.argtypes = [_vp, _i, _i, _vp, _i]


def _p(a):
    return None if a is None else a.ctypes.data_as(_vp)


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- conversions
def to_storage(x, dtype: int) -> np.ndarray:
    """Ops.ConvertToBf16 (Ops.cs:658-680), generalised to f32/f16/bf16 storage."""
    x = _c32(x)
    out = np.empty(x.shape, dtype=_NP_STORAGE[dtype])
    lib().orc_convert(_p(x), _p(out), x.size, dtype)
    return out


def from_storage(a: np.ndarray, dtype: int) -> np.ndarray:
    """Widen stored cache elements to fp32 (Ops.cs:688 for bf16)."""
    if dtype == F32:
        return np.asarray(a, dtype=np.float32)
    if dtype == BF16:
        return (np.asarray(a, dtype=np.uint32) << 16).view(np.float32)
    return np.asarray(a, dtype=np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16_bits(x) -> np.ndarray:
    return to_storage(x, F16)


def f32_to_bf16_bits(x) -> np.ndarray:
    return to_storage(x, BF16)


def f16_bits_to_f32(h) -> np.ndarray:
    L = lib()
    h = np.asarray(h, dtype=np.uint16).ravel()
    return np.array([L.orc_f16_to_f32(int(v)) for v in h], dtype=np.float32)


def fast_exp8(x) -> np.ndarray:
    """FastExp.ExpAvx2 (FastExp.cs:15-46) on 8 lanes."""
    x = _c32(x)
    assert x.size == 8
    y = np.empty(8, dtype=np.float32)
    lib().orc_fast_exp8(_p(x), _p(y))
    return y


# ---------------------------------------------------------------- pointwise ops
def rmsnorm(x, weight, eps: float) -> np.ndarray:
    """Ops.RmsNorm (Ops.cs:12-90) over the last axis."""
    x = _c32(x)
    dim = x.shape[-1]
    y = np.empty_like(x)
    w = None if weight is None else _c32(weight)
    lib().orc_rmsnorm(_p(x), _p(w), _p(y), x.size // dim, dim, eps)
    return y


def rope_table(half: int, base: float, cap: int):
    """Ops.EnsureRopeTable (Ops.cs:170-195)."""
    c = np.empty((cap, half), dtype=np.float32)
    s = np.empty((cap, half), dtype=np.float32)
    lib().orc_rope_table(half, base, cap, _p(c), _p(s))
    return c, s


def neox_rope(x, start_pos: int, base: float, rope_dim: int | None = None) -> np.ndarray:
    """Ops.NeoXRoPE (Ops.cs:98-168) on x[tokens][heads][head_dim]; returns a copy."""
    x = _c32(x).copy()
    tokens, heads, head_dim = x.shape
    lib().orc_neox_rope(_p(x), tokens, heads, head_dim, head_dim if rope_dim is None else rope_dim, start_pos, base)
    return x


def softmax_row(row) -> np.ndarray:
    """Ops.SoftmaxRow (Ops.cs:224-325); returns a copy."""
    r = _c32(row).copy()
    lib().orc_softmax_row(_p(r), r.size)
    return r


def softmax_causal(scores, start_pos: int, threads: int = 1) -> np.ndarray:
    """Ops.SoftmaxCausal (Ops.cs:198-221) on scores[heads][q_len][kv_len]; returns a copy."""
    s = _c32(scores).copy()
    heads, q_len, kv_len = s.shape
    lib().orc_softmax_causal(_p(s), heads, q_len, kv_len, start_pos, threads)
    return s


# ---------------------------------------------------------------- attention ops
def attention_scores(q, cache_k, kv_dtype, heads, kv_heads, head_dim, q_len, kv_len, scale,
                     start_pos, threads=1):
    """Ops.AttentionScores (Ops.cs:359-455); masked tail left at 0."""
    q = _c32(q)
    ck = np.ascontiguousarray(cache_k)
    sc = np.zeros((heads, q_len, kv_len), dtype=np.float32)
    lib().orc_attention_scores(_p(q), _p(ck), kv_dtype, _p(sc), heads, kv_heads, head_dim, q_len,
                               kv_len, heads * head_dim, kv_heads * head_dim, scale, start_pos,
                               threads)
    return sc


def attention_combine(cache_v, kv_dtype, scores, heads, kv_heads, head_dim, q_len, kv_len,
                      start_pos, threads=1):
    """Ops.AttentionCombine (Ops.cs:535-595)."""
    cv = np.ascontiguousarray(cache_v)
    sc = _c32(scores)
    out = np.zeros((q_len, heads * head_dim), dtype=np.float32)
    lib().orc_attention_combine(_p(cv), kv_dtype, _p(sc), _p(out), heads, kv_heads, head_dim,
                                q_len, kv_len, heads * head_dim, kv_heads * head_dim, start_pos,
                                threads)
    return out


def attention_decode(q, cache_k, cache_v, kv_dtype, heads, kv_heads, head_dim, kv_len, scale,
                     start_pos, threads=1):
    """Ops.AttentionDecode (Ops.cs:462-532)."""
    q = _c32(q)
    ck = np.ascontiguousarray(cache_k)
    cv = np.ascontiguousarray(cache_v)
    sc = np.zeros((heads, kv_len), dtype=np.float32)
    out = np.zeros(heads * head_dim, dtype=np.float32)
    lib().orc_attention_decode(_p(q), _p(ck), _p(cv), kv_dtype, _p(sc), _p(out), heads, kv_heads,
                               head_dim, kv_len, kv_heads * head_dim, scale, start_pos, threads)
    return out


def new_cache(cap: int, kv_heads: int, head_dim: int, kv_dtype: int) -> np.ndarray:
    return np.zeros((cap, kv_heads * head_dim), dtype=_NP_STORAGE[kv_dtype])


def decode_attention(q, k, v, qnw, knw, cache_k, cache_v, kv_dtype, heads, kv_heads, head_dim,
                     rope_base, eps, start, rope_dim=None, threads=1):
    """HunyuanDenseModel.DecodeAttention (Decode.cs:64-101), attention part.

    cache_k / cache_v are updated in place (row `start`); q/k are not modified.
    Returns out[heads*head_dim].
    """
    q = _c32(q).copy()
    k = _c32(k).copy()
    v = _c32(v)
    qnw = None if qnw is None else _c32(qnw)
    knw = None if knw is None else _c32(knw)
    out = np.zeros(heads * head_dim, dtype=np.float32)
    assert cache_k.flags.c_contiguous and cache_v.flags.c_contiguous
    lib().orc_decode_attention(_p(q), _p(k), _p(v), _p(qnw), _p(knw), _p(cache_k), _p(cache_v),
                               kv_dtype, heads, kv_heads, head_dim, head_dim if rope_dim is None else rope_dim,
                               rope_base, eps, start, _p(out), threads)
    return out


def prefill_attention(q, k, v, qnw, knw, cache_k, cache_v, kv_dtype, heads, kv_heads, head_dim,
                      rope_base, eps, start, rope_dim=None, threads=1, chunked=True):
    """PrefillAttention (Prefill.cs:38-89) with Forward's 1024-token chunking
    (HunyuanDenseModel.cs:342-355) when `chunked`.  Returns out[seq][heads*head_dim]."""
    q = _c32(q).copy()
    k = _c32(k).copy()
    v = _c32(v)
    seq = q.size // (heads * head_dim)
    qnw = None if qnw is None else _c32(qnw)
    knw = None if knw is None else _c32(knw)
    out = np.zeros((seq, heads * head_dim), dtype=np.float32)
    fn = lib().orc_forward_prefill_attention if chunked else lib().orc_prefill_attention
    fn(_p(q), _p(k), _p(v), _p(qnw), _p(knw), _p(cache_k), _p(cache_v), kv_dtype, heads, kv_heads,
       head_dim, head_dim if rope_dim is None else rope_dim, rope_base, eps, start, seq, _p(out), threads)
    return out


def attention_f64(q, cache_k_f32, cache_v_f32, heads, kv_heads, head_dim, start, seq, scale):
    """fp64 brute force (MetalGemvMicro.RunAttn, MetalGemvMicro.cs:292-384)."""
    q = _c32(q)
    ck = _c32(cache_k_f32)
    cv = _c32(cache_v_f32)
    out = np.zeros((seq, heads * head_dim), dtype=np.float64)
    lib().orc_attention_f64(_p(q), _p(ck), _p(cv), heads, kv_heads, head_dim, start, seq, scale,
                            _p(out))
    return out


def rel_err(a, b) -> float:
    """AttentionTests.AssertClose metric (AttentionTests.cs:151-164):
    max |a-b| / max(1e-3, |a|, |b|)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.maximum(1e-3, np.maximum(np.abs(a), np.abs(b)))
    return float(np.max(np.abs(a - b) / den)) if a.size else 0.0


# ---- quantized weight rows (hymt_quant.c) ------------------------------------

W_F32, W_F16, W_Q8_0, W_Q4_K, W_Q6_K, W_Q2_0C, W_STQ1_0 = 0, 1, 8, 12, 14, 40, 43


def row_bytes(wtype: int, n: int) -> int:
    return int(lib().orc_row_bytes(wtype, n))


def dequant(wtype: int, data, rows: int, cols: int) -> np.ndarray:
    """[rows][cols] fp32 values of a matrix stored as rows of GGUF blocks."""
    raw = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8))
    rb = row_bytes(wtype, cols)
    assert raw.size == rb * rows, (raw.size, rb, rows)
    out = np.empty((rows, cols), np.float32)
    for r in range(rows):
        if lib().orc_dequant_row(wtype, _p(raw[r * rb:(r + 1) * rb]), cols, _p(out[r])) != 0:
            raise ValueError(wtype)
    return out


def q8k_gemv(wtype: int, data, rows: int, cols: int, x, y=None, threads: int = 1) -> np.ndarray:
    """The reference's CPU projection (cpu_decode.c): x quantized to Q8_K,
    integer dots against Q4_K / Q6_K blocks; y given: accumulate."""
    raw = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8))
    x = np.ascontiguousarray(x, np.float32)
    acc = y is not None
    out = np.array(y, np.float32, copy=True) if acc else np.empty(rows, np.float32)
    if lib().orc_cpu_q8k_gemv(wtype, _p(raw), rows, cols, _p(x), _p(out), int(acc), threads) != 0:
        raise ValueError(wtype)
    return out


def gemv(wtype: int, data, rows: int, cols: int, x, y=None) -> np.ndarray:
    """y (+)= W x in double over the dequantized rows (y given: accumulate)."""
    raw = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8))
    x = np.ascontiguousarray(x, np.float32)
    acc = y is not None
    out = np.array(y, np.float32, copy=True) if acc else np.empty(rows, np.float32)
    if lib().orc_gemv(wtype, _p(raw), rows, cols, _p(x), _p(out), int(acc)) != 0:
        raise ValueError(wtype)
    return out
