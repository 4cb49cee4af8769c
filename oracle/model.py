"""CPU oracle of the hunyuan-dense decode step (test infrastructure only:
imported by tests/, never by the product).

Composes the pinned oracle pieces in the reference's order
(HunyuanDenseModel.Decode.cs:30-101, HunyuanDenseModel.cs:390-419):
embedding row (orc_dequant_row), RMSNorm (orc_rmsnorm, Ops.cs:12-90),
projections (orc_gemv: the dequantized rows times fp32 activations, in
double), decode attention with RoPE, QK norm and the bf16/fp16 append
(orc_decode_attention), SiLU(gate) * up (Ops.SiLUMulRange scalar tail,
Ops.cs:1049-1053, in double), residual adds, output norm and projection.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import oracle as O


class OracleModel:
    def __init__(self, cfg, tensors: dict, max_tokens: int, kv_dtype: int):
        self.cfg, self.t, self.kv_dtype = cfg, tensors, kv_dtype
        kd = cfg.num_kv_heads * cfg.head_dim
        self.cache = [(O.new_cache(max_tokens, cfg.num_kv_heads, cfg.head_dim, kv_dtype),
                       O.new_cache(max_tokens, cfg.num_kv_heads, cfg.head_dim, kv_dtype))
                      for _ in range(cfg.num_layers)]
        self.kd = kd

    def _vec(self, name):
        return np.frombuffer(self.t[name].data, dtype=np.float32)

    def _gemv(self, name, x, y=None):
        t = self.t[name]
        return O.gemv(t.type, t.data, t.rows, t.cols, x, y)

    def step(self, token: int, pos: int) -> np.ndarray:
        c = self.cfg
        e = self.t["token_embd.weight"]
        rb = O.row_bytes(e.type, e.cols)
        h = O.dequant(e.type, e.data[token * rb:(token + 1) * rb], 1, e.cols)[0].copy()
        for l in range(c.num_layers):
            p = f"blk.{l}."
            n1 = O.rmsnorm(h[None, :], self._vec(p + "attn_norm.weight"), c.eps)[0]
            q = self._gemv(p + "attn_q.weight", n1)
            k = self._gemv(p + "attn_k.weight", n1)
            v = self._gemv(p + "attn_v.weight", n1)
            ck, cv = self.cache[l]
            ao = O.decode_attention(q, k, v, self._vec(p + "attn_q_norm.weight"),
                                    self._vec(p + "attn_k_norm.weight"), ck, cv, self.kv_dtype,
                                    c.num_heads, c.num_kv_heads, c.head_dim, c.rope_base, c.eps, pos,
                                    rope_dim=c.rope_dim)
            h = self._gemv(p + "attn_output.weight", ao, h)
            n2 = O.rmsnorm(h[None, :], self._vec(p + "ffn_norm.weight"), c.eps)[0]
            g = self._gemv(p + "ffn_gate.weight", n2).astype(np.float64)
            u = self._gemv(p + "ffn_up.weight", n2).astype(np.float64)
            with np.errstate(over="ignore"):  # exp(-g) = inf for g < -709: silu -> -0
                act = (g / (1.0 + np.exp(-g)) * u).astype(np.float32)
            h = self._gemv(p + "ffn_down.weight", act, h)
        hn = O.rmsnorm(h[None, :], self._vec("output_norm.weight"), c.eps)[0]
        return self._gemv("output.weight" if "output.weight" in self.t else "token_embd.weight", hn)

    def forward(self, tokens, pos: int) -> np.ndarray:
        for i, tok in enumerate(tokens):
            logits = self.step(int(tok), pos + i)
        return logits


class _Layer(ctypes.Structure):
    _fields_ = ([(n, ctypes.c_void_p) for n in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")] +
                [(n, ctypes.c_int) for n in ("wq_type", "wk_type", "wv_type", "wo_type", "wg_type", "wu_type",
                                             "wd_type")] +
                [(n, ctypes.c_void_p) for n in ("attn_norm", "ffn_norm", "q_norm", "k_norm", "cache_k", "cache_v")])


class _Model(ctypes.Structure):
    _fields_ = ([(n, ctypes.c_int) for n in ("layers", "hidden", "ffn", "vocab", "heads", "kv_heads", "head_dim",
                                             "rope_dim", "kv_dtype")] +
                [("eps", ctypes.c_float), ("rope_base", ctypes.c_float), ("embd", ctypes.c_void_p),
                 ("embd_type", ctypes.c_int), ("out", ctypes.c_void_p), ("out_type", ctypes.c_int),
                 ("out_norm", ctypes.c_void_p), ("layer", ctypes.c_void_p)])


class CpuDecodePort:
    """The reference's CPU decode step (oracle/cpu_decode.c,
    HunyuanDenseModel.Decode.cs:30-101 over Q8_K activations): the CPU
    baseline bench.py times.  Weights Q4_K / Q6_K as GGUF blocks; the cache
    keeps the reference's bf16 unless kv_dtype says otherwise."""

    def __init__(self, cfg, tensors: dict, max_tokens: int, kv_dtype: int = O.BF16):
        self.cfg = cfg
        self._keep = []

        def arr(name, dtype=np.uint8):
            a = np.ascontiguousarray(np.frombuffer(bytes(tensors[name].data), dtype=dtype))
            self._keep.append(a)
            return a.ctypes.data, tensors[name].type

        layers = (_Layer * cfg.num_layers)()
        self.cache = []
        for l in range(cfg.num_layers):
            p = f"blk.{l}."
            L = layers[l]
            for f, n in (("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"), ("wo", "attn_output"),
                         ("wg", "ffn_gate"), ("wu", "ffn_up"), ("wd", "ffn_down")):
                ptr, t = arr(p + n + ".weight")
                setattr(L, f, ptr)
                setattr(L, f + "_type", t)
            for f, n in (("attn_norm", "attn_norm"), ("ffn_norm", "ffn_norm"), ("q_norm", "attn_q_norm"),
                         ("k_norm", "attn_k_norm")):
                setattr(L, f, arr(p + n + ".weight", np.float32)[0])
            ck = O.new_cache(max_tokens, cfg.num_kv_heads, cfg.head_dim, kv_dtype)
            cv = O.new_cache(max_tokens, cfg.num_kv_heads, cfg.head_dim, kv_dtype)
            self.cache.append((ck, cv))
            L.cache_k, L.cache_v = ck.ctypes.data, cv.ctypes.data
        m = _Model()
        m.layers, m.hidden, m.ffn, m.vocab = cfg.num_layers, cfg.hidden_size, cfg.ffn_size, cfg.vocab_size
        m.heads, m.kv_heads, m.head_dim, m.rope_dim = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.rope_dim
        m.kv_dtype, m.eps, m.rope_base = kv_dtype, cfg.eps, cfg.rope_base
        m.embd, m.embd_type = arr("token_embd.weight")
        m.out, m.out_type = arr("output.weight" if "output.weight" in tensors else "token_embd.weight")
        m.out_norm = arr("output_norm.weight", np.float32)[0]
        m.layer = ctypes.cast(layers, ctypes.c_void_p)
        self._layers, self._m = layers, m

    def step(self, token: int, pos: int, threads: int = 1) -> np.ndarray:
        logits = np.empty(self.cfg.vocab_size, np.float32)
        if O.lib().orc_cpu_decode_step(ctypes.byref(self._m), token, pos, logits.ctypes.data, threads) != 0:
            raise ValueError("orc_cpu_decode_step")
        return logits
