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
