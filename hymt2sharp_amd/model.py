"""hunyuan-dense decode step on the device: the host side of
IComputeBackend.LoadModel / ForwardStep (IComputeBackend.cs:25-47) for the
HIP backend, composed from the C ABI's building blocks the way
HunyuanDenseModel.Forward / DecodeBlock compose the CPU ops
(HunyuanDenseModel.cs:364-430, HunyuanDenseModel.Decode.cs:30-101).

One decode step of a token at position `pos`:
    h = token_embd[token]                                   hymt_embed
    per layer l:
        qkv = [Wq; Wk; Wv] RMSNorm(h, attn_norm)            hymt_gemv IN_RMSNORM
        ao  = attention(q, k, v) (RoPE, QK norm, append)    hymt_attn_decode
        h  += Wo ao                                         hymt_gemv ACCUMULATE
        gu  = [Wgate; Wup] RMSNorm(h, ffn_norm)             hymt_gemv IN_RMSNORM
        h  += Wdown (silu(gate) * up)                       hymt_gemv IN_SWIGLU|ACCUMULATE
    logits = Wout RMSNorm(h, output_norm)                   hymt_gemv IN_RMSNORM
q, k and v (and gate and up) of a layer are uploaded as one matrix when
their types agree (rows concatenated), so each takes one GEMV.  Everything
stays on the device; only the logits come back.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _native as N


@dataclass
class ModelConfig:
    """ModelConfig (ModelConfig.cs:5-51), the fields the decode step uses."""
    num_layers: int = 32
    hidden_size: int = 2048
    ffn_size: int = 6144
    num_heads: int = 16
    num_kv_heads: int = 4
    head_dim: int = 128
    vocab_size: int = 120818
    rope_base: float = 10000.0
    rope_dim: int = 128
    eps: float = 1e-5


@dataclass
class Tensor:
    """A GGUF tensor as GgufFile hands it over: type, rows (ne1), cols (ne0)
    and the raw row-major block bytes (F32 vectors: rows = 1)."""
    type: int
    rows: int
    cols: int
    data: bytes


class DeviceModel:
    def __init__(self, be, cfg: ModelConfig, tensors: dict, max_tokens: int, kv_dtype: int = N.BF16):
        self.be, self.cfg = be, cfg
        c = cfg
        self._weights, self._bufs = [], []
        be.configure(c.num_heads, c.num_kv_heads, c.head_dim, c.rope_dim, c.rope_base, c.eps)
        be.create_cache(c.num_layers, max_tokens, kv_dtype)

        def vec(name):
            t = tensors[name]
            a = np.frombuffer(t.data, dtype=np.float32)
            assert t.type == N.W_F32 and a.size == t.rows * t.cols, name
            p = be.alloc(a.nbytes)
            be.upload(p, a)
            self._bufs.append(p)
            return p

        def mat(*names):
            ts = [tensors[n] for n in names]
            if all(t.type == ts[0].type and t.cols == ts[0].cols for t in ts):
                w = be.weight_upload(ts[0].type, sum(t.rows for t in ts), ts[0].cols,
                                     b"".join(t.data for t in ts))
                self._weights.append(w)
                return [w]
            out = [be.weight_upload(t.type, t.rows, t.cols, t.data) for t in ts]
            self._weights.extend(out)
            return out

        self.layers = []
        for l in range(c.num_layers):
            p = f"blk.{l}."
            self.layers.append({
                "attn_norm": vec(p + "attn_norm.weight"), "ffn_norm": vec(p + "ffn_norm.weight"),
                "q_norm": vec(p + "attn_q_norm.weight"), "k_norm": vec(p + "attn_k_norm.weight"),
                "qkv": mat(p + "attn_q.weight", p + "attn_k.weight", p + "attn_v.weight"),
                "o": mat(p + "attn_output.weight")[0],
                "gate_up": mat(p + "ffn_gate.weight", p + "ffn_up.weight"),
                "down": mat(p + "ffn_down.weight")[0],
            })
        self.embd = mat("token_embd.weight")[0]
        # the output projection falls back to the tied embedding (HunyuanDenseModel.cs:419)
        self.out = mat("output.weight")[0] if "output.weight" in tensors else self.embd
        self.out_norm = vec("output_norm.weight")
        qd, kd = c.num_heads * c.head_dim, c.num_kv_heads * c.head_dim
        self.qd, self.kd = qd, kd
        self.h = self._buf(c.hidden_size)
        self.qkv = self._buf(qd + 2 * kd)
        self.ao = self._buf(qd)
        self.gu = self._buf(2 * c.ffn_size)
        self.logits = self._buf(c.vocab_size)

    def _buf(self, n):
        p = self.be.alloc(4 * n)
        self._bufs.append(p)
        return p

    def step(self, token: int, pos: int):
        """Enqueue one decode step; the logits land in self.logits."""
        be, c = self.be, self.cfg
        be.embed(self.embd, token, self.h)
        for l, L in enumerate(self.layers):
            qkv = L["qkv"]
            if len(qkv) == 1:
                be.gemv(qkv[0], self.h, self.qkv, rmsnorm=L["attn_norm"], eps=c.eps)
            else:
                for w, off in zip(qkv, (0, self.qd, self.qd + self.kd)):
                    be.gemv(w, self.h, self.qkv + 4 * off, rmsnorm=L["attn_norm"], eps=c.eps)
            be.decode_dev(l, pos, self.qkv, self.qkv + 4 * self.qd, self.qkv + 4 * (self.qd + self.kd),
                          L["q_norm"], L["k_norm"], self.ao)
            be.gemv(L["o"], self.ao, self.h, accumulate=True)
            gu = L["gate_up"]
            if len(gu) == 1:
                be.gemv(gu[0], self.h, self.gu, rmsnorm=L["ffn_norm"], eps=c.eps)
            else:
                for w, off in zip(gu, (0, c.ffn_size)):
                    be.gemv(w, self.h, self.gu + 4 * off, rmsnorm=L["ffn_norm"], eps=c.eps)
            be.gemv(L["down"], self.gu, self.h, accumulate=True, swiglu=True)
        be.gemv(self.out, self.h, self.logits, rmsnorm=self.out_norm, eps=c.eps)

    def forward(self, tokens, pos: int) -> np.ndarray:
        """ForwardStep (IComputeBackend.cs:40-47): the tokens at positions
        pos, pos+1, ..., one decode step each; returns the last token's logits.
        (A prompt runs token by token here: the prefill GEMMs are not built.)"""
        for i, t in enumerate(tokens):
            self.step(int(t), pos + i)
        out = np.empty(self.cfg.vocab_size, np.float32)
        self.be.download(out, self.logits)
        return out

    def free(self):
        for w in self._weights:
            self.be.weight_free(w)
        for p in self._bufs:
            self.be.free(p)
        self._weights, self._bufs = [], []
