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
        act = silu(Wgate x') * (Wup x'),
              x' = RMSNorm(h, ffn_norm)                     hymt_gemv IN_RMSNORM|OUT_SWIGLU
        h  += Wdown act                                     hymt_gemv ACCUMULATE
    logits = Wout RMSNorm(h, output_norm)                   hymt_gemv IN_RMSNORM
q, k and v (and gate and up) of a layer are uploaded as one matrix when
their types agree (rows concatenated), so each takes one GEMV.  Separate
gate and up matrices take a GEMV each into [gate | up], and the down GEMV
applies silu(gate) * up to its input (IN_SWIGLU).  Everything stays on the
device; only the logits come back.

A call with several tokens runs them as a prefill, in chunks of up to 2048
rows (Forward chunks a prompt by 1024, HunyuanDenseModel.cs:342-355; the
result does not depend on the chunking, and 2048-row GEMMs fill the chip
better), over bf16
dense copies of the layer weights (the Vulkan prefill's 16-bit weight
copies, VulkanBackend.cs:760-880).  hymt_model_prefill enqueues the whole
prompt natively in one call; prefill_composed issues the same sequence as
separate C ABI calls:
    X = token_embd[tokens]                                  hymt_embed_rows
    per layer l:
        XN = bf16 RMSNorm(X, attn_norm)                     hymt_rows_rmsnorm
        [Q|K|V] = XN . [Wq; Wk; Wv]^T (bf16)                hymt_gemm OUT_BF16
        AO = causal attention (RoPE, QK norm, append)       hymt_attn_prefill_ld
        X += bf16(AO) . Wo^T                                hymt_to_bf16, hymt_gemm ACCUMULATE
        GU = bf16 RMSNorm(X, ffn_norm) . [Wgate; Wup]^T     hymt_rows_rmsnorm, hymt_gemm OUT_BF16
        X += bf16(silu(gate) * up) . Wdown^T                hymt_rows_swiglu_bf16, hymt_gemm ACCUMULATE
    logits = Wout RMSNorm(X[last], output_norm)             hymt_gemv IN_RMSNORM
(hymt_model_prefill has the attention write bf16(AO) itself, with the
rounding of hymt_to_bf16, and runs the gate/up GEMM and the SwiGLU as one
launch (hymt_gemm_swiglu's kernel) wherever that gives the bits of the two
calls, so the two sequences give the same bits.)
"""
from __future__ import annotations

import ctypes
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
    PREFILL_CHUNK = 2048

    def __init__(self, be, cfg: ModelConfig, tensors: dict, max_tokens: int, kv_dtype: int = N.BF16,
                 prefill: bool = True):
        self.be, self.cfg, self.prefill_enabled = be, cfg, prefill
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

        def dense(ws):
            if prefill:
                for w in ws:
                    be.weight_dense(w)
            return ws

        self.layers = []
        for l in range(c.num_layers):
            p = f"blk.{l}."
            self.layers.append({
                "attn_norm": vec(p + "attn_norm.weight"), "ffn_norm": vec(p + "ffn_norm.weight"),
                "q_norm": vec(p + "attn_q_norm.weight"), "k_norm": vec(p + "attn_k_norm.weight"),
                "qkv": dense(mat(p + "attn_q.weight", p + "attn_k.weight", p + "attn_v.weight")),
                "o": dense(mat(p + "attn_output.weight"))[0],
                "gate_up": dense(mat(p + "ffn_gate.weight", p + "ffn_up.weight")),
                "down": dense(mat(p + "ffn_down.weight"))[0],
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
        self._pf = None  # prefill activations, allocated on the first prefill
        # the decode step runs natively: one hymt_model_decode per token
        lib, h = be._lib, ctypes.c_void_p()
        N.check(lib.hymt_model_create(be._h, c.num_layers, c.hidden_size, c.ffn_size, c.vocab_size,
                                      c.eps, ctypes.byref(h)))
        self._native = h.value
        for l, L in enumerate(self.layers):
            qkv, gu = L["qkv"] + [None, None], L["gate_up"] + [None]
            N.check(lib.hymt_model_set_layer(self._native, l, qkv[0], qkv[1], qkv[2], L["o"], gu[0],
                                             gu[1], L["down"], L["attn_norm"], L["ffn_norm"],
                                             L["q_norm"], L["k_norm"]))
        N.check(lib.hymt_model_set_io(self._native, self.embd,
                                      None if self.out is self.embd else self.out, self.out_norm))
        # prompts of an fp32 cache run as decode steps (the prefill kernels
        # read 16-bit pages), as do prompts without dense weight copies
        self.prefill_enabled = prefill and kv_dtype != N.F32

    def _buf(self, n):
        p = self.be.alloc(4 * n)
        self._bufs.append(p)
        return p

    def step(self, token: int, pos: int):
        """Enqueue one decode step; the logits land in self.logits
        (hymt_model_decode runs the sequence of step_composed in C++)."""
        N.check(self.be._lib.hymt_model_decode(self._native, token, pos, self.logits))

    def step_composed(self, token: int, pos: int):
        """The same decode step as separate C ABI calls (the sequence a host
        without hymt_model_decode would issue)."""
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
                be.gemv(gu[0], self.h, self.gu, rmsnorm=L["ffn_norm"], eps=c.eps, swiglu_out=True)
                be.gemv(L["down"], self.gu, self.h, accumulate=True)
            else:
                for w, off in zip(gu, (0, c.ffn_size)):
                    be.gemv(w, self.h, self.gu + 4 * off, rmsnorm=L["ffn_norm"], eps=c.eps)
                be.gemv(L["down"], self.gu, self.h, accumulate=True, swiglu=True)
        be.gemv(self.out, self.h, self.logits, rmsnorm=self.out_norm, eps=c.eps)

    def prefill(self, tokens, pos: int, gate_up_f32: bool = False):
        """Enqueue the prompt `tokens` at positions [pos, pos + len) with one
        hymt_model_prefill call (chunks of 2048 rows, or decode steps without
        dense copies or with an fp32 cache); the last row's logits land in
        self.logits.  gate_up_f32 keeps the gate/up GEMM output in fp32, as
        the reference's prefill does."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        flags = N.PREFILL_GATE_UP_F32 if gate_up_f32 else 0
        N.check(self.be._lib.hymt_model_prefill(self._native, t.ctypes.data_as(ctypes.c_void_p), t.size, pos,
                                                self.logits, flags))

    def _prefill_bufs(self):
        if self._pf is None:
            c, C = self.cfg, self.PREFILL_CHUNK
            H, F, qd, kd = c.hidden_size, c.ffn_size, self.qd, self.kd
            self._pf = {"x": self._buf(C * H), "xn": self._buf(C * H // 2),
                        "qkv": self._buf(C * (qd + 2 * kd) // 2),
                        "q": self._buf(C * qd // 2), "k": self._buf(C * kd // 2),
                        "v": self._buf(C * kd // 2), "ao": self._buf(C * qd),
                        "ao16": self._buf(C * qd // 2), "gu": self._buf(C * 2 * F),
                        "act": self._buf(C * F // 2)}
        return self._pf

    def prefill_composed(self, tokens, pos: int):
        """The sequence of hymt_model_prefill for one chunk (len(tokens) <=
        PREFILL_CHUNK) at positions [pos, pos + len), as separate C ABI calls
        (a model with fused q/k/v and gate/up matrices); the last row's logits
        land in self.logits."""
        be, c, B = self.be, self.cfg, self._prefill_bufs()
        m, H, F, qd, kd = len(tokens), c.hidden_size, c.ffn_size, self.qd, self.kd
        assert 0 < m <= self.PREFILL_CHUNK
        be.embed_rows(self.embd, tokens, B["x"])
        for l, L in enumerate(self.layers):
            be.rows_rmsnorm(B["x"], m, H, L["attn_norm"], c.eps, B["xn"])
            qkv = L["qkv"]
            if len(qkv) == 1:
                # one GEMM into [m][q|k|v]; the attention reads the column ranges
                ld = qd + 2 * kd
                be.gemm(qkv[0], B["xn"], m, B["qkv"], out_bf16=True)
                be.prefill_dev_ld(l, pos, m, B["qkv"], ld, B["qkv"] + 2 * qd, B["qkv"] + 2 * (qd + kd),
                                  ld, N.BF16, L["q_norm"], L["k_norm"], B["ao"])
            else:
                for w, y in zip(qkv, (B["q"], B["k"], B["v"])):
                    be.gemm(w, B["xn"], m, y, out_bf16=True)
                be.prefill_dev(l, pos, m, B["q"], B["k"], B["v"], N.BF16, L["q_norm"], L["k_norm"],
                               B["ao"])
            be.to_bf16(B["ao"], m * qd, B["ao16"])
            be.gemm(L["o"], B["ao16"], m, B["x"], accumulate=True)
            be.rows_rmsnorm(B["x"], m, H, L["ffn_norm"], c.eps, B["xn"])
            be.gemm(L["gate_up"][0], B["xn"], m, B["gu"], out_bf16=True)
            be.rows_swiglu_bf16(B["gu"], m, F, B["act"])
            be.gemm(L["down"], B["act"], m, B["x"], accumulate=True)
        be.gemv(self.out, B["x"] + 4 * (m - 1) * H, self.logits, rmsnorm=self.out_norm, eps=c.eps)

    def forward(self, tokens, pos: int) -> np.ndarray:
        """ForwardStep (IComputeBackend.cs:40-47): the tokens at positions
        pos, pos+1, ...; returns the last token's logits.  One token is a
        decode step; several run as prefill chunks when the dense copies were
        made (LoadModel(prefill=True)), else as decode steps one by one."""
        tokens = [int(t) for t in tokens]
        if len(tokens) > 1:
            self.prefill(tokens, pos)
        else:
            self.step(tokens[0], pos)
        out = np.empty(self.cfg.vocab_size, np.float32)
        self.be.download(out, self.logits)
        return out

    def free(self):
        if getattr(self, "_native", None):
            N.check(self.be._lib.hymt_model_destroy(self._native))
            self._native = None
        for w in self._weights:
            self.be.weight_free(w)
        for p in self._bufs:
            self.be.free(p)
        self._weights, self._bufs = [], []
