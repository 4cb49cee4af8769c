"""The oracle's decode step (oracle/model.py) against an independent float64
numpy forward of the same tiny F32 model, written from the reference's
decode block (HunyuanDenseModel.Decode.cs:30-101): RMSNorm, q/k/v, NeoX RoPE
then per-head Q/K RMSNorm, bf16 cache append, softmax over positions 0..pos,
output projection and residual, RMSNorm, SiLU(gate) * up, down projection
and residual, output norm and the (tied or separate) output projection.
A dropped residual, a swapped norm weight, RoPE applied after the QK norm or
a missing cache row each move the logits far beyond the bound."""
import numpy as np
import pytest

from hymt2sharp_amd import _native as N
from hymt2sharp_amd import synth as S
from hymt2sharp_amd.model import ModelConfig
from oracle import oracle as O
from oracle.model import OracleModel

CFG = ModelConfig(num_layers=2, hidden_size=256, ffn_size=512, num_heads=4, num_kv_heads=2,
                  head_dim=64, vocab_size=48, rope_base=10000.0, rope_dim=64, eps=1e-5)


def _bf16(x):
    b = (np.asarray(x, np.float32).view(np.uint32).astype(np.uint64) + 0x7FFF +
         ((np.asarray(x, np.float32).view(np.uint32) >> 16) & 1)) >> 16
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


class Numpy64:
    def __init__(self, cfg, t):
        self.c, self.t = cfg, t
        self.W = {k: (np.frombuffer(v.data, np.float32).reshape(v.rows, v.cols).astype(np.float64)
                      if v.rows > 1 else np.frombuffer(v.data, np.float32).astype(np.float64))
                  for k, v in t.items()}
        self.K = [[] for _ in range(cfg.num_layers)]
        self.V = [[] for _ in range(cfg.num_layers)]

    def rms(self, x, w):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.c.eps) * w

    def rope(self, x, pos):  # x [heads][dim], NeoX halves
        half = self.c.rope_dim // 2
        i = np.arange(half)
        th = pos * self.c.rope_base ** (-2.0 * i / self.c.rope_dim)
        a, b = x[:, :half].copy(), x[:, half:self.c.rope_dim].copy()
        out = x.copy()
        out[:, :half] = a * np.cos(th) - b * np.sin(th)
        out[:, half:self.c.rope_dim] = b * np.cos(th) + a * np.sin(th)
        return out

    def step(self, tok, pos):
        c, W = self.c, self.W
        d, H, KH = c.head_dim, c.num_heads, c.num_kv_heads
        h = W["token_embd.weight"][tok].copy()
        for l in range(c.num_layers):
            p = f"blk.{l}."
            n1 = self.rms(h, W[p + "attn_norm.weight"])
            q = (W[p + "attn_q.weight"] @ n1).reshape(H, d)
            k = (W[p + "attn_k.weight"] @ n1).reshape(KH, d)
            v = (W[p + "attn_v.weight"] @ n1).reshape(KH, d)
            q = self.rms(self.rope(q, pos), W[p + "attn_q_norm.weight"])
            k = self.rms(self.rope(k, pos), W[p + "attn_k_norm.weight"])
            self.K[l].append(_bf16(k))
            self.V[l].append(_bf16(v))
            Ks, Vs = np.stack(self.K[l]), np.stack(self.V[l])  # [t][KH][d]
            ao = np.empty((H, d))
            for hh in range(H):
                g = hh // (H // KH)
                s = Ks[:, g, :] @ q[hh] / np.sqrt(d)
                e = np.exp(s - s.max())
                ao[hh] = (e / e.sum()) @ Vs[:, g, :]
            h = h + W[p + "attn_output.weight"] @ ao.reshape(-1)
            n2 = self.rms(h, W[p + "ffn_norm.weight"])
            g = W[p + "ffn_gate.weight"] @ n2
            u = W[p + "ffn_up.weight"] @ n2
            h = h + W[p + "ffn_down.weight"] @ (g / (1 + np.exp(-g)) * u)
        hn = self.rms(h, W["output_norm.weight"])
        return W["output.weight" if "output.weight" in W else "token_embd.weight"] @ hn


@pytest.mark.parametrize("tied", [False, True])
def test_oracle_decode_step_matches_numpy(oracle, tied):
    t = S.random_model(7 + tied, CFG, {"attn": N.W_F32, "ffn": N.W_F32, "embd": N.W_F32,
                                       "out": N.W_F32}, tied=tied)
    om = OracleModel(CFG, t, 16, N.BF16)
    ref = Numpy64(CFG, t)
    for pos, tok in enumerate([3, 17, 0, 41, 5]):
        got = om.step(tok, pos)
        want = ref.step(tok, pos)
        # measured ~1e-7; a bf16 cache row rounded from fp32 rather than float64
        # inputs may land one ulp apart, which the bound leaves room for
        assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want)), pos
    # a planted mistake (the second residual dropped) is caught by the bound
    om2 = OracleModel(CFG, t, 16, N.BF16)
    bad = Numpy64(CFG, t)
    orig = bad.step

    def no_ffn_residual(tok, pos):
        save = {k: v.copy() for k, v in bad.W.items() if k.endswith("ffn_down.weight")}
        for k in save:
            bad.W[k][:] = 0
        try:
            return orig(tok, pos)
        finally:
            bad.W.update(save)
    bad.step = no_ffn_residual
    worst = 0.0
    for pos, tok in enumerate([3, 17, 0, 41, 5]):
        a, b = om2.step(tok, pos), bad.step(tok, pos)
        worst = max(worst, np.max(np.abs(a - b)) / np.max(np.abs(b)))
    assert worst > 2e-2


def test_forward_returns_last_step(oracle):
    t = S.random_model(11, CFG, {"attn": N.W_Q8_0, "ffn": N.W_Q4_K, "embd": N.W_Q6_K,
                                 "out": N.W_Q6_K})
    a, b = OracleModel(CFG, t, 16, N.F16), OracleModel(CFG, t, 16, N.F16)
    toks = [1, 2, 3, 4]
    la = a.forward(toks, 0)
    for i, tok in enumerate(toks):
        lb = b.step(tok, i)
    assert np.array_equal(la, lb)
