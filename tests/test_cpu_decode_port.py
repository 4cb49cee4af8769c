"""The restatement of the reference's CPU decode path (oracle/cpu_decode.c),
which bench.py times as the model leg's CPU baseline, pinned three ways:

* the integer Q4_K x Q8_K and Q6_K x Q8_K dots against a float64 numpy
  model of the same arithmetic -- x quantised to Q8_K as Q8K.QuantizeRow
  states it (Q8K.cs:12-137: iscale = -127 / the block's first signed
  extremum, round half to even, clamp to +-127), times the independently
  dequantised weights (the oracle's DequantizeRow restatements, pinned in
  tests/test_quant_oracle.py): equal to fp32 rounding, so a wrong nibble,
  scale or group index fails;
* the Q8_K product against the exact product within the quantisation bound
  sum_b (d_b / 2) sum_{i in b} |w_i| (d_b = the block's amax / 127);
* a 2-layer model step against the exact-product oracle step
  (oracle/model.py), within the same kind of bound scaled by the depth.
"""
import numpy as np
import pytest

from hymt2sharp_amd import _native as N
from hymt2sharp_amd import synth as S
from hymt2sharp_amd.model import ModelConfig
from oracle import oracle as O
from oracle.model import CpuDecodePort, OracleModel


def q8k_model(x):
    """(q, d) of Q8K.QuantizeRow in numpy: int8 values and the block scales."""
    xb = np.asarray(x, np.float32).reshape(-1, 256)
    q = np.zeros(xb.shape, np.float64)
    d = np.zeros(xb.shape[0], np.float64)
    for b, blk in enumerate(xb):
        amax = np.max(np.abs(blk))
        if amax == 0:
            continue
        mx = blk[np.argmax(np.abs(blk) == amax)]
        iscale = np.float32(-127.0) / mx
        d[b] = np.float32(1.0) / iscale
        q[b] = np.clip(np.rint(blk * iscale), -127, 127)
    return q, d


@pytest.mark.parametrize("wtype,rows,cols", [(N.W_Q4_K, 96, 2048), (N.W_Q6_K, 80, 2048), (N.W_Q4_K, 33, 6144)])
def test_q8k_dots_match_the_float64_model(oracle, wtype, rows, cols):
    raw = S.random_weight(300 + wtype + cols, wtype, rows, cols)
    w = O.dequant(wtype, raw, rows, cols).astype(np.float64)
    x = np.random.default_rng(cols + rows).standard_normal(cols).astype(np.float32)
    x[5] = 0.0
    x[256:512] = 0.0  # an all-zero block quantises to d = 0
    got = O.q8k_gemv(wtype, raw, rows, cols, x, threads=4)
    q, d = q8k_model(x)
    ref = w @ (q * d[:, None]).ravel()
    assert np.all(np.abs(got - ref) <= 2e-6 * (np.abs(w) @ np.abs((q * d[:, None]).ravel())) + 1e-6)
    # against the exact product: the Q8_K rounding bound
    exact = w @ x.astype(np.float64)
    amax = np.abs(x.reshape(-1, 256)).max(axis=1)
    bound = (np.abs(w).reshape(rows, -1, 256).sum(axis=2) * (amax / 127 / 2)).sum(axis=1)
    assert np.all(np.abs(got - exact) <= 1.001 * bound + 1e-5)
    # and it does quantise (the bound is not vacuous)
    assert np.max(np.abs(got - exact)) > 0
    # accumulate form
    y0 = np.random.default_rng(1).standard_normal(rows).astype(np.float32)
    acc = O.q8k_gemv(wtype, raw, rows, cols, x, y0, threads=2)
    assert np.allclose(acc, y0 + got, rtol=0, atol=1e-5 * (1 + np.abs(got).max()))


def test_model_step_tracks_the_exact_oracle(oracle):
    cfg = ModelConfig(num_layers=2, hidden_size=512, ffn_size=1024, num_heads=4, num_kv_heads=2,
                      head_dim=128, vocab_size=64, rope_base=10000.0, rope_dim=128, eps=1e-5)
    t = S.random_model(11, cfg)
    port = CpuDecodePort(cfg, t, 8, kv_dtype=O.BF16)
    ref = OracleModel(cfg, t, 8, O.BF16)
    for pos, tok in enumerate((3, 17, 5, 60)):
        a = port.step(tok, pos, threads=4)
        b = ref.step(tok, pos)
        # each projection's input is rounded to 8 bits of mantissa-equivalent
        # (Q8_K, relative error ~ 1/254 per block): a few times that over two
        # layers, against the largest logit
        assert np.max(np.abs(a - b)) <= 0.05 * np.max(np.abs(b)), (pos, np.max(np.abs(a - b)), np.max(np.abs(b)))
        assert np.argmax(a) == np.argmax(b) or np.sort(b)[-1] - np.sort(b)[-2] < 0.05 * np.max(np.abs(b))
