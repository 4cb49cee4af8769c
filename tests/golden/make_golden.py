"""Write tests/golden/attention_golden.npz: small attention cases computed in
fp64 numpy from the definitions (tests/np_ref.py), independent of the C
oracle.  Inputs are seeded (hymt2sharp_amd.synth); K/V are stored in the
case's cache dtype before the fp64 attention, as the reference stores them.

    python tests/golden/make_golden.py
"""
import math
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from hymt2sharp_amd import synth as S  # noqa: E402
from tests import np_ref  # noqa: E402

F32, F16, BF16 = 0, 1, 2


def store(x, dtype):
    x = np.asarray(x, np.float32)
    if dtype == F32:
        return x
    if dtype == F16:
        return x.astype(np.float16).astype(np.float32)
    return S.bf16_bits_to_f32(S.f32_to_bf16_bits(x)).reshape(x.shape)


def case(name, seed, heads, kvh, D, pos, seq, dtype, norm):
    sc = 1 / math.sqrt(D)
    q = S.normal(seed, (seq, heads * D), sc)
    k = S.normal(seed + 1, (seq, kvh * D), sc)
    v = S.normal(seed + 2, (seq, kvh * D), sc)
    kc = S.normal(seed + 3, (pos, kvh * D), sc)
    vc = S.normal(seed + 4, (pos, kvh * D), sc)
    qnw = S.uniform(seed + 5, (D,), 0.9, 1.1) if norm else np.zeros(0, np.float32)
    knw = S.uniform(seed + 6, (D,), 0.9, 1.1) if norm else np.zeros(0, np.float32)
    qh = np_ref.rope(q.reshape(seq, heads, D), pos, 10000.0)
    kh = np_ref.rope(k.reshape(seq, kvh, D), pos, 10000.0)
    if norm:
        qh = np_ref.rmsnorm(qh, qnw, 1e-6)
        kh = np_ref.rmsnorm(kh, knw, 1e-6)
    K = np.concatenate([store(kc, dtype), store(kh.reshape(seq, -1), dtype)]).reshape(-1, kvh, D)
    V = np.concatenate([store(vc, dtype), store(v, dtype)]).reshape(-1, kvh, D)
    out = np_ref.attention(qh, K, V, heads, kvh, pos, sc).reshape(seq, heads * D)
    meta = np.array([heads, kvh, D, pos, seq, dtype], np.int64)
    d = {"meta": meta, "q": q, "k": k, "v": v, "kcache": kc, "vcache": vc, "qnw": qnw,
         "knw": knw, "out": out.astype(np.float32)}
    return {f"{name}__{k}": val for k, val in d.items()}


def main():
    cases = {}
    cases.update(case("decode_bf16_norm", 100, 16, 4, 128, 37, 1, BF16, True))
    cases.update(case("decode_f32_plain", 110, 16, 4, 128, 9, 1, F32, False))
    cases.update(case("decode_f16_norm", 120, 16, 4, 128, 20, 1, F16, True))
    cases.update(case("prefill_bf16_norm", 130, 16, 4, 128, 0, 5, BF16, True))
    cases.update(case("prefill_f16_chunk", 140, 16, 4, 128, 11, 4, F16, False))
    cases.update(case("gqa2_decode", 150, 4, 2, 32, 5, 1, F32, True))
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "attention_golden.npz")
    np.savez_compressed(out, **cases)
    print(out, os.path.getsize(out), "bytes")


if __name__ == "__main__":
    main()
