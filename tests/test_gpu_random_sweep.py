"""Seeded random sweep over the attention entry points' parameter space, each
case against the oracle under the bounds the targeted tests state
(tests/test_gpu_decode.py, tests/test_gpu_prefill.py): cache dtype, position,
chunk length, rotary width, QK norm on or off, and fp32 or bf16 inputs.  The
draws are fixed by the seed, so a failure names a reproducible case."""
import numpy as np
import pytest

from hymt2sharp_amd import BF16, F16, F32
from tests.attn_cases import max_rel
from tests.test_gpu_decode import run_case as decode_case
from tests.test_gpu_decode import ulp_close
from tests.test_gpu_prefill import check, run_prefill

pytestmark = pytest.mark.gpu

_rng = np.random.default_rng(20261202)
DECODE_CASES = [
    (int(_rng.choice([F16, BF16, F32])), int(_rng.integers(1, 20000)), str(_rng.choice(["gamma", "none"])),
     int(_rng.choice([128, 64, 0])), int(_rng.integers(0, 1000)))
    for _ in range(12)
]
PREFILL_CASES = [
    (int(_rng.choice([F16, BF16])), int(_rng.integers(0, 2000)), int(_rng.integers(1, 300)),
     str(_rng.choice(["gamma", "none"])), int(_rng.choice([128, 64, 0])), bool(_rng.integers(0, 2)),
     int(_rng.integers(0, 1000)))
    for _ in range(12)
]


@pytest.mark.parametrize("dtype,pos,norm,rope_dim,salt", DECODE_CASES)
def test_decode_random(oracle, hip_available, dtype, pos, norm, rope_dim, salt):
    print(f"decode dtype={dtype} pos={pos} norm={norm} rope_dim={rope_dim} salt={salt}", flush=True)
    got, ref, (kd, vd), (kr, vr) = decode_case(oracle, dtype, pos, None if norm == "none" else norm, config=12,
                                               salt=salt, rope_dim=rope_dim)
    assert max_rel(got, ref) <= 1e-3
    assert ulp_close(kd, kr, dtype) and ulp_close(vd, vr, dtype)


@pytest.mark.parametrize("dtype,pos,seq,norm,rope_dim,io_bf16,salt", PREFILL_CASES)
def test_prefill_random(oracle, hip_available, dtype, pos, seq, norm, rope_dim, io_bf16, salt):
    print(f"prefill dtype={dtype} pos={pos} seq={seq} norm={norm} rope_dim={rope_dim} io_bf16={io_bf16} "
          f"salt={salt}", flush=True)
    got, ref, model, vf, (kd, vd), (kref, vref) = run_prefill(oracle, dtype, pos, seq,
                                                              None if norm == "none" else norm, 13,
                                                              salt=salt, io_bf16=io_bf16, rope_dim=rope_dim)
    check(got, ref, vf, dtype, model)
    assert np.array_equal(vd, vref)
