"""The C ABI from a plain C host (tests/c/abi_host.c, built by build()):
the calls a non-Python binding of IComputeBackend (IComputeBackend.cs:14-88)
makes for one layer's attention -- UploadKv, a prefill chunk, a decode step
-- through include/hymt_hip.h alone.

CPU: the program links and loads the library, the device probe answers, and
a NULL context is refused with a message (exit 3 with no device).  GPU: its
results are bit-identical to the same calls made through the Python mirror
(hymt2sharp_amd/backend.py) and within the stated bounds of the oracle
(prefill: 4 u max|V| with u = 2^-11 for an fp16 cache, as
tests/test_gpu_prefill.py; decode: 1e-3 relative, as tests/test_gpu_decode.py).
"""
import os
import subprocess

import numpy as np
import pytest

from hymt2sharp_amd import F16, HipBackend
from tests.attn_cases import BASE, D, EPS, HKV, HQ, cache_rows, max_rel, new_token, oracle_cache

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "tests", "c", "abi_host")
POS, SEQ = 200, 37


def inputs():
    kb, vb = cache_rows(21, POS, salt=1)
    pq, pk, pv, qnw, knw = new_token(21, 1, "gamma", seq=SEQ)
    dq, dk, dv, _, _ = new_token(21, 2, None)
    return kb, vb, pq, pk, pv, dq.ravel(), dk.ravel(), dv.ravel(), qnw, knw


def write_in(path, kv_dtype):
    kb, vb, pq, pk, pv, dq, dk, dv, qnw, knw = inputs()
    with open(path, "wb") as f:
        f.write(np.array([HQ, HKV, D, POS, SEQ, kv_dtype], np.int32).tobytes())
        for a, t in ((qnw, np.float32), (knw, np.float32), (kb, np.uint16), (vb, np.uint16),
                     (pq, np.float32), (pk, np.float32), (pv, np.float32),
                     (dq, np.float32), (dk, np.float32), (dv, np.float32)):
            f.write(np.ascontiguousarray(a, t).tobytes())


def run_host(tmp_path, kv_dtype):
    if not os.path.exists(HOST):
        pytest.fail(f"{HOST} is not built; run __graft_entry__.build()")
    fin, fout = tmp_path / "in.bin", tmp_path / "out.bin"
    write_in(fin, kv_dtype)
    r = subprocess.run([HOST, str(fin), str(fout)], capture_output=True, text=True, timeout=120)
    return r, fout


def test_c_host_loads_probes_and_refuses(tmp_path):
    """Runs in every suite: without a GPU the host stops after the probe
    (exit 3); with one it runs to the end (exit 0).  Exit 4 would mean the
    NULL-context call was not refused with a message."""
    r, _ = run_host(tmp_path, F16)
    assert r.returncode in (0, 3), (r.returncode, r.stdout, r.stderr)
    if r.returncode == 3:
        assert "no HIP device" in r.stdout


@pytest.mark.gpu
def test_c_host_matches_python_mirror_and_oracle(tmp_path, hip_available, oracle):
    r, fout = run_host(tmp_path, F16)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    got = np.fromfile(fout, np.float32)
    assert got.size == SEQ * HQ * D + HQ * D
    c_pf, c_dec = got[:SEQ * HQ * D].reshape(SEQ, HQ * D), got[SEQ * HQ * D:]

    kb, vb, pq, pk, pv, dq, dk, dv, qnw, knw = inputs()
    be = HipBackend(0).configure(HQ, HKV, D, D, BASE, EPS).create_cache(1, POS + SEQ + 1, F16)
    try:
        be.UploadKv(0, 0, POS, kb, vb)
        py_pf = be.PrefillAttention(0, POS, pq, pk, pv, qnw, knw)
        py_dec = be.DecodeAttention(0, POS + SEQ, dq, dk, dv, qnw, knw)
        be.sync()
    finally:
        be.Dispose()
    assert np.array_equal(c_pf, py_pf)
    assert np.array_equal(c_dec, py_dec)

    cap = POS + SEQ + 1
    ck, cv = oracle_cache(kb, vb, cap, F16)
    ref_pf = oracle.prefill_attention(pq, pk, pv, qnw, knw, ck, cv, F16, HQ, HKV, D, BASE, EPS, POS,
                                      threads=8)
    ref_dec = oracle.decode_attention(dq, dk, dv, qnw, knw, ck, cv, F16, HQ, HKV, D, BASE, EPS, POS + SEQ)
    vmax = float(np.max(np.abs(oracle.from_storage(cv, F16)[:POS + SEQ])))
    assert np.max(np.abs(c_pf - ref_pf)) <= 4 * 2.0 ** -11 * vmax
    assert max_rel(c_dec, ref_dec) <= 1e-3
