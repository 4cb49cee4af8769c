"""Decode GEMV on the GPU (gemv.hip through hymt_gemv) against the oracle's
y = W x over the dequantized rows in double (oracle/hymt_quant.c), for every
weight format the reference's models use.  The bound is fp32 summation error
relative to sum |w x| of the row."""
import numpy as np
import pytest

from hymt2sharp_amd import HipBackend
from hymt2sharp_amd import _native as N
from hymt2sharp_amd import synth as S
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TYPES = [N.W_F32, N.W_F16, N.W_Q8_0, N.W_Q4_K, N.W_Q6_K, N.W_Q2_0C, N.W_STQ1_0]


def run(be, wtype, rows, cols, seed, accumulate=False):
    raw = S.random_weight(seed, wtype, rows, cols)
    rng = np.random.default_rng(seed + 1)
    x = rng.standard_normal(cols).astype(np.float32)
    y0 = rng.standard_normal(rows).astype(np.float32)
    w = be.weight_upload(wtype, rows, cols, raw)
    dx, dy = be.alloc(x.nbytes), be.alloc(y0.nbytes)
    try:
        be.upload(dx, x)
        be.upload(dy, y0)
        be.gemv(w, dx, dy, accumulate)
        be.sync()
        got = be.download(np.empty(rows, np.float32), dy)
    finally:
        be.free(dx)
        be.free(dy)
        be.weight_free(w)
    ref = O.gemv(wtype, raw, rows, cols, x, y=y0 if accumulate else None)
    wd = O.dequant(wtype, raw, rows, cols).astype(np.float64)
    mag = np.abs(wd) @ np.abs(x.astype(np.float64)) + (np.abs(y0) if accumulate else 0)
    return got, ref, mag


@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("rows,cols", [(37, 2048), (11, 6144)])
def test_gemv_matches_oracle(hip_available, wtype, rows, cols):
    be = HipBackend(0)
    try:
        got, ref, mag = run(be, wtype, rows, cols, 100 + wtype + cols)
    finally:
        be.Dispose()
    assert np.all(np.abs(got - ref) <= 2e-6 * mag + 1e-6), np.max(np.abs(got - ref) / mag)


@pytest.mark.parametrize("wtype", [N.W_Q4_K, N.W_Q2_0C, N.W_Q6_K])
def test_gemv_accumulates_and_covers_many_rows(hip_available, wtype):
    # enough rows that the work spans many workgroups with a partial last one
    be = HipBackend(0)
    try:
        got, ref, mag = run(be, wtype, 3001, 2048, 300 + wtype, accumulate=True)
    finally:
        be.Dispose()
    assert np.all(np.abs(got - ref) <= 2e-6 * mag + 1e-6), np.max(np.abs(got - ref) / mag)


def test_weight_upload_checks_shape_and_size(hip_available):
    be = HipBackend(0)
    try:
        with pytest.raises(N.NotSupportedError):
            be.weight_upload(N.W_Q4_K, 4, 1024, S.random_weight(1, N.W_Q4_K, 4, 1024))
        with pytest.raises(N.ArgumentError):
            be.weight_upload(N.W_Q4_K, 4, 2048, S.random_weight(1, N.W_Q4_K, 3, 2048))
        with pytest.raises(N.NotSupportedError):
            be.weight_upload(2, 4, 2048, b"\0" * 4 * 1152)  # Q4_0: not a format of the models
        w = be.weight_upload(N.W_STQ1_0, 4, 2048, S.random_weight(1, N.W_STQ1_0, 4, 2048))
        info = be.weight_info(w)
        be.weight_free(w)
        assert (info["type"], info["rows"], info["cols"]) == (N.W_STQ1_0, 4, 2048)
    finally:
        be.Dispose()
