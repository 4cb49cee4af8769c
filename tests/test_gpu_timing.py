"""The per-kernel timing mode (HYMT_HIP_TIMING=1, the counterpart of the
reference's HYMT_VK_TIMING, VulkanBackend.cs:55,488-540): read when a context
is created; every call then prints one stderr line naming its kernels with
their summed GPU times, the context prints its totals when destroyed, and the
results are those of an untimed context, bit for bit."""
import re

import numpy as np
import pytest

from hymt2sharp_amd import BF16, F16, HipBackend
from tests.attn_cases import BASE, D, EPS, HKV, HQ, cache_rows, new_token

pytestmark = pytest.mark.gpu

LINE = re.compile(r"^\[hymt timing\] (\w+)\((-?\d+)\): ([0-9.]+) us on the GPU, (\d+) kernels((?: \| \w+ \d+x [0-9.]+ us)+)$")


def run(dtype, pos, seq):
    kb, vb = cache_rows(2, pos)
    q, k, v, qnw, knw = new_token(2, 0, "gamma", seq=seq + 1)
    be = HipBackend(0).configure(HQ, HKV, D, D, BASE, EPS).create_cache(1, pos + seq + 1, dtype)
    try:
        be.UploadKv(0, 0, pos, kb, vb)
        pf = be.PrefillAttention(0, pos, q[:seq], k[:seq], v[:seq], qnw, knw)
        dec = be.DecodeAttention(0, pos + seq, q[seq], k[seq], v[seq], qnw, knw)
    finally:
        be.Dispose()
    return pf, dec


def parse(err):
    calls, totals = [], None
    for ln in err.splitlines():
        if not ln.startswith("[hymt timing]"):
            continue
        if ln.startswith("[hymt timing] totals over"):
            totals = ln
            continue
        m = LINE.match(ln)
        assert m, ln
        kernels = {}
        for part in m.group(5).split(" | ")[1:]:
            name, count, us, _ = part.split()
            kernels[name] = (int(count[:-1]), float(us))
        calls.append((m.group(1), int(m.group(2)), float(m.group(3)), int(m.group(4)), kernels))
    return calls, totals


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_timing_lines_and_unchanged_results(hip_available, monkeypatch, capfd, dtype):
    monkeypatch.delenv("HYMT_HIP_TIMING", raising=False)
    pf0, dec0 = run(dtype, 4096, 300)
    err0 = capfd.readouterr().err
    assert "[hymt timing]" not in err0

    monkeypatch.setenv("HYMT_HIP_TIMING", "1")
    pf1, dec1 = run(dtype, 4096, 300)
    err1 = capfd.readouterr().err
    np.testing.assert_array_equal(pf0, pf1)
    np.testing.assert_array_equal(dec0, dec1)

    calls, totals = parse(err1)
    names = [c[0] for c in calls]
    assert "attn_prefill" in names and "attn_decode" in names, err1
    pf = calls[names.index("attn_prefill")]
    assert pf[1] == 300
    assert {"prefill_kv", "prefill_flash"} <= set(pf[4]), pf
    dec = calls[names.index("attn_decode")]
    assert dec[1] == 4396
    assert dec[4]["decode_attn"][0] == 1 and dec[4]["decode_merge"][0] == 1, dec
    for _, _, span, n, kernels in calls:
        assert n == sum(cnt for cnt, _ in kernels.values())
        assert 0 < sum(us for _, us in kernels.values()) <= span * 1.01 + 1.0
    assert totals is not None and "decode_attn 1x" in totals


def test_quiet_mode_totals(hip_available, monkeypatch, capfd):
    """HYMT_HIP_TIMING=quiet prints nothing; hymt_timing_get returns the
    launches and summed time per kernel, hymt_timing_reset clears them."""
    from hymt2sharp_amd import _native as N
    monkeypatch.setenv("HYMT_HIP_TIMING", "quiet")
    kb, vb = cache_rows(2, 1000)
    q, k, v, qnw, knw = new_token(2, 0, "gamma", seq=3)
    be = HipBackend(0).configure(HQ, HKV, D, D, BASE, EPS).create_cache(1, 1003, F16)
    try:
        be.UploadKv(0, 0, 1000, kb, vb)
        for i in range(3):
            be.DecodeAttention(0, 1000 + i, q[i], k[i], v[i], qnw, knw)
        n, us = be.timing("decode_attn")
        assert n == 3 and us > 0
        assert be.timing("decode_merge")[0] == 3
        with pytest.raises(N.ArgumentError):
            be.timing("prefill_flash")
        be.timing_reset()
        with pytest.raises(N.ArgumentError):
            be.timing("decode_attn")
    finally:
        be.Dispose()
    assert "[hymt timing]" not in capfd.readouterr().err


def test_runtime_switch(hip_available, monkeypatch, capfd):
    """hymt_timing_enable: a context created without timing times nothing
    until mode 2 (quiet) or 1 (print) is set; mode 0 stops timing and keeps
    the totals."""
    monkeypatch.delenv("HYMT_HIP_TIMING", raising=False)
    from hymt2sharp_amd import _native as N
    kb, vb = cache_rows(2, 1000)
    q, k, v, qnw, knw = new_token(2, 0, "gamma", seq=4)
    be = HipBackend(0).configure(HQ, HKV, D, D, BASE, EPS).create_cache(1, 1004, F16)
    try:
        be.UploadKv(0, 0, 1000, kb, vb)
        be.DecodeAttention(0, 1000, q[0], k[0], v[0], qnw, knw)
        with pytest.raises(N.InvalidOperationError):
            be.timing("decode_attn")  # no timer yet
        be.timing_enable(2)
        be.DecodeAttention(0, 1001, q[1], k[1], v[1], qnw, knw)
        be.timing_enable(0)
        be.DecodeAttention(0, 1002, q[2], k[2], v[2], qnw, knw)
        assert be.timing("decode_attn")[0] == 1
        be.timing_enable(1)
        be.DecodeAttention(0, 1003, q[3], k[3], v[3], qnw, knw)
        assert be.timing("decode_attn")[0] == 2
        with pytest.raises(N.ArgumentError):
            be.timing_enable(3)
    finally:
        be.Dispose()
    err = capfd.readouterr().err
    assert err.count("[hymt timing] attn_decode(") == 1 and "attn_decode(1003)" in err
