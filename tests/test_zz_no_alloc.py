"""hymt_attn_decode_noalloc through the C ABI: the decode entry point for
callers that cannot allocate device memory (its split partials live in a
static device array of the library).  It must give the same bits as
hymt_attn_decode on the same inputs, for two calls in a row, the second over
a smaller context (the array keeps the first call's contents), refuse a
position its RoPE table does not cover instead of growing the table, run
inside a recording, and refuse a second live context on the same GPU."""
import ctypes

import numpy as np
import pytest

from hymt2sharp_amd import F16, HipBackend
from hymt2sharp_amd import _native as N
from tests.attn_cases import BASE, D, EPS, HKV, HQ, cache_rows, new_token

pytestmark = pytest.mark.gpu


def _dev(be, a):
    p = be.alloc(max(a.nbytes, 16))
    be.upload(p, a)
    return p


def test_noalloc_decode_matches_decode(hip_available):
    L = N.lib()
    big, small = 9000, 700  # 141 pages (two per split), then 11 (one per split)
    be = HipBackend(0).configure(HQ, HKV, D, D, BASE, EPS).create_cache(2, big + 1, F16)
    try:
        kb, vb = cache_rows(21, big)
        be.UploadKv(0, 0, big, kb, vb)
        be.UploadKv(1, 0, big, kb, vb)
        q, k, v, qnw, knw = new_token(21, 0, "gamma")
        dq, dk, dv, dqn, dkn = (_dev(be, a) for a in (q, k, v, qnw, knw))
        o_ref, o_na = be.alloc(q.nbytes), be.alloc(q.nbytes)
        for pos in (big, small):  # the second call over a smaller context
            print(f"noalloc decode pos={pos}", flush=True)
            be.decode_dev(0, pos, dq, dk, dv, dqn, dkn, o_ref)
            N.check(L.hymt_attn_decode_noalloc(be.handle, 1, pos, dq, dk, dv, dqn, dkn, o_na))
            be.sync()
            ref = be.download(np.empty(HQ * D, np.float32), o_ref)
            got = be.download(np.empty(HQ * D, np.float32), o_na)
            assert np.array_equal(got, ref), pos
            k0, v0 = be.ReadKv(0, pos, 1)
            k1, v1 = be.ReadKv(1, pos, 1)
            assert np.array_equal(k0, k1) and np.array_equal(v0, v1), pos
        # recorded and replayed: the static array needs no growth
        be.graph_begin()
        N.check(L.hymt_attn_decode_noalloc(be.handle, 1, small, dq, dk, dv, dqn, dkn, o_na))
        g = be.graph_end()
        be.upload(o_na, np.zeros_like(q))
        be.graph_launch(g)
        be.sync()
        assert np.array_equal(be.download(np.empty(HQ * D, np.float32), o_na), ref)
        be.graph_destroy(g)
        for p in (dq, dk, dv, dqn, dkn, o_ref, o_na):
            be.free(p)
    finally:
        be.Dispose()


def test_noalloc_decode_refusals(hip_available):
    """The first call of a fresh context runs at its last position (the RoPE
    table covers the capacity from hymt_kv_create); a position past the
    capacity, a missing prefix and misaligned pointers are refused before
    anything is enqueued."""
    L = N.lib()
    be = HipBackend(0).configure(HQ, HKV, D, D, BASE, EPS).create_cache(1, 5000, F16)
    try:
        q, k, v, qnw, knw = new_token(22, 0, "gamma")
        dq, dk, dv = (_dev(be, a) for a in (q, k, v))
        dout = be.alloc(q.nbytes)
        assert L.hymt_attn_decode_noalloc(be.handle, 0, 100, dq, dk, dv, None, None, dout) == N.HYMT_E_STATE
        cap = be.cache_info()["max_tokens"]
        kb, vb = cache_rows(22, cap - 1)  # known, finite rows for the whole prefix
        be.UploadKv(0, 0, cap - 1, kb, vb)
        assert L.hymt_attn_decode_noalloc(be.handle, 0, cap, dq, dk, dv, None, None, dout) == N.HYMT_E_CAPACITY
        N.check(L.hymt_attn_decode_noalloc(be.handle, 0, cap - 1, dq, dk, dv, None, None, dout))
        assert L.hymt_attn_decode_noalloc(be.handle, 0, 100, dq + 4, dk, dv, None, None, dout) == N.HYMT_E_ARG
        be.sync()
        got = be.download(np.empty(HQ * D, np.float32), dout)
        be.decode_dev(0, cap - 1, dq, dk, dv, None, None, dout)
        be.sync()
        assert np.all(np.isfinite(got))
        assert np.array_equal(be.download(np.empty(HQ * D, np.float32), dout), got)
        for p in (dq, dk, dv, dout):
            be.free(p)
    finally:
        be.Dispose()


def test_noalloc_decode_one_context_per_gpu(hip_available):
    """The static array belongs to the first context that calls the entry
    point on a GPU: a second live context on that GPU gets HYMT_E_STATE (its
    partials would otherwise overwrite the owner's), and gets the array once
    the owner is destroyed."""
    L = N.lib()
    pos = 1000
    kb, vb = cache_rows(23, pos)
    q, k, v, qnw, knw = new_token(23, 0, "gamma")
    a = HipBackend(0).configure(HQ, HKV, D, D, BASE, EPS).create_cache(1, pos + 1, F16)
    b = HipBackend(0).configure(HQ, HKV, D, D, BASE, EPS).create_cache(1, pos + 1, F16)
    try:
        bufs = {}
        for name, be in (("a", a), ("b", b)):
            be.UploadKv(0, 0, pos, kb, vb)
            bufs[name] = [_dev(be, x) for x in (q, k, v, qnw, knw)] + [be.alloc(q.nbytes)]
        N.check(L.hymt_attn_decode_noalloc(a.handle, 0, pos, *bufs["a"]))
        assert L.hymt_attn_decode_noalloc(b.handle, 0, pos, *bufs["b"]) == N.HYMT_E_STATE
        b.decode_dev(0, pos, *bufs["b"])  # the allocating entry point is not affected
        a.sync()
        b.sync()
        ref = b.download(np.empty(HQ * D, np.float32), bufs["b"][-1])
        assert np.array_equal(a.download(np.empty(HQ * D, np.float32), bufs["a"][-1]), ref)
        for p in bufs["a"]:
            a.free(p)
        a.Dispose()
        N.check(L.hymt_attn_decode_noalloc(b.handle, 0, pos, *bufs["b"]))
        b.sync()
        assert np.array_equal(b.download(np.empty(HQ * D, np.float32), bufs["b"][-1]), ref)
        for p in bufs["b"]:
            b.free(p)
    finally:
        a.Dispose()
        b.Dispose()
