"""Device block store on the GPU (HarvestPrefix / RestorePrefix with
copy-on-write, MetalBackend.cs:224-387): restored blocks hold exactly the
K/V that was harvested, a write into a harvested block copies the block's
leading rows in every layer and leaves the harvested page intact, decode
after a restore equals decode on the original cache bit for bit, and a
copy-on-write cannot be recorded.  The page bookkeeping itself is checked
against the oracle on the CPU (test_block_store.py)."""
import numpy as np
import pytest

from hymt2sharp_amd import F16, HipBackend
from hymt2sharp_amd import _native as N
from tests.attn_cases import BASE, D, EPS, HKV, HQ, cache_rows, new_token

pytestmark = pytest.mark.gpu

PAGE = 64
LAYERS = 2


def backend(cap):
    return HipBackend(0).configure(HQ, HKV, D, D, BASE, EPS).create_cache(LAYERS, cap, F16)


def prompt(salt, n):
    return (np.arange(n, dtype=np.int32) * 31 + 1000 * salt) % 50000


def fill(be, salt, n):
    """Prefill n tokens of seeded data at position 0 in every layer."""
    for l in range(LAYERS):
        q, k, v, qnw, knw = new_token(21, salt * 10 + l, "gamma", seq=n)
        be.PrefillAttention(l, 0, q, k, v, qnw, knw)


def read_all(be, pos, n):
    return [be.ReadKv(l, pos, n) for l in range(LAYERS)]


def same(a, b):
    return all(np.array_equal(x[0], y[0]) and np.array_equal(x[1], y[1]) for x, y in zip(a, b))


def test_restore_returns_the_harvested_kv(hip_available):
    n = 3 * PAGE
    be = backend(8 * PAGE)
    try:
        fill(be, 1, n)
        ka = read_all(be, 0, n)
        be.HarvestPrefix(prompt(1, n), PAGE)
        be.SetCacheLen(0)
        fill(be, 2, n)                       # blocks 0-2 pinned: fresh pages
        kb = read_all(be, 0, n)
        assert not same(ka, kb)
        be.SetCacheLen(0)
        assert be.RestorePrefix(prompt(1, n), PAGE) == n
        be.SetCacheLen(n)
        assert same(read_all(be, 0, n), ka)
    finally:
        be.Dispose()


def test_write_inside_a_harvested_block_copies_its_rows(hip_available):
    n = 3 * PAGE
    be = backend(8 * PAGE)
    try:
        fill(be, 3, n)
        ka = read_all(be, 0, n)
        toks = prompt(3, n)
        be.HarvestPrefix(toks, PAGE)
        old = be.page_of(2)
        pos = 2 * PAGE + 2                   # decode into block 2, after 2 of its rows
        be.SetCacheLen(pos)
        q, k, v, qnw, knw = new_token(22, 0, "gamma")
        be.DecodeAttention(0, pos, q[0], k[0], v[0], qnw, knw)
        assert be.page_of(2) != old
        kb = read_all(be, 0, pos)
        for l in range(LAYERS):              # leading rows copied in every layer
            assert np.array_equal(kb[l][0], ka[l][0][:pos])
            assert np.array_equal(kb[l][1], ka[l][1][:pos])
        be.SetCacheLen(0)
        assert be.RestorePrefix(toks, PAGE) == n
        be.SetCacheLen(n)
        assert same(read_all(be, 0, n), ka)  # the harvested page is intact
    finally:
        be.Dispose()


def test_decode_after_restore_is_bit_identical(hip_available):
    n = 3 * PAGE
    be = backend(8 * PAGE)
    try:
        fill(be, 4, n)
        q, k, v, qnw, knw = new_token(23, 0, "gamma")
        ref = be.DecodeAttention(1, n, q[0], k[0], v[0], qnw, knw)
        be.HarvestPrefix(prompt(4, n), PAGE)
        be.SetCacheLen(0)
        fill(be, 5, n)
        be.SetCacheLen(0)
        assert be.RestorePrefix(prompt(4, n), PAGE) == n
        be.SetCacheLen(n)
        got = be.DecodeAttention(1, n, q[0], k[0], v[0], qnw, knw)
        assert np.array_equal(got, ref)
    finally:
        be.Dispose()


def test_copy_on_write_is_not_recorded(hip_available):
    n = 2 * PAGE
    be = backend(8 * PAGE)
    try:
        fill(be, 6, n)
        be.HarvestPrefix(prompt(6, n), PAGE)
        pos = PAGE + 7
        be.SetCacheLen(pos)
        q, k, v, qnw, knw = new_token(24, 0, "gamma")
        ptrs = []
        for a in (q, k, v, qnw, knw, np.zeros_like(q)):
            p = be.alloc(a.nbytes)
            be.upload(p, a)
            ptrs.append(p)
        be.graph_begin()
        with pytest.raises(N.InvalidOperationError):
            be.decode_dev(0, pos, *ptrs)
        with pytest.raises(N.InvalidOperationError):
            be.graph_end()
        be.decode_dev(0, pos, *ptrs)         # eagerly it copies and proceeds
        be.sync()
        for p in ptrs:
            be.free(p)
    finally:
        be.Dispose()
