"""Device block store (HarvestPrefix / RestorePrefix / copy-on-write) and the
page allocator under it, on the CPU: the C ABI on a host-only context
(HYMT_DEVICE_NONE) against oracle/block_store.py, the restatement of the
Metal backend's algorithm (MetalBackend.cs:224-387).

The oracle's chain hash is pinned by the published FNV-1a 64-bit test
vectors (for token values below 256 KvBlockStore.ChainHash is byte-wise
FNV-1a); the directed cases follow the reference's KvBlockStoreTests
(KvBlockStoreTests.cs: token mismatch is a miss, the key depends on the
prefix, least recently used entries go first)."""
import random

import numpy as np
import pytest

from hymt2sharp_amd import _native as N
from hymt2sharp_amd.backend import HipBackend, NotSupportedError
from oracle import block_store as B

PAGE = 64


def host(max_tokens, layers=2):
    return HipBackend(N.DEVICE_NONE).configure(16, 4, 128, 128, 1e4, 1e-6).create_cache(
        layers, max_tokens, N.BF16)


def table(be, n):
    return [be.page_of(b) for b in range(n)]


def blocks(*vals):
    """Token list of one 64-token block per value (block i = value i repeated,
    with its position mixed in so blocks differ inside)."""
    return np.concatenate([np.full(PAGE, v, np.int32) + np.arange(PAGE, dtype=np.int32) * 7
                           for v in vals])


# ---- the oracle's hash --------------------------------------------------------

def test_chain_hash_fnv1a_test_vectors():
    # FNV-1a 64: "" -> cbf29ce484222325, "a" -> af63dc4c8601ec8c,
    # "foobar" -> 85944171f73967e8
    assert B.chain_hash(B.SEED, []) == 0xcbf29ce484222325
    assert B.chain_hash(B.SEED, [ord("a")]) == 0xaf63dc4c8601ec8c
    assert B.chain_hash(B.SEED, [ord(ch) for ch in "foobar"]) == 0x85944171f73967e8
    # chaining = hashing the concatenation
    assert B.chain_hash(B.chain_hash(B.SEED, [ord("f"), ord("o")]), [ord(ch) for ch in "obar"]) == \
        0x85944171f73967e8


def test_chain_hash_is_order_dependent():
    # KvBlockStoreTests.ChainHash_IsOrderDependent
    a = B.chain_hash(B.chain_hash(B.SEED, [1, 2]), [3, 4])
    b = B.chain_hash(B.chain_hash(B.SEED, [9, 9]), [3, 4])
    assert a != b


# ---- directed cases through the C ABI -------------------------------------------

def test_harvest_then_restore_maps_the_same_pages():
    be = host(64 * 8)
    try:
        toks = blocks(1, 2, 3)
        be.MapRange(0, 3 * PAGE + 10)
        before = table(be, 4)
        be.HarvestPrefix(toks, PAGE)
        assert be.store_info()["entries"] == 3
        be.SetCacheLen(0)                      # pinned pages stay with the store
        assert table(be, 4) == [-1] * 4
        assert be.RestorePrefix(toks, PAGE) == 3 * PAGE
        assert table(be, 3) == before[:3]      # zero-copy: the same pages
    finally:
        be.Dispose()


def test_token_mismatch_is_a_miss():
    # KvBlockStoreTests.Find_TokenMismatch_IsMiss
    be = host(64 * 8)
    try:
        toks = blocks(1, 2)
        be.MapRange(0, 2 * PAGE)
        be.HarvestPrefix(toks, PAGE)
        other = toks.copy()
        other[PAGE + 5] += 1                   # second block differs
        assert be.RestorePrefix(other, PAGE) == PAGE
        other[3] += 1                          # first block differs too
        assert be.RestorePrefix(other, PAGE) == 0
    finally:
        be.Dispose()


def test_key_depends_on_the_prefix():
    be = host(64 * 8)
    try:
        be.MapRange(0, 2 * PAGE)
        be.HarvestPrefix(blocks(1, 2), PAGE)
        # same second block after another first block: no hit at all
        assert be.RestorePrefix(blocks(9, 2), PAGE) == 0
    finally:
        be.Dispose()


def test_write_into_a_harvested_block_takes_a_fresh_page():
    be = host(64 * 8)
    try:
        toks = blocks(1, 2)
        be.MapRange(0, 2 * PAGE)
        be.HarvestPrefix(toks, PAGE)
        old = table(be, 2)
        be.MapRange(PAGE + 5, 3)               # inside block 1: copy-on-write
        new = table(be, 2)
        assert new[0] == old[0] and new[1] != old[1]
        be.SetCacheLen(0)
        assert be.RestorePrefix(toks, PAGE) == 2 * PAGE
        assert table(be, 2) == old             # the harvested page is intact
    finally:
        be.Dispose()


def test_least_recently_harvested_is_evicted_first():
    # KvBlockStoreTests.EvictsLeastRecentlyUsed_WhenOverCap, for a pool of 3 pages
    be = host(3 * PAGE)
    try:
        t0, t1, t2 = blocks(1), blocks(2), blocks(3)
        for t in (t0, t1, t2):
            be.SetCacheLen(0)
            be.MapRange(0, PAGE)
            be.HarvestPrefix(t, PAGE)
        assert be.store_info() == {"entries": 3, "pages_free": 0}
        be.SetCacheLen(0)
        be.MapRange(0, PAGE)                   # evicts t0's entry
        assert be.store_info()["entries"] == 2
        be.SetCacheLen(0)
        assert be.RestorePrefix(t0, PAGE) == 0
        assert be.RestorePrefix(t1, PAGE) == PAGE
        be.SetCacheLen(0)
        assert be.RestorePrefix(t2, PAGE) == PAGE
    finally:
        be.Dispose()


def test_pool_exhausted_when_every_page_is_live():
    be = host(2 * PAGE)
    try:
        be.MapRange(0, 2 * PAGE)
        be.HarvestPrefix(blocks(1, 2), PAGE)
        with pytest.raises(NotSupportedError):  # both pinned pages are live
            be.MapRange(70, 1)
    finally:
        be.Dispose()


def test_block_size_must_be_the_page():
    be = host(64 * 4)
    try:
        with pytest.raises(NotSupportedError):
            be.HarvestPrefix(blocks(1), 32)
        with pytest.raises(NotSupportedError):
            be.RestorePrefix(blocks(1), 128)
        assert HipBackend.SupportsBlockStore and HipBackend.DeviceBlockTokens == PAGE
    finally:
        be.Dispose()


# ---- randomized sequences: C ABI == oracle --------------------------------------

@pytest.mark.parametrize("seed", range(6))
def test_random_sequences_match_the_oracle(seed):
    rng = random.Random(seed)
    pages = rng.choice([4, 6, 9])
    be = host(pages * PAGE)
    model = B.BlockStoreModel(pages * PAGE)
    vocab = [blocks(v) for v in range(5)]
    try:
        for step in range(120):
            op = rng.choice(["map", "map", "set_len", "harvest", "restore"])
            if op == "map":
                pos = rng.randrange(0, pages * PAGE)
                ln = rng.randrange(1, 2 * PAGE)
                ln = min(ln, pages * PAGE - pos)
                got = exp = None
                try:
                    be.MapRange(pos, ln)
                except NotSupportedError:
                    got = "capacity"
                try:
                    model.ensure_written(pos, ln)
                except B.CapacityError:
                    exp = "capacity"
                assert got == exp, (step, op, pos, ln)  # a failed call keeps what it mapped
            elif op == "set_len":
                ln = rng.randrange(0, pages * PAGE + 1)
                be.SetCacheLen(ln)
                model.set_len(ln)
            else:
                nb = rng.randrange(1, pages + 1)
                toks = np.concatenate([vocab[rng.randrange(5)] for _ in range(nb)])
                cut = rng.randrange(0, len(toks) + 1)
                if op == "harvest":
                    be.HarvestPrefix(toks[:cut], PAGE)
                    model.harvest(toks[:cut], PAGE)
                else:
                    assert be.RestorePrefix(toks[:cut], PAGE) == model.restore(toks[:cut], PAGE), step
            assert table(be, pages) == model.tab, (step, op)
            info = be.store_info()
            assert info == {"entries": len(model.store), "pages_free": model.pages_free()}, (step, op)
    finally:
        be.Dispose()
