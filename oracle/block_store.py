"""CPU restatement of the reference's device block store and page allocator.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the page
bookkeeping behind hymt_kv_map / hymt_kv_set_len / hymt_kv_harvest /
hymt_kv_restore.  The product (hymt2sharp_amd) never imports this module.

Restates, in plain Python, the Metal backend's block table and hash store
(src/HyMT2Sharp/Backends/Metal/MetalBackend.cs):
  * EnsureWrittenRange (:294-318): map every block of a write range; a block
    whose page is pinned by a store entry gets a fresh page, with a page copy
    queued when the write starts inside the block;
  * AllocPhys (:233-253): free list (last freed first), then an untouched
    page, then evict entries least recently harvested first whose page is
    not mapped in the live range;
  * RemoveEntry / ReleaseOrFree (:265-281);
  * HarvestPrefix (:330-356) and RestorePrefix (:358-382);
and KvBlockStore.ChainHash / Seed (src/HyMT2Sharp/KvBlockStore.cs:49-60).

One deliberate difference, shared with the HIP build: SetCacheLen
(IComputeBackend.cs:82-87) unmaps the blocks that start at or past the new
length and recycles their pages unless pinned (the Metal backend only
records the length and leaves the blocks mapped until reused).
"""
from __future__ import annotations

SEED = 14695981039346656037  # KvBlockStore.Seed (KvBlockStore.cs:49)
PRIME = 1099511628211        # FNV-1a 64-bit prime (KvBlockStore.cs:57)
MASK = (1 << 64) - 1
PAGE = 64                    # DeviceBlockTokens (MetalBackend.cs:49-50)


def chain_hash(prev: int, tokens) -> int:
    """KvBlockStore.ChainHash (KvBlockStore.cs:51-60): h ^= (uint)t; h *= prime."""
    h = prev
    for t in tokens:
        h ^= int(t) & 0xFFFFFFFF
        h = (h * PRIME) & MASK
    return h


class CapacityError(Exception):
    pass


class BlockSizeError(Exception):
    pass


class BlockStoreModel:
    def __init__(self, max_tokens: int):
        self.max_pages = (max_tokens + PAGE - 1) // PAGE
        self.tab = [-1] * self.max_pages
        self.free = []          # stack: last freed is reused first
        self.next = 0
        self.live_len = 0
        self.store = {}         # hash -> (phys, tokens tuple)
        self.phys_hash = {}     # phys -> hash
        self.lru = []           # hashes, least recently harvested first
        self.copies = []        # (src, dst) page copies queued by copy-on-write

    # -- queries -------------------------------------------------------------
    def pinned(self, p: int) -> bool:
        return p in self.phys_hash

    def pages_free(self) -> int:
        return len(self.free) + self.max_pages - self.next

    def mapped(self) -> int:
        return sum(p >= 0 for p in self.tab)

    # -- allocator (MetalBackend.cs:233-281) ---------------------------------
    def _alloc(self) -> int:
        if self.free:
            return self.free.pop()
        if self.next < self.max_pages:
            self.next += 1
            return self.next - 1
        live_blocks = (self.live_len + PAGE - 1) // PAGE
        live = {self.tab[i] for i in range(min(live_blocks, self.max_pages)) if self.tab[i] >= 0}
        for h in list(self.lru):
            p = self.store[h][0]
            if p not in live:
                self._remove_entry(h)
                return self.free.pop()
        raise CapacityError("KV page pool exhausted")

    def _unpin(self, h: int):
        p, _ = self.store.pop(h)
        del self.phys_hash[p]
        self.lru.remove(h)

    def _remove_entry(self, h: int):
        p = self.store[h][0]
        self._unpin(h)
        for i in range(self.max_pages):
            if self.tab[i] == p:
                self.tab[i] = -1
        self.free.append(p)

    def _release_or_free(self, p: int):
        if p < 0 or self.pinned(p) or p in self.tab:
            return
        self.free.append(p)

    # -- EnsureWrittenRange (MetalBackend.cs:294-318) ----------------------------
    def ensure_written(self, pos: int, length: int):
        if length <= 0:
            return
        if pos < 0 or pos + length > self.max_pages * PAGE:
            raise CapacityError("KV capacity exceeded")
        self.live_len = max(self.live_len, pos + length)
        first, last = pos // PAGE, (pos + length - 1) // PAGE
        for b in range(first, last + 1):
            if self.tab[b] < 0:
                self.tab[b] = self._alloc()
            elif self.pinned(self.tab[b]):
                fresh = self._alloc()
                if b == first and pos % PAGE:
                    self.copies.append((self.tab[b], fresh))
                self.tab[b] = fresh

    # -- SetCacheLen (see the module docstring) -----------------------------
    def set_len(self, length: int):
        length = max(length, 0)
        keep = (length + PAGE - 1) // PAGE
        for b in range(keep, self.max_pages):
            p = self.tab[b]
            if p >= 0:
                self.tab[b] = -1
                self._release_or_free(p)
        self.live_len = min(length, self.max_pages * PAGE)

    # -- HarvestPrefix (MetalBackend.cs:330-356) --------------------------------
    def harvest(self, tokens, block_tokens: int):
        if block_tokens != PAGE:
            raise BlockSizeError(block_tokens)
        h = SEED
        b = 0
        while b * PAGE + PAGE <= len(tokens) and b < self.max_pages:
            toks = tuple(int(t) for t in tokens[b * PAGE:(b + 1) * PAGE])
            h = chain_hash(h, toks)
            phys = self.tab[b]
            b += 1
            if phys < 0:
                continue
            cur = self.store.get(h)
            if cur is not None and cur[1] == toks:
                self.lru.remove(h)
                self.lru.append(h)
                continue
            if cur is not None:
                self._unpin(h)
                self._release_or_free(cur[0])
            if phys in self.phys_hash:
                self._unpin(self.phys_hash[phys])
            self.store[h] = (phys, toks)
            self.phys_hash[phys] = h
            self.lru.append(h)

    # -- RestorePrefix (MetalBackend.cs:358-382) --------------------------------
    def restore(self, tokens, block_tokens: int) -> int:
        if block_tokens != PAGE:
            raise BlockSizeError(block_tokens)
        h = SEED
        hit = 0
        i = 0
        while i * PAGE + PAGE <= len(tokens) and i < self.max_pages:
            toks = tuple(int(t) for t in tokens[i * PAGE:(i + 1) * PAGE])
            h = chain_hash(h, toks)
            e = self.store.get(h)
            if e is None or e[1] != toks:
                break
            old = self.tab[i]
            self.tab[i] = e[0]
            if old != e[0]:
                self._release_or_free(old)
            hit += 1
            i += 1
        return hit * PAGE
