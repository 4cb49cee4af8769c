// kv_pages.hpp -- host bookkeeping of the paged K/V cache and its block store.
//
// Logical positions reach physical pages through one table shared by all
// layers: page(j) = tab[j / 64], row = j % 64, as in the reference's Metal
// backend (MetalBackend.cs:44-61 for the table, MslDecodeKernels.cs:96-100
// for the addressing).  Every layer owns a K pool and a V pool of the same
// page count, so one table entry names the same page slot in every layer.
//
// Block store (IComputeBackend.SupportsBlockStore / DeviceBlockTokens /
// HarvestPrefix / RestorePrefix, IComputeBackend.cs:49-87), after the Metal
// backend (MetalBackend.cs:224-387): a full 64-token block of a sequence is
// keyed by the chained FNV-1a hash of every token up to its end
// (KvBlockStore.ChainHash, KvBlockStore.cs:51-60).  Harvesting pins the
// block's page under that key; restoring points the table at pinned pages,
// so a shared prefix is reused without copying.  A pinned page is never
// written: a write into its block maps a fresh page (copy-on-write), and
// when the write starts inside the block the page's rows before it are
// copied over (the owner runs the queued copies before any kernel that
// writes the block).  Entries are evicted least recently harvested first
// when the pool runs out, never while their page is mapped in the live
// range.
//
// This class holds no device state.  The owner mirrors changed entries to
// the device copy of the table (dirty list) and runs the queued page copies
// before launching kernels that read them.
#pragma once

#include <cstdint>
#include <list>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace hymt {

struct CapacityError : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct BlockSizeError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

class KvPages {
  public:
    static constexpr int kPageTokens = 64;
    // KvBlockStore.Seed and the FNV-1a 64-bit prime (KvBlockStore.cs:49-60)
    static constexpr uint64_t kSeed = 14695981039346656037ULL;
    static constexpr uint64_t kPrime = 1099511628211ULL;

    struct Copy {
        int src, dst;  // whole-page copy src -> dst, every layer, K and V
    };

    KvPages() = default;
    KvPages(int max_tokens)
        : max_pages_((max_tokens + kPageTokens - 1) / kPageTokens),
          tab_(max_pages_, -1),
          refs_(max_pages_, 0),
          dirty_flag_(max_pages_, 0) {}

    static uint64_t chain_hash(uint64_t prev, const int32_t *tokens, int n) {
        uint64_t h = prev;
        for (int i = 0; i < n; i++) {
            h ^= (uint32_t)tokens[i];
            h *= kPrime;
        }
        return h;
    }

    int max_pages() const { return max_pages_; }
    int max_tokens() const { return max_pages_ * kPageTokens; }
    int live_len() const { return live_len_; }
    int store_entries() const { return (int)store_.size(); }
    // pages held neither by the table nor by a store entry
    int pages_free() const { return (int)free_.size() + (max_pages_ - next_); }
    int mapped() const {
        int n = 0;
        for (int p : tab_) n += p >= 0;
        return n;
    }
    const std::vector<int32_t> &table() const { return tab_; }
    bool pinned(int phys) const { return phys_hash_.count(phys) != 0; }

    // Physical page of logical block b, or -1.
    int phys(int b) const { return (b >= 0 && b < max_pages_) ? tab_[b] : -1; }

    // Map every logical block covering [pos, pos+len) for writing
    // (MetalBackend.cs EnsureWrittenRange, :294-318): unmapped blocks get a
    // page, blocks on a pinned page get a fresh one (copy queued when the
    // write starts inside the block).  Throws CapacityError past the pool.
    void ensure_written(int pos, int len) {
        if (len <= 0) return;
        if (pos < 0 || (long)pos + len > (long)max_tokens())
            throw CapacityError("KV capacity " + std::to_string(max_tokens()) +
                                " exceeded at " + std::to_string((long)pos + len));
        if (pos + len > live_len_) live_len_ = pos + len;
        int first = pos / kPageTokens, last = (pos + len - 1) / kPageTokens;
        for (int b = first; b <= last; b++) {
            if (tab_[b] < 0) {
                set_slot(b, alloc());
            } else if (pinned(tab_[b])) {
                const int fresh = alloc();
                if (b == first && pos % kPageTokens != 0) copies_.push_back({tab_[b], fresh});
                set_slot(b, fresh);
            }
        }
    }

    // True when a write of [pos, pos+len) would queue a copy-on-write copy.
    bool needs_copy(int pos, int len) const {
        if (len <= 0 || pos < 0 || pos % kPageTokens == 0) return false;
        const int p = phys(pos / kPageTokens);
        return p >= 0 && pinned(p);
    }

    // True when every position of [0, len) is mapped.
    bool resident(int len) const {
        if (len > max_tokens()) return false;
        for (int b = 0; b * kPageTokens < len; b++)
            if (tab_[b] < 0) return false;
        return true;
    }

    // Live prefix length (IComputeBackend.SetCacheLen, IComputeBackend.cs:82-87):
    // blocks that start at or past `len` are unmapped; their pages return to
    // the pool unless a store entry pins them.
    void set_len(int len) {
        if (len < 0) len = 0;
        int keep = (len + kPageTokens - 1) / kPageTokens;
        for (int b = keep; b < max_pages_; b++)
            if (tab_[b] >= 0) {
                const int p = tab_[b];
                set_slot(b, -1);
                release_or_free(p);
            }
        live_len_ = len < max_tokens() ? len : max_tokens();
    }

    // HarvestPrefix (MetalBackend.cs:330-356): pin the page of every full
    // block of tokens[0, n) under its chained hash.  Blocks never mapped are
    // skipped (the chain still advances).  block_tokens must be 64.
    void harvest(const int32_t *tokens, int n, int block_tokens) {
        check_block(block_tokens);
        uint64_t h = kSeed;
        for (int b = 0; (long)b * kPageTokens + kPageTokens <= n && b < max_pages_; b++) {
            const int32_t *toks = tokens + (size_t)b * kPageTokens;
            h = chain_hash(h, toks, kPageTokens);
            const int phys = tab_[b];
            if (phys < 0) continue;
            auto it = store_.find(h);
            if (it != store_.end() && same(it->second.toks, toks)) {
                lru_.splice(lru_.end(), lru_, it->second.node);  // most recent
                continue;
            }
            if (it != store_.end()) {  // same key, other tokens: replace
                const int op = it->second.phys;
                unpin(h);
                release_or_free(op);
            }
            auto ph = phys_hash_.find(phys);
            if (ph != phys_hash_.end()) unpin(ph->second);
            Entry e;
            e.phys = phys;
            e.toks.assign(toks, toks + kPageTokens);
            e.node = lru_.insert(lru_.end(), h);
            store_.emplace(h, std::move(e));
            phys_hash_[phys] = h;
        }
    }

    // RestorePrefix (MetalBackend.cs:358-382): map the longest run of full
    // blocks of tokens[0, n) found in the store, from block 0; returns the
    // number of tokens restored (a multiple of 64).
    int restore(const int32_t *tokens, int n, int block_tokens) {
        check_block(block_tokens);
        uint64_t h = kSeed;
        int hit = 0;
        for (int i = 0; (long)i * kPageTokens + kPageTokens <= n && i < max_pages_; i++) {
            const int32_t *toks = tokens + (size_t)i * kPageTokens;
            h = chain_hash(h, toks, kPageTokens);
            auto it = store_.find(h);
            if (it == store_.end() || !same(it->second.toks, toks)) break;
            const int old = tab_[i];
            set_slot(i, it->second.phys);
            if (old != it->second.phys) release_or_free(old);
            hit++;
        }
        return hit * kPageTokens;
    }

    // Entries changed since the last take_dirty(); clears the list.
    std::vector<int> take_dirty() {
        std::vector<int> d;
        d.swap(dirty_);
        for (int b : d) dirty_flag_[b] = 0;
        return d;
    }
    bool has_dirty() const { return !dirty_.empty(); }

    // Page copies queued by copy-on-write; clears the list.
    std::vector<Copy> take_copies() {
        std::vector<Copy> c;
        c.swap(copies_);
        return c;
    }
    bool has_copies() const { return !copies_.empty(); }

  private:
    struct Entry {
        int phys = -1;
        std::vector<int32_t> toks;
        std::list<uint64_t>::iterator node;
    };

    static void check_block(int block_tokens) {
        if (block_tokens != kPageTokens)
            throw BlockSizeError("the device block store uses " + std::to_string(kPageTokens) +
                                 "-token blocks, got " + std::to_string(block_tokens));
    }
    static bool same(const std::vector<int32_t> &a, const int32_t *b) {
        for (int i = 0; i < kPageTokens; i++)
            if (a[i] != b[i]) return false;
        return true;
    }

    // AllocPhys (MetalBackend.cs:233-253): free list, then an untouched page,
    // then evict least recently harvested entries until one whose page is not
    // mapped in the live range frees.
    int alloc() {
        if (!free_.empty()) {
            const int p = free_.back();
            free_.pop_back();
            return p;
        }
        if (next_ < max_pages_) return next_++;
        const int live_blocks = (live_len_ + kPageTokens - 1) / kPageTokens;
        std::unordered_set<int> live;
        for (int i = 0; i < live_blocks && i < max_pages_; i++)
            if (tab_[i] >= 0) live.insert(tab_[i]);
        for (auto it = lru_.begin(); it != lru_.end(); ++it) {
            const int p = store_.at(*it).phys;
            if (!live.count(p)) {
                remove_entry(*it);
                const int q = free_.back();
                free_.pop_back();
                return q;
            }
        }
        throw CapacityError("KV page pool exhausted (" + std::to_string(max_pages_) + " pages of " +
                            std::to_string(kPageTokens) + " tokens)");
    }
    void unpin(uint64_t h) {
        auto it = store_.find(h);
        phys_hash_.erase(it->second.phys);
        lru_.erase(it->second.node);
        store_.erase(it);
    }
    // Eviction (MetalBackend.cs:265-272): the page is outside the live range;
    // stale table slots still naming it are cleared, then it is recycled.
    void remove_entry(uint64_t h) {
        const int p = store_.at(h).phys;
        unpin(h);
        for (int i = 0; i < max_pages_ && refs_[p] > 0; i++)
            if (tab_[i] == p) set_slot(i, -1);
        free_.push_back(p);
    }
    // Recycle a page no table slot names and no entry pins
    // (MetalBackend.cs:274-281).
    void release_or_free(int p) {
        if (p < 0 || pinned(p) || refs_[p] > 0) return;
        free_.push_back(p);
    }
    void set_slot(int b, int p) {
        if (tab_[b] >= 0) refs_[tab_[b]]--;
        tab_[b] = p;
        if (p >= 0) refs_[p]++;
        mark(b);
    }
    void mark(int b) {
        if (!dirty_flag_[b]) {
            dirty_flag_[b] = 1;
            dirty_.push_back(b);
        }
    }

    int max_pages_ = 0;
    std::vector<int32_t> tab_;
    std::vector<int> refs_;  // table slots naming each page
    std::vector<int> free_;
    int next_ = 0;
    int live_len_ = 0;
    std::vector<int> dirty_;
    std::vector<uint8_t> dirty_flag_;
    std::vector<Copy> copies_;
    std::unordered_map<uint64_t, Entry> store_;
    std::unordered_map<int, uint64_t> phys_hash_;
    std::list<uint64_t> lru_;  // front: least recently harvested
};

}  // namespace hymt
