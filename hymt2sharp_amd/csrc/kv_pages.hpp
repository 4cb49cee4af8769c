// kv_pages.hpp -- host bookkeeping of the paged K/V cache.
//
// Logical positions reach physical pages through one table shared by all
// layers: page(j) = tab[j / 64], row = j % 64, as in the reference's Metal
// backend (MetalBackend.cs:44-61 for the table, MslDecodeKernels.cs:96-100
// for the addressing).  Every layer owns a K pool and a V pool of the same
// page count, so one table entry names the same page slot in every layer.
//
// This class holds no device state.  The owner mirrors changed entries to
// the device copy of the table (dirty list) before launching kernels that
// read it.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace hymt {

struct CapacityError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

class KvPages {
  public:
    static constexpr int kPageTokens = 64;

    KvPages() = default;
    KvPages(int max_tokens)
        : max_pages_((max_tokens + kPageTokens - 1) / kPageTokens),
          tab_(max_pages_, -1) {}

    int max_pages() const { return max_pages_; }
    int max_tokens() const { return max_pages_ * kPageTokens; }
    int mapped() const { return mapped_; }
    int live_len() const { return live_len_; }
    const std::vector<int32_t> &table() const { return tab_; }

    // Physical page of logical block b, or -1.
    int phys(int b) const { return (b >= 0 && b < max_pages_) ? tab_[b] : -1; }

    // Map every logical block covering [pos, pos+len) (MetalBackend.cs
    // EnsureWrittenRange, :294-318).  Throws CapacityError past the pool.
    void ensure_written(int pos, int len) {
        if (len <= 0) return;
        if (pos < 0 || (long)pos + len > (long)max_tokens())
            throw CapacityError("KV capacity " + std::to_string(max_tokens()) +
                                " exceeded at " + std::to_string((long)pos + len));
        int first = pos / kPageTokens, last = (pos + len - 1) / kPageTokens;
        for (int b = first; b <= last; b++)
            if (tab_[b] < 0) {
                tab_[b] = alloc();
                mark(b);
            }
        if (pos + len > live_len_) live_len_ = pos + len;
    }

    // True when every position of [0, len) is mapped.
    bool resident(int len) const {
        if (len > max_tokens()) return false;
        for (int b = 0; b * kPageTokens < len; b++)
            if (tab_[b] < 0) return false;
        return true;
    }

    // Live prefix length (IComputeBackend.SetCacheLen, IComputeBackend.cs:82-87):
    // pages that start at or past `len` are unmapped and recycled.
    void set_len(int len) {
        if (len < 0) len = 0;
        int keep = (len + kPageTokens - 1) / kPageTokens;
        for (int b = keep; b < max_pages_; b++)
            if (tab_[b] >= 0) {
                free_.push_back(tab_[b]);
                tab_[b] = -1;
                mapped_--;
                mark(b);
            }
        live_len_ = len < max_tokens() ? len : max_tokens();
    }

    // Entries changed since the last take_dirty(); clears the list.
    std::vector<int> take_dirty() {
        std::vector<int> d;
        d.swap(dirty_);
        for (int b : d) dirty_flag_[b] = 0;
        return d;
    }
    bool has_dirty() const { return !dirty_.empty(); }

  private:
    int alloc() {
        int p;
        if (!free_.empty()) {
            p = free_.back();
            free_.pop_back();
        } else {
            p = next_++;
        }
        mapped_++;
        return p;
    }
    void mark(int b) {
        if ((int)dirty_flag_.size() < max_pages_) dirty_flag_.assign(max_pages_, 0);
        if (!dirty_flag_[b]) {
            dirty_flag_[b] = 1;
            dirty_.push_back(b);
        }
    }

    int max_pages_ = 0;
    std::vector<int32_t> tab_;
    std::vector<int> free_;
    int next_ = 0;
    int mapped_ = 0;
    int live_len_ = 0;
    std::vector<int> dirty_;
    std::vector<uint8_t> dirty_flag_;
};

}  // namespace hymt
