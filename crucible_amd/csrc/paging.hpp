// Paged KV bookkeeping on the host: the reference allocator restated in C++.
//
// Reference: engine/src/paged.rs (PagePool :64-144, SequencePages :151-242) and
// engine/src/prefill.rs (request_page_reservation :160-172, PageReservations :175-206).
// The policy is unchanged: a stack of free ids initialised in reverse (the first
// alloc returns page 0), explicit exhaustion and double-free errors, all-or-nothing
// growth, and zero-padded tables for the device. Plain C++ with no HIP dependency,
// so its known-answer tests run on any CPU.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace crucible {

constexpr int64_t kPagingTokens = 16;

class PagingError : public std::runtime_error {
  public:
    using std::runtime_error::runtime_error;
};

class PagePool {
  public:
    PagePool(int64_t n_pages, int64_t n_layer, int64_t kv_dim);

    int64_t n_pages() const { return n_pages_; }
    int64_t free_pages() const { return (int64_t)free_.size(); }
    int64_t used_pages() const { return n_pages_ - free_pages(); }
    // Elements of one page in each pool: n_layer * 16 * kv_dim.
    int64_t page_elems() const { return page_elems_; }
    // Bytes of one page in each pool for fp16 storage.
    int64_t page_bytes() const { return page_elems_ * 2; }
    int64_t total_bytes() const { return 2 * n_pages_ * page_bytes(); }
    int64_t capacity_tokens() const { return n_pages_ * kPagingTokens; }

    uint32_t alloc();               // throws PagingError("... exhausted ...")
    void release(int64_t id);       // throws on out of range / double free

  private:
    int64_t n_pages_;
    int64_t page_elems_;
    std::vector<uint32_t> free_;
    std::vector<bool> in_use_;
};

class SequencePages {
  public:
    int64_t len() const { return len_; }
    bool empty() const { return len_ == 0; }
    const std::vector<uint32_t>& pages() const { return pages_; }
    int64_t n_pages() const { return (int64_t)pages_.size(); }
    int64_t wasted_slots() const { return n_pages() * kPagingTokens - len_; }

    std::pair<uint32_t, int64_t> translate(int64_t pos) const;
    void grow(PagePool& pool, int64_t extra);
    void release(PagePool& pool);
    std::vector<int32_t> table_padded(int64_t stride) const;

  private:
    std::vector<uint32_t> pages_;
    int64_t len_ = 0;
};

// Pages a request needs through its final generated token: ceil((prompt + gen - 1) / 16).
int64_t request_page_reservation(int64_t prompt, int64_t generated, int64_t context);

class PageReservations {
  public:
    explicit PageReservations(int64_t capacity) : capacity_(capacity) {}
    bool try_reserve(int64_t pages);
    void release(int64_t pages);
    int64_t held() const { return held_; }

  private:
    int64_t capacity_;
    int64_t held_ = 0;
};

}  // namespace crucible
