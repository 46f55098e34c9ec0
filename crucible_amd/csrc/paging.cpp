// Paged KV bookkeeping (see paging.hpp) and its C API from crucible_attn.h.
#include "paging.hpp"

#include <cstdint>
#include <cstdio>
#include <cstring>

namespace crucible {

namespace {
// The pool's shape, checked before anything is allocated: page ids reach the device in
// int32 tables, so a pool holds at most 2^31 pages, and the byte count of both pools
// (2 x pages x elements x 2 bytes) must fit int64.
int64_t checked_pages(int64_t n_pages) {
    if (n_pages < 0 || n_pages > (int64_t)INT32_MAX + 1)
        throw PagingError("page count out of range");
    return n_pages;
}

int64_t checked_page_elems(int64_t n_pages, int64_t n_layer, int64_t kv_dim) {
    if (n_layer <= 0 || kv_dim <= 0) throw PagingError("n_layer and kv_dim must be positive");
    int64_t elems, bytes;
    if (__builtin_mul_overflow(n_layer, kPagingTokens, &elems) ||
        __builtin_mul_overflow(elems, kv_dim, &elems) ||
        __builtin_mul_overflow(elems, (int64_t)4, &bytes) ||
        __builtin_mul_overflow(bytes, n_pages, &bytes))
        throw PagingError("pool size overflows");
    return elems;
}
}  // namespace

PagePool::PagePool(int64_t n_pages, int64_t n_layer, int64_t kv_dim)
    : n_pages_(checked_pages(n_pages)),
      page_elems_(checked_page_elems(n_pages, n_layer, kv_dim)),
      in_use_((size_t)n_pages, false) {
    free_.reserve(n_pages);
    // Reverse order so the first allocation is page 0 (paged.rs:76-78).
    for (int64_t i = n_pages; i-- > 0;) free_.push_back((uint32_t)i);
}

uint32_t PagePool::alloc() {
    if (free_.empty())
        throw PagingError("kv page pool exhausted: all " + std::to_string(n_pages_) + " pages (" +
                          std::to_string(capacity_tokens()) + " tokens) are in use");
    const uint32_t id = free_.back();
    free_.pop_back();
    in_use_[id] = true;
    return id;
}

void PagePool::release(int64_t id) {
    if (id < 0 || id >= n_pages_)
        throw PagingError("page " + std::to_string(id) + " out of range (pool has " +
                          std::to_string(n_pages_) + " pages)");
    if (!in_use_[id]) throw PagingError("double free of kv page " + std::to_string(id));
    in_use_[id] = false;
    free_.push_back((uint32_t)id);
}

std::pair<uint32_t, int64_t> SequencePages::translate(int64_t pos) const {
    if (pos < 0 || pos >= len_)
        throw PagingError("position " + std::to_string(pos) + " outside sequence of length " +
                          std::to_string(len_));
    return {pages_[pos / kPagingTokens], pos % kPagingTokens};
}

void SequencePages::grow(PagePool& pool, int64_t extra) {
    if (extra < 0) throw PagingError("negative growth");
    if (extra > INT64_MAX - kPagingTokens - len_) throw PagingError("growth overflows");
    const int64_t target = len_ + extra;
    const int64_t needed = (target + kPagingTokens - 1) / kPagingTokens;
    std::vector<uint32_t> taken;
    while ((int64_t)(pages_.size() + taken.size()) < needed) {
        try {
            taken.push_back(pool.alloc());
        } catch (const PagingError&) {
            // Return every page taken by this call before reporting (paged.rs:193-217).
            for (uint32_t id : taken) pool.release(id);
            throw;
        }
    }
    pages_.insert(pages_.end(), taken.begin(), taken.end());
    len_ = target;
}

void SequencePages::release(PagePool& pool) {
    for (uint32_t id : pages_) pool.release(id);
    pages_.clear();
    len_ = 0;
}

std::vector<int32_t> SequencePages::table_padded(int64_t stride) const {
    if (stride < n_pages()) throw PagingError("table stride smaller than the page count");
    std::vector<int32_t> out((size_t)stride, 0);
    for (size_t i = 0; i < pages_.size(); ++i) out[i] = (int32_t)pages_[i];
    return out;
}

int64_t request_page_reservation(int64_t prompt, int64_t generated, int64_t context) {
    if (prompt <= 0 || generated <= 0)
        throw PagingError("prompt length and output token budget must be positive");
    int64_t positions;
    if (__builtin_add_overflow(prompt, generated - 1, &positions) ||
        positions > INT64_MAX - kPagingTokens)
        throw PagingError("request length overflows");
    if (positions > context)
        throw PagingError("request needs " + std::to_string(positions) +
                          " cache positions, capacity is " + std::to_string(context));
    return (positions + kPagingTokens - 1) / kPagingTokens;
}

bool PageReservations::try_reserve(int64_t pages) {
    if (pages <= 0 || pages > capacity_)
        throw PagingError("request needs " + std::to_string(pages) +
                          " KV pages but pool capacity is " + std::to_string(capacity_));
    if (pages > capacity_ - held_) return false;
    held_ += pages;
    return true;
}

void PageReservations::release(int64_t pages) {
    if (pages < 0 || pages > held_) throw PagingError("released more KV reservation than held");
    held_ -= pages;
}

}  // namespace crucible

// ------------------------------------------------------------------ C API
#include "../../include/crucible_attn.h"

namespace crucible {
void set_error(int status, const char* fmt, ...);
}

struct crucible_page_pool {
    crucible::PagePool pool;
};
struct crucible_seq_pages {
    crucible::SequencePages seq;
};

namespace {
int paging_fail(const std::exception& e) {
    crucible::set_error(CRUCIBLE_ERR_INVALID, "%s", e.what());
    return CRUCIBLE_ERR_INVALID;
}
}  // namespace

extern "C" crucible_page_pool* crucible_page_pool_new(int64_t n_pages, int64_t n_layer,
                                                      int64_t kv_dim) {
    try {
        return new crucible_page_pool{crucible::PagePool(n_pages, n_layer, kv_dim)};
    } catch (const std::exception& e) {
        paging_fail(e);
        return nullptr;
    }
}
extern "C" void crucible_page_pool_free(crucible_page_pool* p) { delete p; }
extern "C" int64_t crucible_page_pool_free_pages(const crucible_page_pool* p) {
    return p->pool.free_pages();
}
extern "C" int64_t crucible_page_pool_used_pages(const crucible_page_pool* p) {
    return p->pool.used_pages();
}
extern "C" int64_t crucible_page_pool_alloc(crucible_page_pool* p) {
    try {
        return p->pool.alloc();
    } catch (const std::exception& e) {
        paging_fail(e);
        return -1;
    }
}
extern "C" int crucible_page_pool_release(crucible_page_pool* p, int64_t page) {
    try {
        p->pool.release(page);
        return CRUCIBLE_OK;
    } catch (const std::exception& e) {
        return paging_fail(e);
    }
}
extern "C" crucible_seq_pages* crucible_seq_pages_new(void) { return new crucible_seq_pages{}; }
extern "C" void crucible_seq_pages_free(crucible_seq_pages* s) { delete s; }
extern "C" int64_t crucible_seq_pages_len(const crucible_seq_pages* s) { return s->seq.len(); }
extern "C" int64_t crucible_seq_pages_n_pages(const crucible_seq_pages* s) {
    return s->seq.n_pages();
}
extern "C" int crucible_seq_pages_grow(crucible_seq_pages* s, crucible_page_pool* p,
                                       int64_t extra) {
    try {
        s->seq.grow(p->pool, extra);
        return CRUCIBLE_OK;
    } catch (const std::exception& e) {
        return paging_fail(e);
    }
}
extern "C" int crucible_seq_pages_release(crucible_seq_pages* s, crucible_page_pool* p) {
    try {
        s->seq.release(p->pool);
        return CRUCIBLE_OK;
    } catch (const std::exception& e) {
        return paging_fail(e);
    }
}
extern "C" int crucible_seq_pages_translate(const crucible_seq_pages* s, int64_t pos,
                                            int64_t* page, int64_t* slot) {
    try {
        const auto ps = s->seq.translate(pos);
        *page = ps.first;
        *slot = ps.second;
        return CRUCIBLE_OK;
    } catch (const std::exception& e) {
        return paging_fail(e);
    }
}
extern "C" int crucible_seq_pages_table_padded(const crucible_seq_pages* s, int64_t stride,
                                               int32_t* out) {
    try {
        const auto t = s->seq.table_padded(stride);
        std::memcpy(out, t.data(), t.size() * sizeof(int32_t));
        return CRUCIBLE_OK;
    } catch (const std::exception& e) {
        return paging_fail(e);
    }
}
extern "C" int64_t crucible_request_page_reservation(int64_t prompt, int64_t generated,
                                                     int64_t context) {
    try {
        return crucible::request_page_reservation(prompt, generated, context);
    } catch (const std::exception& e) {
        paging_fail(e);
        return -1;
    }
}
