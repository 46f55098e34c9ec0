// Known-answer tests for paging.hpp, ported one for one from the reference's own unit
// tests: engine/src/paged.rs:244-496 (15 tests) and engine/src/prefill.rs:394-453
// (reservations). Built with plain g++ (no GPU) and run by tests/test_paging.py.
// The one intended difference: pages hold fp16, so byte sizes are half the
// reference's f32 figures (page_geometry_matches_layout).
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <set>
#include <string>
#include <vector>

#include "paging.hpp"

namespace crucible {
void set_error(int, const char*, ...) {}
}  // namespace crucible

using namespace crucible;

static int g_failures = 0;
#define CHECK(cond)                                                                   \
    do {                                                                              \
        if (!(cond)) {                                                                \
            std::fprintf(stderr, "  CHECK failed at %s:%d: %s\n", __FILE__, __LINE__, \
                         #cond);                                                      \
            ++g_failures;                                                             \
        }                                                                             \
    } while (0)

template <class F>
static std::string error_of(F&& f) {
    try {
        f();
    } catch (const PagingError& e) {
        return e.what();
    }
    return "";
}

static const int64_t N_LAYER = 12;
static const int64_t KV_DIM = 192;
static PagePool pool(int64_t n) { return PagePool(n, N_LAYER, KV_DIM); }

static void allocates_in_order_and_tracks_counts() {
    PagePool p = pool(4);
    CHECK(p.free_pages() == 4);
    CHECK(p.used_pages() == 0);
    CHECK(p.alloc() == 0);
    CHECK(p.alloc() == 1);
    CHECK(p.free_pages() == 2);
    CHECK(p.used_pages() == 2);
}

static void page_geometry_matches_layout() {
    PagePool p = pool(64);
    CHECK(p.page_elems() == N_LAYER * 16 * KV_DIM);
    CHECK(p.capacity_tokens() == 64 * 16);
    // Both fp16 pools together equal the contiguous fp16 cache they replace.
    CHECK(p.total_bytes() == 2 * N_LAYER * 1024 * KV_DIM * 2);
}

static void grows_lazily_one_page_at_a_time() {
    PagePool pl = pool(8);
    SequencePages s;
    s.grow(pl, 1);
    CHECK(s.n_pages() == 1);
    CHECK(pl.used_pages() == 1);
    s.grow(pl, 16 - 1);
    CHECK(s.len() == 16);
    CHECK(s.n_pages() == 1);
    CHECK(s.wasted_slots() == 0);
    s.grow(pl, 1);
    CHECK(s.n_pages() == 2);
    CHECK(s.wasted_slots() == 16 - 1);
}

static void translation_crosses_page_boundaries() {
    PagePool pl = pool(8);
    SequencePages s;
    s.grow(pl, 16 * 2 + 3);
    CHECK(s.n_pages() == 3);
    const auto& pg = s.pages();
    CHECK(s.translate(0) == std::make_pair(pg[0], (int64_t)0));
    CHECK(s.translate(15) == std::make_pair(pg[0], (int64_t)15));
    CHECK(s.translate(16) == std::make_pair(pg[1], (int64_t)0));
    CHECK(s.translate(17) == std::make_pair(pg[1], (int64_t)1));
    CHECK(s.translate(32) == std::make_pair(pg[2], (int64_t)0));
}

static void translation_rejects_positions_past_the_end() {
    PagePool pl = pool(8);
    SequencePages s;
    s.grow(pl, 5);
    CHECK(!error_of([&] { s.translate(5); }).empty());
    CHECK(!error_of([&] { s.translate(INT64_MAX); }).empty());
}

static void sequences_never_share_a_physical_page() {
    PagePool pl = pool(16);
    SequencePages a, b, c;
    for (int i = 0; i < 3; ++i) {
        a.grow(pl, 16);
        b.grow(pl, 16);
        c.grow(pl, 16);
    }
    std::vector<uint32_t> all;
    for (auto* s : {&a, &b, &c}) all.insert(all.end(), s->pages().begin(), s->pages().end());
    std::set<uint32_t> unique(all.begin(), all.end());
    CHECK(all.size() == 9);
    CHECK(unique.size() == 9);
}

static void release_returns_pages_and_they_are_reused() {
    PagePool pl = pool(4);
    SequencePages s;
    s.grow(pl, 16 * 3);
    CHECK(pl.free_pages() == 1);
    s.release(pl);
    CHECK(pl.free_pages() == 4);
    CHECK(s.len() == 0);
    CHECK(s.n_pages() == 0);
    SequencePages t;
    t.grow(pl, 16 * 4);
    CHECK(t.n_pages() == 4);
    CHECK(pl.free_pages() == 0);
}

static void exhaustion_is_an_explicit_error() {
    PagePool pl = pool(2);
    SequencePages s;
    const std::string err = error_of([&] { s.grow(pl, 16 * 3); });
    CHECK(err.find("exhausted") != std::string::npos);
}

static void a_failed_grow_leaves_the_pool_untouched() {
    PagePool pl = pool(3);
    SequencePages s;
    s.grow(pl, 16);
    CHECK(pl.used_pages() == 1);
    CHECK(!error_of([&] { s.grow(pl, 16 * 4); }).empty());
    CHECK(pl.used_pages() == 1);
    CHECK(pl.free_pages() == 2);
    CHECK(s.len() == 16);
    CHECK(s.n_pages() == 1);
}

static void double_free_is_rejected() {
    PagePool pl = pool(2);
    const uint32_t id = pl.alloc();
    pl.release(id);
    const std::string err = error_of([&] { pl.release(id); });
    CHECK(err.find("double free") != std::string::npos);
}

static void releasing_an_out_of_range_page_is_rejected() {
    PagePool pl = pool(2);
    CHECK(!error_of([&] { pl.release(7); }).empty());
}

static void reset_then_reuse_gives_a_clean_sequence() {
    PagePool pl = pool(8);
    SequencePages s;
    s.grow(pl, 40);
    s.release(pl);
    CHECK(!error_of([&] { s.translate(0); }).empty());
    s.grow(pl, 3);
    CHECK(s.len() == 3);
    CHECK(s.n_pages() == 1);
}

static void padded_table_is_deterministic() {
    PagePool pl = pool(8);
    SequencePages s;
    s.grow(pl, 16 + 1);
    const auto t = s.table_padded(6);
    CHECK(t.size() == 6);
    CHECK(t[0] == (int32_t)s.pages()[0]);
    CHECK(t[1] == (int32_t)s.pages()[1]);
    CHECK(t[2] == 0 && t[3] == 0 && t[4] == 0 && t[5] == 0);
}

static void admission_after_reclaim_reuses_the_freed_pages() {
    PagePool pl = pool(4);
    SequencePages a, b;
    a.grow(pl, 16 * 2);
    b.grow(pl, 16 * 2);
    CHECK(pl.free_pages() == 0);
    SequencePages waiting;
    CHECK(!error_of([&] { waiting.grow(pl, 16); }).empty());
    a.release(pl);
    waiting.grow(pl, 16 * 2);
    CHECK(pl.free_pages() == 0);
    CHECK(waiting.n_pages() == 2);
    CHECK(b.len() == 16 * 2);
}

static void capacity_accounting_adds_up() {
    PagePool pl = pool(10);
    std::vector<SequencePages> seqs;
    for (int64_t len : {1, 17, 33}) {
        SequencePages s;
        s.grow(pl, len);
        seqs.push_back(s);
    }
    int64_t held = 0, wasted = 0, live = 0;
    for (const auto& s : seqs) {
        held += s.n_pages();
        wasted += s.wasted_slots();
        live += s.len();
    }
    CHECK(held == pl.used_pages());
    CHECK(held + pl.free_pages() == pl.n_pages());
    CHECK(held * 16 == live + wasted);
}

static void interleaved_free_and_realloc_stays_consistent() {
    PagePool pl = pool(6);
    SequencePages a, b;
    a.grow(pl, 16 * 2);
    b.grow(pl, 16 * 2);
    a.release(pl);
    SequencePages c;
    c.grow(pl, 16 * 4);
    CHECK(pl.free_pages() == 0);
    CHECK(b.len() == 16 * 2);
    for (uint32_t p : b.pages())
        for (uint32_t q : c.pages()) CHECK(p != q);
}

static void reservations_include_decode_growth_and_one_token_completion() {
    CHECK(request_page_reservation(16, 1, 1024) == 1);
    CHECK(request_page_reservation(16, 2, 1024) == 2);
    CHECK(request_page_reservation(17, 16, 1024) == 2);
    CHECK(request_page_reservation(17, 17, 1024) == 3);
    CHECK(!error_of([] { request_page_reservation(0, 1, 1024); }).empty());
    CHECK(!error_of([] { request_page_reservation(1, 0, 1024); }).empty());
    CHECK(!error_of([] { request_page_reservation(1024, 2, 1024); }).empty());
}

static void page_pressure_keeps_future_decode_pages_and_cancellation_returns_budget() {
    PagePool pl(4, 12, 192);
    PageReservations res(pl.n_pages());
    SequencePages first, second;
    CHECK(res.try_reserve(request_page_reservation(16, 17, 1024)));
    first.grow(pl, 16);
    CHECK(res.try_reserve(request_page_reservation(16, 17, 1024)));
    second.grow(pl, 16);
    CHECK(pl.free_pages() == 2);
    CHECK(!res.try_reserve(1));
    first.grow(pl, 1);
    second.grow(pl, 1);
    CHECK(pl.free_pages() == 0);
    first.release(pl);
    res.release(2);
    CHECK(res.try_reserve(2));
    SequencePages replacement;
    replacement.grow(pl, 32);
    for (uint32_t p : replacement.pages())
        for (uint32_t q : second.pages()) CHECK(p != q);
    CHECK(!res.try_reserve(1));
}

static void impossible_and_failed_reservations_do_not_leak_capacity() {
    PageReservations res(4);
    CHECK(!error_of([&] { res.try_reserve(5); }).empty());
    CHECK(!error_of([&] { res.try_reserve(0); }).empty());
    CHECK(res.try_reserve(3));
    CHECK(!res.try_reserve(2));
    res.release(3);
    CHECK(res.try_reserve(4));
    CHECK(!error_of([&] { res.release(5); }).empty());
    res.release(4);
    CHECK(res.try_reserve(4));
}

int main() {
    const std::vector<std::pair<const char*, std::function<void()>>> tests = {
        {"allocates_in_order_and_tracks_counts", allocates_in_order_and_tracks_counts},
        {"page_geometry_matches_layout", page_geometry_matches_layout},
        {"grows_lazily_one_page_at_a_time", grows_lazily_one_page_at_a_time},
        {"translation_crosses_page_boundaries", translation_crosses_page_boundaries},
        {"translation_rejects_positions_past_the_end", translation_rejects_positions_past_the_end},
        {"sequences_never_share_a_physical_page", sequences_never_share_a_physical_page},
        {"release_returns_pages_and_they_are_reused", release_returns_pages_and_they_are_reused},
        {"exhaustion_is_an_explicit_error", exhaustion_is_an_explicit_error},
        {"a_failed_grow_leaves_the_pool_untouched", a_failed_grow_leaves_the_pool_untouched},
        {"double_free_is_rejected", double_free_is_rejected},
        {"releasing_an_out_of_range_page_is_rejected", releasing_an_out_of_range_page_is_rejected},
        {"reset_then_reuse_gives_a_clean_sequence", reset_then_reuse_gives_a_clean_sequence},
        {"padded_table_is_deterministic", padded_table_is_deterministic},
        {"admission_after_reclaim_reuses_the_freed_pages",
         admission_after_reclaim_reuses_the_freed_pages},
        {"capacity_accounting_adds_up", capacity_accounting_adds_up},
        {"interleaved_free_and_realloc_stays_consistent",
         interleaved_free_and_realloc_stays_consistent},
        {"reservations_include_decode_growth_and_one_token_completion",
         reservations_include_decode_growth_and_one_token_completion},
        {"page_pressure_keeps_future_decode_pages_and_cancellation_returns_budget",
         page_pressure_keeps_future_decode_pages_and_cancellation_returns_budget},
        {"impossible_and_failed_reservations_do_not_leak_capacity",
         impossible_and_failed_reservations_do_not_leak_capacity},
    };
    int failed_tests = 0;
    for (const auto& t : tests) {
        const int before = g_failures;
        try {
            t.second();
        } catch (const std::exception& e) {
            std::fprintf(stderr, "  unexpected exception: %s\n", e.what());
            ++g_failures;
        }
        const bool ok = g_failures == before;
        failed_tests += !ok;
        std::printf("%s %s\n", ok ? "PASS" : "FAIL", t.first);
    }
    std::printf("%zu tests, %d failed\n", tests.size(), failed_tests);
    return failed_tests ? 1 : 0;
}
