// Pre-launch argument validation of every C-ABI entry point, for a build of the library's
// sources with AddressSanitizer and UBSan on the host code, linked against a HIP runtime
// with no device (tests/hip_stub.cpp; tests/test_abi_sanitized.py builds both).
//
// Every entry point is called with fake device pointers (never dereferenced: validation
// must reject the call before any launch) from a baseline of ordinary arguments, then with
// each integer argument in turn replaced by extreme values (-1, 0, 2^31, 2^40, INT64_MAX,
// INT64_MIN, ...). A call that validation lets through reaches the runtime, which has no
// device and fails the launch (CRUCIBLE_ERR_LAUNCH); no call may do anything else with the
// fake pointers. The sanitizers abort on the first report (-fno-sanitize-recover), so the
// run reaching its end is the check for overflow, out-of-bounds and lifetime errors in the
// validation code; the explicit expectations below pin the status of the cases whose
// answer the header documents.
#include <cinttypes>
#include <climits>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "crucible_attn.h"

namespace {

int g_failed = 0, g_checks = 0, g_swept = 0, g_reached_launch = 0;

void expect(const char* what, int got, int want) {
    ++g_checks;
    if (got != want) {
        char msg[256];
        crucible_attn_last_error(msg, sizeof msg);
        std::printf("FAIL %s: status %d, want %d (%s)\n", what, got, want, msg);
        ++g_failed;
    }
}

void expect_rejected(const char* what, int got) {
    ++g_checks;
    if (got == CRUCIBLE_OK || got == CRUCIBLE_ERR_LAUNCH) {
        std::printf("FAIL %s: accepted (status %d)\n", what, got);
        ++g_failed;
    }
}

void* const F = reinterpret_cast<void*>(0x1000);  // 16-byte aligned, never dereferenced
const int32_t* const FI = reinterpret_cast<const int32_t*>(0x1000);
int32_t* const FO = reinterpret_cast<int32_t*>(0x1000);
const float* const FF = reinterpret_cast<const float*>(0x1000);
float* const FW = reinterpret_cast<float*>(0x1000);

const int64_t kExtremes[] = {-1, 0, 1, 7, INT32_MAX, (int64_t)INT32_MAX + 1, (int64_t)1 << 40,
                             INT64_MAX, INT64_MIN, INT64_MAX / 64};

// An entry point over its integer arguments.
struct Entry {
    const char* name;
    std::vector<int64_t> base;
    std::function<int(const std::vector<int64_t>&)> call;
};

std::vector<Entry> entries() {
    using V = const std::vector<int64_t>&;
    std::vector<Entry> e;
    e.push_back({"cache_store", {4, 192, 0, 0}, [](V a) {
        return crucible_cache_store(F, CRUCIBLE_F32, F, CRUCIBLE_POOL_K, a[0], a[1], a[2], a[3],
                                    nullptr);
    }});
    e.push_back({"cache_store_paged", {4, 192, 12, 0}, [](V a) {
        return crucible_cache_store_paged(F, CRUCIBLE_F32, F, CRUCIBLE_POOL_V, FI, a[0], a[1],
                                          a[2], a[3], FI, nullptr);
    }});
    e.push_back({"cache_store_rows_paged", {4, 192, 64, 12, 0}, [](V a) {
        return crucible_cache_store_rows_paged(F, CRUCIBLE_F16, F, CRUCIBLE_POOL_K, FI, FI, a[0],
                                               a[1], a[2], a[3], a[4], nullptr);
    }});
    e.push_back({"cache_store_packed_paged", {4, 192, 64, 12, 0}, [](V a) {
        return crucible_cache_store_packed_paged(F, CRUCIBLE_F32, F, CRUCIBLE_POOL_V, FI, FI, FI,
                                                 a[0], a[1], a[2], a[3], a[4], nullptr);
    }});
    e.push_back({"attention_decode_paged", {16, 12, 3, 64, 128, 12, 0, 192, 2048, 1 << 24},
                 [](V a) {
        return crucible_attention_decode_paged(F, CRUCIBLE_F16, F, F, F, CRUCIBLE_F32, FI, FI,
                                               a[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7],
                                               a[8], F, (size_t)a[9], nullptr);
    }});
    e.push_back({"attention_decode_paged_append", {16, 12, 3, 64, 128, 12, 0, 192, 2048, 1 << 24},
                 [](V a) {
        return crucible_attention_decode_paged_append(
            F, CRUCIBLE_F32, F, F, CRUCIBLE_F32, F, F, F, CRUCIBLE_F32, FI, FI, FI, a[0], a[1],
            a[2], a[3], a[4], a[5], a[6], a[7], a[8], F, (size_t)a[9], nullptr);
    }});
    e.push_back({"attention_decode_paged_append_noalloc", {16, 12, 3, 64, 128, 12, 0, 192, 2048},
                 [](V a) {
        return crucible_attention_decode_paged_append_noalloc(
            F, CRUCIBLE_F16, F, F, CRUCIBLE_F16, F, F, F, CRUCIBLE_F16, FI, FI, FI, a[0], a[1],
            a[2], a[3], a[4], a[5], a[6], a[7], a[8], nullptr);
    }});
    e.push_back({"attention_decode_qkv_paged_append",
                 {1152, 2048, 16, 12, 3, 64, 128, 12, 0, 192, 2048, 1 << 24}, [](V a) {
        return crucible_attention_decode_qkv_paged_append(
            FF, a[0], FF, FF, a[1], F, F, F, CRUCIBLE_F32, FI, FI, FI, a[2], a[3], a[4], a[5],
            a[6], a[7], a[8], a[9], a[10], F, (size_t)a[11], nullptr);
    }});
    e.push_back({"attention_decode", {12, 3, 64, 2048, 192, 0, 1 << 24}, [](V a) {
        return crucible_attention_decode(F, CRUCIBLE_F32, F, F, F, CRUCIBLE_F32, a[0], a[1], a[2],
                                         FI, a[3], a[4], a[5], F, (size_t)a[6], nullptr);
    }});
    e.push_back({"attention_split", {12, 3, 64, 2048, 192, 0}, [](V a) {
        return crucible_attention_split(F, CRUCIBLE_F32, F, F, FW, FW, FW, F, CRUCIBLE_F32, a[0],
                                        a[1], a[2], FI, a[3], a[4], a[5], nullptr);
    }});
    e.push_back({"attention_prefill_paged", {512, 12, 3, 64, 12, 0, 192, 1024}, [](V a) {
        return crucible_attention_prefill_paged(F, CRUCIBLE_F32, F, F, F, CRUCIBLE_F32, FI, a[0],
                                                a[1], a[2], a[3], a[4], a[5], a[6], a[7], FI,
                                                nullptr);
    }});
    e.push_back({"attention_prefill_packed", {512, 64, 12, 3, 64, 12, 0, 192, 1024}, [](V a) {
        return crucible_attention_prefill_packed(F, CRUCIBLE_F16, F, F, F, CRUCIBLE_F32, FI, FI,
                                                 FI, a[0], a[1], a[2], a[3], a[4], a[5], a[6],
                                                 a[7], a[8], nullptr);
    }});
    e.push_back({"attention_prefill_tiled", {8, 420, 64, 16, 4, 64, 12, 0, 256, 0, 1024},
                 [](V a) {
        return crucible_attention_prefill_tiled(F, CRUCIBLE_F16, F, F, nullptr, nullptr, F,
                                                CRUCIBLE_F32, FI, FI, a[0], a[1], a[2], a[3],
                                                a[4], a[5], a[6], a[7], a[8], (int)a[9], a[10],
                                                nullptr);
    }});
    e.push_back({"attention_prefill", {512, 12, 3, 64, 1024, 192, 0, 0}, [](V a) {
        return crucible_attention_prefill(F, CRUCIBLE_F32, F, F, F, CRUCIBLE_F32, a[0], a[1],
                                          a[2], a[3], a[4], a[5], a[6], a[7], nullptr);
    }});
    e.push_back({"argmax_rows", {16, 50257}, [](V a) {
        return crucible_argmax_rows(FF, FO, a[0], a[1], nullptr);
    }});
    e.push_back({"greedy_advance", {16, 50257, 768, 768, 256}, [](V a) {
        return crucible_greedy_advance(FF, a[0], a[1], FF, a[2], FW, a[3], FO, FO,
                                       reinterpret_cast<int64_t*>(F), a[4], FO, FO,
                                       reinterpret_cast<uint32_t*>(F), nullptr);
    }});
    e.push_back({"linear_f64acc", {768, 1152, 768, 1152, 16}, [](V a) {
        return crucible_linear_f64acc(FF, a[0], FF, 1e-5f, F, a[1], a[2], nullptr, FW, a[3], a[4],
                                      nullptr);
    }});
    e.push_back({"linear_swiglu_f64acc", {768, 3072, 768, 3072, 16}, [](V a) {
        return crucible_linear_swiglu_f64acc(FF, a[0], FF, 1e-5f, F, F, a[1], a[2], FW, a[3],
                                             a[4], nullptr);
    }});
    e.push_back({"linear_f64acc_prefetch", {768, 1152, 768, 1152, 16, 1 << 20}, [](V a) {
        return crucible_linear_f64acc_prefetch(FF, a[0], FF, 1e-5f, F, a[1], a[2], nullptr, FW,
                                               a[3], a[4], F, a[5], nullptr);
    }});
    e.push_back({"linear_swiglu_f64acc_prefetch", {768, 3072, 768, 3072, 16, 1 << 20}, [](V a) {
        return crucible_linear_swiglu_f64acc_prefetch(FF, a[0], FF, 1e-5f, F, F, a[1], a[2], FW,
                                                      a[3], a[4], F, a[5], nullptr);
    }});
    e.push_back({"rmsnorm_rows", {768, 768, 16, 768}, [](V a) {
        return crucible_rmsnorm_rows(FF, a[0], FF, 1e-5f, FW, a[1], a[2], a[3], nullptr);
    }});
    e.push_back({"rope_split_qkv", {1152, 16, 12, 3, 64, 2048}, [](V a) {
        return crucible_rope_split_qkv(FF, a[0], FW, FW, FW, FF, FF, FI, a[1], a[2], a[3], a[4],
                                       a[5], nullptr);
    }});
    e.push_back({"decode_kernel_name", {16, 12, 3, 2048, 1, 16}, [](V a) {
        char buf[64];
        const size_t n = a[5] < 0 ? 0 : (a[5] > 64 ? 64 : (size_t)a[5]);
        return crucible_attention_decode_kernel_name(a[0], a[1], a[2], a[3], CRUCIBLE_F16,
                                                     (int)a[4], buf, n);
    }});
    return e;
}

void sweep() {
    for (const Entry& en : entries()) {
        const int base = en.call(en.base);
        // the baseline passes validation: the call reaches the (device-less) runtime
        if (base != CRUCIBLE_ERR_LAUNCH && base != CRUCIBLE_OK) {
            char msg[256];
            crucible_attn_last_error(msg, sizeof msg);
            std::printf("note %s baseline: status %d (%s)\n", en.name, base, msg);
        }
        for (size_t i = 0; i < en.base.size(); ++i) {
            for (int64_t v : kExtremes) {
                std::vector<int64_t> a = en.base;
                a[i] = v;
                const int rc = en.call(a);
                ++g_swept;
                if (rc == CRUCIBLE_ERR_LAUNCH) {
                    ++g_reached_launch;
                    if (v < 0 || v > INT32_MAX)
                        std::printf("accepted %s arg %zu = %" PRId64 "\n", en.name, i, v);
                }
                if (rc < CRUCIBLE_OK || rc > CRUCIBLE_ERR_LAUNCH) {
                    std::printf("FAIL %s arg %zu = %" PRId64 ": unknown status %d\n", en.name, i,
                                v, rc);
                    ++g_failed;
                }
            }
        }
    }
}

void explicit_cases() {
    // decode: head_dim outside this build, layer outside n_layer, kv_dim mismatch, GQA ratio
    expect("decode head_dim 100",
           crucible_attention_decode_paged(F, 1, F, F, F, 0, FI, FI, 1, 12, 3, 100, 64, 12, 0, 300,
                                           1024, F, 1 << 20, nullptr),
           CRUCIBLE_ERR_UNSUPPORTED);
    expect("decode layer == n_layer",
           crucible_attention_decode_paged(F, 1, F, F, F, 0, FI, FI, 1, 12, 3, 64, 64, 12, 12, 192,
                                           1024, F, 1 << 20, nullptr),
           CRUCIBLE_ERR_INVALID);
    expect("decode huge n_kv_head",
           crucible_attention_decode_paged(F, 1, F, F, F, 0, FI, FI, 1, INT64_MAX / 8,
                                           INT64_MAX / 8, 64, 64, 12, 0, 192, 1024, F, 1 << 20,
                                           nullptr),
           CRUCIBLE_ERR_INVALID);
    expect("decode workspace too small",
           crucible_attention_decode_paged(F, 1, F, F, F, 0, FI, FI, 16, 12, 3, 64, 128, 12, 0,
                                           192, 2048, F, 16, nullptr),
           CRUCIBLE_ERR_WORKSPACE);
    expect("decode empty batch",
           crucible_attention_decode_paged(nullptr, 1, nullptr, nullptr, nullptr, 0, nullptr,
                                           nullptr, 0, 12, 3, 64, 64, 12, 0, 192, 1024, nullptr,
                                           0, nullptr),
           CRUCIBLE_OK);
    expect("decode bad dtype",
           crucible_attention_decode_paged(F, 5, F, F, F, 0, FI, FI, 1, 12, 3, 64, 64, 12, 0, 192,
                                           1024, F, 1 << 20, nullptr),
           CRUCIBLE_ERR_INVALID);
    expect_rejected("decode null tables",
                    crucible_attention_decode_paged(F, 1, F, F, F, 0, nullptr, FI, 1, 12, 3, 64,
                                                    64, 12, 0, 192, 1024, F, 1 << 20, nullptr));
    expect_rejected("decode misaligned workspace",
                    crucible_attention_decode_paged(
                        F, 1, F, F, F, 0, FI, FI, 16, 12, 3, 64, 128, 12, 0, 192, 2048,
                        reinterpret_cast<void*>(0x1004), 1 << 24, nullptr));
    // the allocation-free decode's documented limit
    expect("noalloc past the scratch",
           crucible_attention_decode_paged_append_noalloc(
               F, CRUCIBLE_F16, F, F, CRUCIBLE_F32, F, F, F, CRUCIBLE_F32, FI, FI, FI, 16, 12, 3,
               64, 1313, 1, 0, 192, 20992 + 16, nullptr),
           CRUCIBLE_ERR_WORKSPACE);
    // appends: dtype, pool kind
    expect("append bad dtype",
           crucible_cache_store_rows_paged(F, 7, F, 0, FI, FI, 1, 192, 8, 12, 0, nullptr),
           CRUCIBLE_ERR_INVALID);
    expect("append bad kind",
           crucible_cache_store_rows_paged(F, 0, F, 9, FI, FI, 1, 192, 8, 12, 0, nullptr),
           CRUCIBLE_ERR_INVALID);
    // prefill: GQA ratio, hybrid without the chunk's rows
    expect("prefill n_head % n_kv_head",
           crucible_attention_prefill_paged(F, 1, F, F, F, 0, FI, 10, 12, 5, 64, 12, 0, 320, 1024,
                                            FI, nullptr),
           CRUCIBLE_ERR_INVALID);
    expect("prefill hybrid without current K/V",
           crucible_attention_prefill_tiled(F, 1, F, F, nullptr, nullptr, F, 0, FI, FI, 1, 16, 4,
                                            12, 3, 64, 12, 0, 192, 1, 256, nullptr),
           CRUCIBLE_ERR_INVALID);
    // model-step glue
    expect("linear k_in not a multiple of 32",
           crucible_linear_f64acc(FF, 100, nullptr, 1e-6f, F, 64, 100, nullptr, FW, 64, 4,
                                  nullptr),
           CRUCIBLE_ERR_UNSUPPORTED);
    expect("linear misaligned x",
           crucible_linear_f64acc(reinterpret_cast<const float*>(0x1004), 128, nullptr, 1e-6f, F,
                                  64, 128, nullptr, FW, 64, 4, nullptr),
           CRUCIBLE_ERR_INVALID);
    expect("linear prefetch not whole 64-byte lines",
           crucible_linear_f64acc_prefetch(FF, 128, nullptr, 1e-6f, F, 64, 128, nullptr, FW, 64, 4,
                                           F, 100, nullptr),
           CRUCIBLE_ERR_INVALID);
    expect("linear prefetch misaligned",
           crucible_linear_swiglu_f64acc_prefetch(FF, 128, nullptr, 1e-6f, F, F, 64, 128, FW, 64,
                                                  4, reinterpret_cast<const void*>(0x1002), 64,
                                                  nullptr),
           CRUCIBLE_ERR_INVALID);
    expect("linear prefetch bytes without a buffer",
           crucible_linear_f64acc_prefetch(FF, 128, nullptr, 1e-6f, F, 64, 128, nullptr, FW, 64, 4,
                                           nullptr, 64, nullptr),
           CRUCIBLE_ERR_INVALID);
    expect("rope odd head_dim",
           crucible_rope_split_qkv(FF, 1152, FW, FW, FW, FF, FF, FI, 16, 12, 3, 63, 1024, nullptr),
           CRUCIBLE_ERR_UNSUPPORTED);
    expect("greedy empty vocabulary",
           crucible_greedy_advance(FF, 16, 0, FF, 768, FW, 768, FO, FO,
                                   reinterpret_cast<int64_t*>(F), 8, FO, FO,
                                   reinterpret_cast<uint32_t*>(F), nullptr),
           CRUCIBLE_ERR_INVALID);
    // host-only helpers
    expect("workspace bytes of an empty batch", (int)crucible_attention_decode_workspace_bytes(
                                                    0, 12, 2048), 0);
    for (int64_t v : kExtremes)
        (void)crucible_attention_decode_workspace_bytes(v, 12, 2048),
            (void)crucible_attention_decode_workspace_bytes(16, v, 2048),
            (void)crucible_attention_decode_workspace_bytes(16, 12, v);
    char small[1];
    expect("last_error into one byte", crucible_attn_last_error(small, 1) >= 0 ? 0 : 1, 0);
    expect("last_error with n = 0", crucible_attn_last_error(small, 0) >= 0 ? 0 : 1, 0);
    ++g_checks;
    if (small[0] != '\0') {
        std::printf("FAIL last_error into one byte: not terminated\n");
        ++g_failed;
    }
    for (int key : {-1, (int)CRUCIBLE_TUNE_COUNT, INT32_MAX, INT32_MIN}) {
        expect("set_tuning bad key", crucible_attn_set_tuning(key, 1), CRUCIBLE_ERR_INVALID);
        expect("get_tuning bad key", crucible_attn_get_tuning(key), -1);
        ++g_checks;
        if (crucible_attn_tuning_name(key) != nullptr) {
            std::printf("FAIL tuning_name(%d) not null\n", key);
            ++g_failed;
        }
    }
    expect("set_tuning bad value",
           crucible_attn_set_tuning(CRUCIBLE_TUNE_DECODE_WAVES, 5), CRUCIBLE_ERR_INVALID);
    expect("set_tuning reset", crucible_attn_set_tuning(CRUCIBLE_TUNE_DECODE_WAVES, -1),
           CRUCIBLE_OK);
    // segment descriptors (host): a decreasing cu_seqlens, a non-zero start, then a good one
    {
        const int32_t bad[] = {0, 5, 3};
        int32_t seg[8];
        expect("segments decreasing", (int)crucible_segments_from_cu_seqlens(bad, 2, nullptr, seg),
               -1);
        const int32_t start[] = {1, 5};
        expect("segments non-zero start",
               (int)crucible_segments_from_cu_seqlens(start, 1, nullptr, seg), -1);
        const int32_t good[] = {0, 5, 12};
        const int32_t abs_start[] = {100, 0};
        expect("segments max chunk",
               (int)crucible_segments_from_cu_seqlens(good, 2, abs_start, seg), 7);
        expect("segments second descriptor", seg[4] == 5 && seg[5] == 7 && seg[6] == 0 &&
                                                     seg[7] == 1 && seg[2] == 100
                                                 ? 0
                                                 : 1,
               0);
        expect("segments null output",
               (int)crucible_segments_from_cu_seqlens(good, 2, nullptr, nullptr), -1);
    }
    // paging C API at its edges
    {
        // pool sizes: small ones, and ones past the 2^31 pages int32 tables can address
        // (INT32_MAX itself is a valid, 8 GiB free list, and not built here)
        for (int64_t v : {(int64_t)-1, (int64_t)0, (int64_t)1, (int64_t)7,
                          (int64_t)INT32_MAX + 2, (int64_t)1 << 40, INT64_MAX, INT64_MIN}) {
            crucible_page_pool* p = crucible_page_pool_new(v, 12, 192);
            expect("pool size accepted iff in range", p != nullptr, v >= 0 && v <= 7);
            if (p) crucible_page_pool_free(p);
        }
        for (int64_t v : kExtremes) {
            crucible_page_pool* p = crucible_page_pool_new(4, v, 192);
            if (p) crucible_page_pool_free(p);
            p = crucible_page_pool_new(4, 12, v);
            if (p) crucible_page_pool_free(p);
            (void)crucible_request_page_reservation(v, 16, 1024);
            (void)crucible_request_page_reservation(16, v, 1024);
            (void)crucible_request_page_reservation(16, 16, v);
        }
        crucible_page_pool* p = crucible_page_pool_new(4, 12, 192);
        crucible_seq_pages* s = crucible_seq_pages_new();
        for (int64_t v : kExtremes) {
            int64_t page = 0, slot = 0;
            (void)crucible_seq_pages_translate(s, v, &page, &slot);
            (void)crucible_page_pool_release(p, v);
        }
        expect_rejected("grow past the pool", crucible_seq_pages_grow(s, p, 16 * 5));
        expect_rejected("grow by INT64_MAX", crucible_seq_pages_grow(s, p, INT64_MAX));
        expect("reservation overflow", (int)crucible_request_page_reservation(INT64_MAX, 2, INT64_MAX),
               -1);
        expect("reservation", (int)crucible_request_page_reservation(20, 5, 1024), 2);
        expect("grow into the pool", crucible_seq_pages_grow(s, p, 16 * 2 + 3), CRUCIBLE_OK);
        int32_t row[3] = {-7, -7, -7};
        expect_rejected("padded table too narrow", crucible_seq_pages_table_padded(s, 2, row));
        expect("padded table", crucible_seq_pages_table_padded(s, 3, row), CRUCIBLE_OK);
        expect("release", crucible_seq_pages_release(s, p), CRUCIBLE_OK);
        crucible_seq_pages_free(s);
        crucible_page_pool_free(p);
    }
}

}  // namespace

int main() {
    std::setvbuf(stdout, nullptr, _IOLBF, 0);
    std::printf("%s\n", crucible_attn_version());
    explicit_cases();
    sweep();
    std::printf("%d checks, %d failed; %d extreme-value calls swept, %d passed validation\n",
                g_checks, g_failed, g_swept, g_reached_launch);
    return g_failed ? 1 : 0;
}
