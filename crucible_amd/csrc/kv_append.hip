// KV-cache append: dense [rows][kv_dim] rows (f32 or fp16) scattered into fp16 pages.
//
// One kernel serves the four reference scatters; they differ only in where a row's
// position and page table come from (reference kernels.cu):
//   ROWS    cache_store_rows_paged_f32   (1713-1731)  positions[r], tables[r]
//   PARAMS  cache_store_paged_f32        (1646-1669)  params[5] + r, one table
//   PACKED  cache_store_packed_paged_f32 (2280-2292)  positions[r], tables[owners[r]]
//   CONTIG  cache_store_f32              (1079-1092)  pos_offset + r, no table
// A thread moves 8 channels of one row: a 32-byte f32 read, and either one 16-byte
// store (K, reference order) or eight 2-byte stores 32 bytes apart (V, transposed
// block). f32 -> fp16 is v_cvt_f16_f32 under the default round-to-nearest-even mode.
#include "common.hpp"

namespace crucible {
namespace {

enum StoreMode { kRows = 0, kParams = 1, kPacked = 2, kContig = 3 };

struct AppendArgs {
    const void* src;
    int src_f16;
    half_t* pool;
    int v_kind;
    const int32_t* tables;
    const int32_t* positions;
    const int32_t* owners;
    const int32_t* params;
    int64_t rows;
    int64_t table_stride;
    int64_t pos_offset;
    PoolAddr addr;
    int mode;
};

template <int VEC>
__global__ __launch_bounds__(256) void kv_append_kernel(AppendArgs a) {
    const int64_t per_row = a.addr.kv_dim / VEC;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.rows * per_row) return;
    const int64_t row = i / per_row;
    const int c0 = (int)(i - row * per_row) * VEC;

    int64_t pos;
    int64_t page;
    // A row whose position lies outside its table (an inactive request's -1, or a position
    // past table_stride * 16) is skipped, as the fused decode append skips it: the reference
    // kernels would index the table out of bounds there.
    switch (a.mode) {
        case kRows:
            pos = a.positions[row];
            if (pos < 0 || (pos >> kPageShift) >= a.table_stride) return;
            page = a.tables[row * a.table_stride + (pos >> kPageShift)];
            break;
        case kParams:
            pos = (int64_t)a.params[kParamPrefillPos] + row;
            if (pos < 0) return;
            page = a.tables[pos >> kPageShift];
            break;
        case kPacked:
            pos = a.positions[row];
            if (pos < 0 || (pos >> kPageShift) >= a.table_stride) return;
            page = a.tables[(int64_t)a.owners[row] * a.table_stride + (pos >> kPageShift)];
            break;
        default:
            pos = a.pos_offset + row;
            page = pos >> kPageShift;
            break;
    }
    const int slot = (int)(pos & kPageMask);
    const int64_t base = block_base(a.addr, page);
    const int64_t src_off = row * a.addr.kv_dim + c0;

    half_t h[VEC];
    if (a.src_f16) {
        const half_t* s = static_cast<const half_t*>(a.src) + src_off;
#pragma unroll
        for (int j = 0; j < VEC; ++j) h[j] = s[j];
    } else {
        const float* s = static_cast<const float*>(a.src) + src_off;
#pragma unroll
        for (int j = 0; j < VEC; ++j) h[j] = (half_t)s[j];
    }
    if (!a.v_kind) {
        half_t* d = a.pool + base + (int64_t)slot * a.addr.kv_dim + c0;
        if constexpr (VEC == 8) {
            half8_t v = {h[0], h[1], h[2], h[3], h[4], h[5], h[6], h[7]};
            *reinterpret_cast<half8_t*>(d) = v;
        } else {
#pragma unroll
            for (int j = 0; j < VEC; ++j) d[j] = h[j];
        }
    } else {
        half_t* d = a.pool + base + (int64_t)c0 * kPageTokens + slot;
#pragma unroll
        for (int j = 0; j < VEC; ++j) d[(int64_t)j * kPageTokens] = h[j];
    }
}

int launch_append(AppendArgs a, hipStream_t stream, const char* what) {
    if (a.rows == 0) return CRUCIBLE_OK;
    const bool vec = (a.addr.kv_dim % 8) == 0;
    const int64_t threads = a.rows * (vec ? a.addr.kv_dim / 8 : a.addr.kv_dim);
    const int64_t blocks = (threads + 255) / 256;
    CRUCIBLE_CHECK(blocks <= INT32_MAX, CRUCIBLE_ERR_INVALID, "%s: too many rows", what);
    if (vec)
        hipLaunchKernelGGL(kv_append_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(kv_append_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
    return fail_launch(what);
}

int check_common(const char* what, const void* src, int src_dtype, const void* pool, int kind,
                 int64_t rows, int64_t kv_dim) {
    CRUCIBLE_CHECK(dtype_ok(src_dtype), CRUCIBLE_ERR_INVALID, "%s: bad src dtype %d", what,
                   src_dtype);
    CRUCIBLE_CHECK(kind_ok(kind), CRUCIBLE_ERR_INVALID, "%s: bad pool kind %d", what, kind);
    CRUCIBLE_CHECK(rows >= 0 && rows <= INT32_MAX && kv_dim > 0 && kv_dim <= INT32_MAX,
                   CRUCIBLE_ERR_INVALID, "%s: rows=%lld kv_dim=%lld", what, (long long)rows,
                   (long long)kv_dim);
    CRUCIBLE_CHECK(rows == 0 || (src && pool), CRUCIBLE_ERR_INVALID, "%s: null buffer", what);
    return CRUCIBLE_OK;
}

AppendArgs base_args(const void* src, int src_dtype, void* pool, int kind, int64_t rows,
                     int64_t kv_dim) {
    AppendArgs a{};
    a.src = src;
    a.src_f16 = src_dtype == CRUCIBLE_F16;
    a.pool = static_cast<half_t*>(pool);
    a.v_kind = kind == CRUCIBLE_POOL_V;
    a.rows = rows;
    a.addr.kv_dim = (int32_t)kv_dim;
    return a;
}

int check_paged(const char* what, int64_t n_layer, int64_t layer, int64_t table_stride,
                bool need_stride) {
    CRUCIBLE_CHECK(n_layer > 0 && layer >= 0 && layer < n_layer, CRUCIBLE_ERR_INVALID,
                   "%s: layer %lld outside n_layer %lld", what, (long long)layer,
                   (long long)n_layer);
    CRUCIBLE_CHECK(!need_stride || (table_stride > 0 && table_stride <= INT32_MAX),
                   CRUCIBLE_ERR_INVALID, "%s: table_stride %lld outside 1..INT32_MAX", what,
                   (long long)table_stride);
    return CRUCIBLE_OK;
}

}  // namespace
}  // namespace crucible

using namespace crucible;

extern "C" int crucible_cache_store(const void* src, int src_dtype, void* cache, int kind,
                                    int64_t rows, int64_t kv_dim, int64_t layer_base,
                                    int64_t pos_offset, crucible_stream_t stream) {
    const char* what = "cache_store";
    if (int rc = check_common(what, src, src_dtype, cache, kind, rows, kv_dim)) return rc;
    CRUCIBLE_CHECK(layer_base >= 0 && pos_offset >= 0 && pos_offset <= INT32_MAX,
                   CRUCIBLE_ERR_INVALID, "%s: layer_base %lld, pos_offset %lld", what,
                   (long long)layer_base, (long long)pos_offset);
    // the last row's element index, layer_base + (pos_offset + rows) * kv_dim, fits int64
    const int64_t span = checked_mul(pos_offset + rows, kv_dim);
    CRUCIBLE_CHECK(span >= 0 && layer_base <= INT64_MAX - span, CRUCIBLE_ERR_INVALID,
                   "%s: cache offsets overflow", what);
    AppendArgs a = base_args(src, src_dtype, cache, kind, rows, kv_dim);
    a.mode = kContig;
    a.pos_offset = pos_offset;
    a.addr.page_stride = (int64_t)kPageTokens * kv_dim;
    a.addr.layer_off = layer_base;
    return launch_append(a, stream, what);
}

extern "C" int crucible_cache_store_paged(const void* src, int src_dtype, void* pool, int kind,
                                          const int32_t* page_table, int64_t rows,
                                          int64_t kv_dim, int64_t n_layer, int64_t layer,
                                          const int32_t* params, crucible_stream_t stream) {
    const char* what = "cache_store_paged";
    if (int rc = check_common(what, src, src_dtype, pool, kind, rows, kv_dim)) return rc;
    if (int rc = check_paged(what, n_layer, layer, 0, false)) return rc;
    CRUCIBLE_CHECK(rows == 0 || (page_table && params), CRUCIBLE_ERR_INVALID,
                   "%s: null table/params", what);
    AppendArgs a = base_args(src, src_dtype, pool, kind, rows, kv_dim);
    a.mode = kParams;
    a.tables = page_table;
    a.params = params;
    CRUCIBLE_CHECK(paged_addr(n_layer, layer, kv_dim, a.addr), CRUCIBLE_ERR_INVALID,
                   "%s: page geometry of %lld layers x %lld channels overflows", what,
                   (long long)n_layer, (long long)kv_dim);
    return launch_append(a, stream, what);
}

extern "C" int crucible_cache_store_rows_paged(const void* src, int src_dtype, void* pool,
                                               int kind, const int32_t* page_tables,
                                               const int32_t* positions, int64_t rows,
                                               int64_t kv_dim, int64_t table_stride,
                                               int64_t n_layer, int64_t layer,
                                               crucible_stream_t stream) {
    const char* what = "cache_store_rows_paged";
    if (int rc = check_common(what, src, src_dtype, pool, kind, rows, kv_dim)) return rc;
    if (int rc = check_paged(what, n_layer, layer, table_stride, true)) return rc;
    CRUCIBLE_CHECK(rows == 0 || (page_tables && positions), CRUCIBLE_ERR_INVALID,
                   "%s: null tables/positions", what);
    AppendArgs a = base_args(src, src_dtype, pool, kind, rows, kv_dim);
    a.mode = kRows;
    a.tables = page_tables;
    a.positions = positions;
    a.table_stride = table_stride;
    CRUCIBLE_CHECK(paged_addr(n_layer, layer, kv_dim, a.addr), CRUCIBLE_ERR_INVALID,
                   "%s: page geometry of %lld layers x %lld channels overflows", what,
                   (long long)n_layer, (long long)kv_dim);
    return launch_append(a, stream, what);
}

extern "C" int crucible_cache_store_packed_paged(const void* src, int src_dtype, void* pool,
                                                 int kind, const int32_t* tables,
                                                 const int32_t* owners,
                                                 const int32_t* positions, int64_t rows,
                                                 int64_t kv_dim, int64_t table_stride,
                                                 int64_t n_layer, int64_t layer,
                                                 crucible_stream_t stream) {
    const char* what = "cache_store_packed_paged";
    if (int rc = check_common(what, src, src_dtype, pool, kind, rows, kv_dim)) return rc;
    if (int rc = check_paged(what, n_layer, layer, table_stride, true)) return rc;
    CRUCIBLE_CHECK(rows == 0 || (tables && owners && positions), CRUCIBLE_ERR_INVALID,
                   "%s: null tables/owners/positions", what);
    AppendArgs a = base_args(src, src_dtype, pool, kind, rows, kv_dim);
    a.mode = kPacked;
    a.tables = tables;
    a.owners = owners;
    a.positions = positions;
    a.table_stride = table_stride;
    CRUCIBLE_CHECK(paged_addr(n_layer, layer, kv_dim, a.addr), CRUCIBLE_ERR_INVALID,
                   "%s: page geometry of %lld layers x %lld channels overflows", what,
                   (long long)n_layer, (long long)kv_dim);
    return launch_append(a, stream, what);
}
