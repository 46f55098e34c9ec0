// Paged decode attention for gfx950: split-K over pages, MFMA for QK^T and PV.
//
// Reference semantics (engine/kernels/kernels.cu:1741-1839, attention_decode_paged_f32):
// for request b and query head h, kv head g = h / (n_head / n_kv_head),
//   s_j = (q . k_j) / sqrt(64) for j < seq_lens[b];  out = softmax(s) . V.
// seq_lens[b] <= 0 marks an inactive request (no output is written).
//
// Work decomposition. A workgroup owns one (request b, kv head g, split s); a split
// is WAVES * PAGES consecutive logical pages. Each of the 4 waves owns PAGES pages and
// serves all n_rep query heads that share kv head g, so a K/V page is read from HBM
// once per GQA group, not once per query head. Grid size depends only on
// (batch, n_kv_head, max_seq), never on the current lengths, so the launch can be
// captured in a hipGraph; splits past a request's end exit at once.
//
// Per page and wave (16 tokens):
//   S^T[16 tok x 16 col] = K[16 tok x 64] . Q^T[64 x 16 col]   2x mfma_f32_16x16x32_f16
//     (col = query head within the group; columns >= n_rep are padding)
//   online softmax per column in base 2; cross-lane max over the 4 lane groups
//   O^T[64 dim x 16 col] += V^T[64 dim x 16 tok] . P^T[16 tok x 16 col]
//     4 dim blocks x mfma_f32_16x16x16f16, with P split into fp16 hi + lo parts so
//     the product keeps ~22 bits of P (an f32 query is split the same way for QK).
// K operands come straight from the page (row `tok`, 8 channels per lane); V operands
// come straight from the transposed V page (channel row, 4 slots per lane). No LDS is
// needed until the 4 waves of a workgroup merge their partial softmax states.
//
// The combine across splits (reference kernels.cu:806-850) uses the exact algebra
//   M = max m_s, L = sum l_s 2^(m_s - M), out = sum o_s 2^(m_s - M) / L
// and a request that fits in one split is written directly by its only workgroup.
#include "common.hpp"

#include <cmath>
#include <cstdlib>

namespace crucible {
namespace {

constexpr int kWaves = 4;

enum LenMode { kLensArray = 0, kPositionsPlusOne = 1, kParamsSeq = 2 };

struct DecodeArgs {
    const void* q;
    const half_t* k_pool;
    const half_t* v_pool;
    void* out;
    const int32_t* tables;       // nullptr: contiguous cache (page = pos >> 4)
    const int32_t* table_index;  // nullptr: row b uses table row b
    const int32_t* lens;
    float* po;                   // [batch][n_head][n_splits][64]
    float* pm;                   // [batch][n_head][n_splits]
    float* pl;                   // [batch][n_head][n_splits]
    PoolAddr addr;
    int64_t table_stride;
    int64_t q_row_stride;        // elements between query rows (n_head * 64)
    int len_mode;
    int batch;
    int n_head;
    int n_kv_head;
    int n_rep;
    int n_splits;
    int split_pages;
    int max_seq;
    int out_f16;
    float scale_log2;            // (1/sqrt(64)) * log2(e)
};

__device__ __forceinline__ int request_len(const DecodeArgs& a, int b) {
    int len;
    if (a.len_mode == kParamsSeq) len = a.lens[kParamSeq];
    else len = a.lens[b] + (a.len_mode == kPositionsPlusOne ? 1 : 0);
    return len < a.max_seq ? len : a.max_seq;  // never index past the table
}

__device__ __forceinline__ void store_out4(const DecodeArgs& a, int64_t off, float4_t v) {
    if (a.out_f16) {
        half4_t h = {(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
        *reinterpret_cast<half4_t*>(static_cast<half_t*>(a.out) + off) = h;
    } else {
        *reinterpret_cast<float4_t*>(static_cast<float*>(a.out) + off) = v;
    }
}

template <int PAGES, bool QF32>
__global__ __launch_bounds__(256) void decode_split_kernel(DecodeArgs a) {
    __shared__ float4_t s_acc[kWaves][16][17];  // [wave][col][dim/4], padded
    __shared__ float s_m[kWaves][16];
    __shared__ float s_l[kWaves][16];

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;
    const int grp = lane >> 4;

    const int unit = blockIdx.x;
    const int s = unit % a.n_splits;
    const int bg = unit / a.n_splits;
    const int g = bg % a.n_kv_head;
    const int b = bg / a.n_kv_head;

    const int len = request_len(a, b);
    if (len <= 0) return;
    const int n_pages = (len + kPageMask) >> kPageShift;
    const int p_begin = s * a.split_pages;
    if (p_begin >= n_pages) return;
    const int n_active = (n_pages + a.split_pages - 1) / a.split_pages;
    const int wp0 = p_begin + wave * PAGES;
    const int wp_end = min(wp0 + PAGES, n_pages);

    const int32_t* table = nullptr;
    if (a.tables)
        table = a.tables + (int64_t)(a.table_index ? a.table_index[b] : b) * a.table_stride;

    // Query operand: B[k = channel][col = head], 8 channels per lane per MFMA.
    const int h = g * a.n_rep + col;
    half8_t qh0 = {}, qh1 = {}, ql0 = {}, ql1 = {};
    if (col < a.n_rep) {
        const int64_t qoff = (int64_t)b * a.q_row_stride + (int64_t)h * kHeadDim + 8 * grp;
        if constexpr (QF32) {
            const float* qp = static_cast<const float*>(a.q) + qoff;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x0 = qp[j], x1 = qp[32 + j];
                qh0[j] = (half_t)x0;
                qh1[j] = (half_t)x1;
                ql0[j] = (half_t)(x0 - (float)qh0[j]);
                ql1[j] = (half_t)(x1 - (float)qh1[j]);
            }
        } else {
            const half_t* qp = static_cast<const half_t*>(a.q) + qoff;
            qh0 = *reinterpret_cast<const half8_t*>(qp);
            qh1 = *reinterpret_cast<const half8_t*>(qp + 32);
        }
    }

    // Issue every load of this wave's pages before any arithmetic.
    half8_t ka[PAGES][2];
    half4_t va[PAGES][4];
    const int kv_dim = a.addr.kv_dim;
#pragma unroll
    for (int i = 0; i < PAGES; ++i) {
        const int p = wp0 + i;
        if (p < wp_end) {
            const int64_t page = table ? (int64_t)table[p] : (int64_t)p;
            const int64_t base = block_base(a.addr, page);
            const half_t* kp = a.k_pool + base + (int64_t)col * kv_dim + g * kHeadDim + 8 * grp;
            ka[i][0] = *reinterpret_cast<const half8_t*>(kp);
            ka[i][1] = *reinterpret_cast<const half8_t*>(kp + 32);
            const half_t* vp = a.v_pool + base + (int64_t)(g * kHeadDim + col) * kPageTokens + 4 * grp;
#pragma unroll
            for (int db = 0; db < 4; ++db)
                va[i][db] = *reinterpret_cast<const half4_t*>(vp + db * 16 * kPageTokens);
        }
    }

    float m = -INFINITY;
    float l = 0.0f;
    float4_t acc[4] = {};
#pragma unroll
    for (int i = 0; i < PAGES; ++i) {
        const int p = wp0 + i;
        if (p < wp_end) {
            float4_t st = {};
            st = mfma_16x16x32(ka[i][0], qh0, st);
            st = mfma_16x16x32(ka[i][1], qh1, st);
            if constexpr (QF32) {
                st = mfma_16x16x32(ka[i][0], ql0, st);
                st = mfma_16x16x32(ka[i][1], ql1, st);
            }
            // st[r] = S^T[token 4*grp + r][col]
            const int tok0 = p * kPageTokens + 4 * grp;
            float sv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) sv[r] = (tok0 + r < len) ? st[r] * a.scale_log2 : -INFINITY;
            float tm = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
            tm = fmaxf(tm, __shfl_xor(tm, 16));
            tm = fmaxf(tm, __shfl_xor(tm, 32));
            const float mn = fmaxf(m, tm);
            const float alpha = fast_exp2(m - mn);
            float pv[4];
            float ps = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pv[r] = fast_exp2(sv[r] - mn);
                ps += pv[r];
            }
            l = l * alpha + ps;
            m = mn;
            half4_t ph, plo;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                ph[r] = (half_t)pv[r];
                plo[r] = (half_t)(pv[r] - (float)ph[r]);
            }
            const bool tail = (p == n_pages - 1) && (len & kPageMask);
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                half4_t v = va[i][db];
                if (tail) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (tok0 + r >= len) v[r] = (half_t)0.0f;  // unwritten slots may hold NaN
                }
                acc[db] = acc[db] * alpha;
                acc[db] = mfma_16x16x16(v, ph, acc[db]);
                acc[db] = mfma_16x16x16(v, plo, acc[db]);
            }
        }
    }
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);

    // Merge the 4 waves' states: acc[db][r] = O^T[16*db + 4*grp + r][col].
    if (grp == 0) {
        s_m[wave][col] = m;
        s_l[wave][col] = l;
    }
#pragma unroll
    for (int db = 0; db < 4; ++db) s_acc[wave][col][4 * db + grp] = acc[db];
    __syncthreads();

    const int t = threadIdx.x;
    const int ccol = t >> 4;  // query head within the group
    const int d4 = t & 15;    // dims 4*d4 .. 4*d4+3
    if (ccol >= a.n_rep) return;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][ccol]);
    float L = 0.0f;
    float4_t o = {};
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        if (s_l[w][ccol] > 0.0f) {
            const float wgt = fast_exp2(s_m[w][ccol] - M);
            L += s_l[w][ccol] * wgt;
            o += s_acc[w][ccol][d4] * wgt;
        }
    }
    const int hh = g * a.n_rep + ccol;
    if (n_active == 1) {
        store_out4(a, (int64_t)b * a.q_row_stride + (int64_t)hh * kHeadDim + 4 * d4, o * (1.0f / L));
    } else {
        const int64_t slot = ((int64_t)b * a.n_head + hh) * a.n_splits + s;
        *reinterpret_cast<float4_t*>(a.po + slot * kHeadDim + 4 * d4) = o;
        if (d4 == 0) {
            a.pm[slot] = M;
            a.pl[slot] = L;
        }
    }
}

// One workgroup per (request, kv head): merges the split partials of the n_rep heads.
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeArgs a) {
    const int b = blockIdx.x / a.n_kv_head;
    const int g = blockIdx.x % a.n_kv_head;
    const int len = request_len(a, b);
    if (len <= 0) return;
    const int n_pages = (len + kPageMask) >> kPageShift;
    const int n_active = (n_pages + a.split_pages - 1) / a.split_pages;
    if (n_active <= 1) return;
    const int t = threadIdx.x;
    const int ccol = t >> 4;
    const int d4 = t & 15;
    if (ccol >= a.n_rep) return;
    const int hh = g * a.n_rep + ccol;
    const int64_t slot0 = ((int64_t)b * a.n_head + hh) * a.n_splits;
    float M = -INFINITY;
    for (int s = 0; s < n_active; ++s) M = fmaxf(M, a.pm[slot0 + s]);
    float L = 0.0f;
    float4_t o = {};
    for (int s = 0; s < n_active; ++s) {
        const float wgt = fast_exp2(a.pm[slot0 + s] - M);
        L += a.pl[slot0 + s] * wgt;
        o += *reinterpret_cast<const float4_t*>(a.po + (slot0 + s) * kHeadDim + 4 * d4) * wgt;
    }
    store_out4(a, (int64_t)b * a.q_row_stride + (int64_t)hh * kHeadDim + 4 * d4, o * (1.0f / L));
}

// Pages per wave. A split (one workgroup) covers 4x this many pages. Larger splits
// mean fewer partials to merge; smaller ones mean more waves in flight.
int pages_per_wave(int64_t batch, int64_t n_kv_head, int64_t max_pages) {
    if (const char* env = std::getenv("CRUCIBLE_DECODE_PAGES")) {
        const int v = std::atoi(env);
        if (v == 1 || v == 2 || v == 4) return v;
    }
    const int64_t work = batch * n_kv_head * max_pages;
    if (work >= 16384) return 4;
    if (work >= 4096) return 2;
    return 1;
}

int launch_decode(DecodeArgs a, int pages, bool q_f32, hipStream_t stream, const char* what) {
    const int64_t units = (int64_t)a.batch * a.n_kv_head * a.n_splits;
    CRUCIBLE_CHECK(units > 0 && units <= INT32_MAX, CRUCIBLE_ERR_INVALID, "%s: grid too large",
                   what);
    const dim3 grid((unsigned)units), block(256);
#define CRUCIBLE_DECODE_CASE(P)                                                              \
    case P:                                                                                   \
        if (q_f32) hipLaunchKernelGGL((decode_split_kernel<P, true>), grid, block, 0, stream, a); \
        else hipLaunchKernelGGL((decode_split_kernel<P, false>), grid, block, 0, stream, a);  \
        break;
    switch (pages) {
        CRUCIBLE_DECODE_CASE(1)
        CRUCIBLE_DECODE_CASE(2)
        CRUCIBLE_DECODE_CASE(4)
        default:
            set_error(CRUCIBLE_ERR_INVALID, "%s: bad pages per wave %d", what, pages);
            return CRUCIBLE_ERR_INVALID;
    }
#undef CRUCIBLE_DECODE_CASE
    if (int rc = fail_launch(what)) return rc;
    if (a.n_splits > 1) {
        hipLaunchKernelGGL(decode_combine_kernel, dim3((unsigned)(a.batch * a.n_kv_head)),
                           dim3(256), 0, stream, a);
        if (int rc = fail_launch(what)) return rc;
    }
    return CRUCIBLE_OK;
}

int check_geometry(const char* what, int64_t n_head, int64_t n_kv_head, int64_t head_dim,
                   int64_t kv_dim) {
    CRUCIBLE_CHECK(n_head > 0 && n_kv_head > 0 && n_head % n_kv_head == 0, CRUCIBLE_ERR_INVALID,
                   "%s: n_head %lld must be a positive multiple of n_kv_head %lld", what,
                   (long long)n_head, (long long)n_kv_head);
    CRUCIBLE_CHECK(head_dim == kHeadDim, CRUCIBLE_ERR_UNSUPPORTED,
                   "%s: head_dim %lld unsupported (this build implements 64)", what,
                   (long long)head_dim);
    CRUCIBLE_CHECK(n_head / n_kv_head <= 16, CRUCIBLE_ERR_UNSUPPORTED,
                   "%s: more than 16 query heads per kv head", what);
    CRUCIBLE_CHECK(kv_dim == n_kv_head * head_dim, CRUCIBLE_ERR_INVALID,
                   "%s: kv_dim %lld != n_kv_head * head_dim", what, (long long)kv_dim);
    CRUCIBLE_CHECK(n_head <= (1 << 20), CRUCIBLE_ERR_INVALID, "%s: n_head too large", what);
    return CRUCIBLE_OK;
}

size_t workspace_floats(int64_t batch, int64_t n_head, int64_t n_splits) {
    return (size_t)batch * n_head * n_splits * (kHeadDim + 2);
}

void bind_workspace(DecodeArgs& a, void* ws) {
    float* f = static_cast<float*>(ws);
    const size_t n = (size_t)a.batch * a.n_head * a.n_splits;
    a.po = f;
    a.pm = f + n * kHeadDim;
    a.pl = a.pm + n;
}

}  // namespace
}  // namespace crucible

using namespace crucible;

extern "C" size_t crucible_attention_decode_workspace_bytes(int64_t batch, int64_t n_head,
                                                            int64_t max_seq) {
    if (batch <= 0 || n_head <= 0 || max_seq <= 0) return 0;
    const int64_t max_pages = (max_seq + kPageMask) >> kPageShift;
    const int64_t n_splits = (max_pages + kWaves - 1) / kWaves;  // worst case: 1 page per wave
    return workspace_floats(batch, n_head, n_splits) * sizeof(float);
}

extern "C" int crucible_attention_decode_paged(
    const void* q, int q_dtype, const void* k_pool, const void* v_pool, void* out, int out_dtype,
    const int32_t* page_tables, const int32_t* seq_lens, int64_t batch, int64_t n_head,
    int64_t n_kv_head, int64_t head_dim, int64_t table_stride, int64_t n_layer, int64_t layer,
    int64_t kv_dim, int64_t max_seq, void* workspace, size_t workspace_bytes,
    crucible_stream_t stream) {
    const char* what = "attention_decode_paged";
    CRUCIBLE_CHECK(dtype_ok(q_dtype) && dtype_ok(out_dtype), CRUCIBLE_ERR_INVALID,
                   "%s: bad dtype", what);
    if (int rc = check_geometry(what, n_head, n_kv_head, head_dim, kv_dim)) return rc;
    CRUCIBLE_CHECK(batch >= 0 && batch <= INT32_MAX, CRUCIBLE_ERR_INVALID, "%s: batch %lld",
                   what, (long long)batch);
    if (batch == 0) return CRUCIBLE_OK;
    CRUCIBLE_CHECK(q && k_pool && v_pool && out && page_tables && seq_lens, CRUCIBLE_ERR_INVALID,
                   "%s: null buffer", what);
    CRUCIBLE_CHECK(n_layer > 0 && layer >= 0 && layer < n_layer, CRUCIBLE_ERR_INVALID,
                   "%s: layer %lld outside n_layer %lld", what, (long long)layer,
                   (long long)n_layer);
    CRUCIBLE_CHECK(table_stride > 0 && max_seq > 0 && max_seq <= table_stride * kPageTokens &&
                       max_seq <= INT32_MAX,
                   CRUCIBLE_ERR_INVALID, "%s: max_seq %lld must be in 1..table_stride*16", what,
                   (long long)max_seq);
    DecodeArgs a{};
    a.q = q;
    a.k_pool = static_cast<const half_t*>(k_pool);
    a.v_pool = static_cast<const half_t*>(v_pool);
    a.out = out;
    a.tables = page_tables;
    a.lens = seq_lens;
    a.len_mode = kLensArray;
    a.addr.kv_dim = (int32_t)kv_dim;
    a.addr.page_stride = n_layer * kPageTokens * kv_dim;
    a.addr.layer_off = layer * kPageTokens * kv_dim;
    a.table_stride = table_stride;
    a.q_row_stride = n_head * kHeadDim;
    a.batch = (int)batch;
    a.n_head = (int)n_head;
    a.n_kv_head = (int)n_kv_head;
    a.n_rep = (int)(n_head / n_kv_head);
    a.max_seq = (int)max_seq;
    a.out_f16 = out_dtype == CRUCIBLE_F16;
    a.scale_log2 = 0.125f * kLog2e;
    const int64_t max_pages = (max_seq + kPageMask) >> kPageShift;
    const int pages = pages_per_wave(batch, n_kv_head, max_pages);
    a.split_pages = pages * kWaves;
    a.n_splits = (int)((max_pages + a.split_pages - 1) / a.split_pages);
    const size_t need = workspace_floats(batch, n_head, a.n_splits) * sizeof(float);
    CRUCIBLE_CHECK(a.n_splits == 1 || (workspace && workspace_bytes >= need),
                   CRUCIBLE_ERR_WORKSPACE, "%s: workspace needs %zu bytes, got %zu", what, need,
                   workspace ? workspace_bytes : (size_t)0);
    if (a.n_splits > 1) bind_workspace(a, workspace);
    return launch_decode(a, pages, q_dtype == CRUCIBLE_F32, stream, what);
}

extern "C" int crucible_attention_decode(const void* q, int q_dtype, const void* k_cache,
                                         const void* v_cache, void* out, int out_dtype,
                                         int64_t n_head, int64_t n_kv_head, int64_t head_dim,
                                         const int32_t* params, int64_t max_seq,
                                         int64_t cache_stride, int64_t layer_base,
                                         void* workspace, size_t workspace_bytes,
                                         crucible_stream_t stream) {
    const char* what = "attention_decode";
    CRUCIBLE_CHECK(dtype_ok(q_dtype) && dtype_ok(out_dtype), CRUCIBLE_ERR_INVALID,
                   "%s: bad dtype", what);
    if (int rc = check_geometry(what, n_head, n_kv_head, head_dim, cache_stride)) return rc;
    CRUCIBLE_CHECK(q && k_cache && v_cache && out && params, CRUCIBLE_ERR_INVALID,
                   "%s: null buffer", what);
    CRUCIBLE_CHECK(max_seq > 0 && max_seq <= INT32_MAX && layer_base >= 0, CRUCIBLE_ERR_INVALID,
                   "%s: max_seq %lld", what, (long long)max_seq);
    DecodeArgs a{};
    a.q = q;
    a.k_pool = static_cast<const half_t*>(k_cache);
    a.v_pool = static_cast<const half_t*>(v_cache);
    a.out = out;
    a.lens = params;
    a.len_mode = kParamsSeq;
    a.addr.kv_dim = (int32_t)cache_stride;
    a.addr.page_stride = kPageTokens * cache_stride;
    a.addr.layer_off = layer_base;
    a.q_row_stride = n_head * kHeadDim;
    a.batch = 1;
    a.n_head = (int)n_head;
    a.n_kv_head = (int)n_kv_head;
    a.n_rep = (int)(n_head / n_kv_head);
    a.max_seq = (int)max_seq;
    a.out_f16 = out_dtype == CRUCIBLE_F16;
    a.scale_log2 = 0.125f * kLog2e;
    const int64_t max_pages = (max_seq + kPageMask) >> kPageShift;
    const int pages = pages_per_wave(1, n_kv_head, max_pages);
    a.split_pages = pages * kWaves;
    a.n_splits = (int)((max_pages + a.split_pages - 1) / a.split_pages);
    const size_t need = workspace_floats(1, n_head, a.n_splits) * sizeof(float);
    CRUCIBLE_CHECK(a.n_splits == 1 || (workspace && workspace_bytes >= need),
                   CRUCIBLE_ERR_WORKSPACE, "%s: workspace needs %zu bytes, got %zu", what, need,
                   workspace ? workspace_bytes : (size_t)0);
    if (a.n_splits > 1) bind_workspace(a, workspace);
    return launch_decode(a, pages, q_dtype == CRUCIBLE_F32, stream, what);
}

extern "C" int crucible_attention_split(const void* q, int q_dtype, const void* k_cache,
                                        const void* v_cache, float* partial_o,
                                        float* partial_m, float* partial_l, void* out,
                                        int out_dtype, int64_t n_head, int64_t n_kv_head,
                                        int64_t head_dim, const int32_t* params,
                                        int64_t capacity, int64_t cache_stride,
                                        int64_t layer_base, crucible_stream_t stream) {
    const char* what = "attention_split";
    CRUCIBLE_CHECK(dtype_ok(q_dtype) && dtype_ok(out_dtype), CRUCIBLE_ERR_INVALID,
                   "%s: bad dtype", what);
    if (int rc = check_geometry(what, n_head, n_kv_head, head_dim, cache_stride)) return rc;
    CRUCIBLE_CHECK(q && k_cache && v_cache && out && params && partial_o && partial_m &&
                       partial_l,
                   CRUCIBLE_ERR_INVALID, "%s: null buffer", what);
    CRUCIBLE_CHECK(capacity > 0 && capacity <= INT32_MAX && layer_base >= 0,
                   CRUCIBLE_ERR_INVALID, "%s: capacity %lld", what, (long long)capacity);
    DecodeArgs a{};
    a.q = q;
    a.k_pool = static_cast<const half_t*>(k_cache);
    a.v_pool = static_cast<const half_t*>(v_cache);
    a.out = out;
    a.lens = params;
    a.len_mode = kParamsSeq;
    a.addr.kv_dim = (int32_t)cache_stride;
    a.addr.page_stride = kPageTokens * cache_stride;
    a.addr.layer_off = layer_base;
    a.q_row_stride = n_head * kHeadDim;
    a.batch = 1;
    a.n_head = (int)n_head;
    a.n_kv_head = (int)n_kv_head;
    a.n_rep = (int)(n_head / n_kv_head);
    a.max_seq = (int)capacity;
    a.out_f16 = out_dtype == CRUCIBLE_F16;
    a.scale_log2 = 0.125f * kLog2e;
    // 128-position chunks as in the reference (gpu.rs:37 ATTN_CHUNK): 4 waves x 2 pages.
    a.split_pages = 8;
    a.n_splits = (int)((capacity + 127) / 128);
    a.po = partial_o;
    a.pm = partial_m;
    a.pl = partial_l;
    return launch_decode(a, 2, q_dtype == CRUCIBLE_F32, stream, what);
}
