// Paged decode attention for gfx950: split-K over pages, MFMA for QK^T and PV, and the
// cross-split combine fused into the same launch.
//
// Reference semantics (engine/kernels/kernels.cu:1741-1839, attention_decode_paged_f32):
// for request b and query head h, kv head g = h / (n_head / n_kv_head),
//   s_j = (q . k_j) / sqrt(64) for j < seq_lens[b];  out = softmax(s) . V.
// seq_lens[b] <= 0 marks an inactive request (no output is written).
//
// Work decomposition. A workgroup owns one (request b, kv head g, split s); a split is
// WAVES * PAGES consecutive logical pages. Each wave owns PAGES pages and serves all
// n_rep query heads that share kv head g, so a K/V page is read from HBM once per GQA
// group, not once per query head. Grid size depends only on (batch, n_kv_head, max_seq),
// never on the current lengths, so the launch can be captured in a hipGraph; splits past
// a request's end exit at once.
//
// Latency chain. The request length and the page ids of the wave's pages are loaded
// together (page ids below the table capacity are always in bounds), so one dependent
// round trip precedes the K/V loads, and every K/V load of the wave is in flight before
// any arithmetic.
//
// Per page and wave (16 tokens):
//   S^T[16 tok x 16 col] = K[16 tok x 64] . Q^T[64 x 16 col]   2x mfma_f32_16x16x32_f16
//     (col = query head within the group; columns >= n_rep are padding)
//   online softmax per column in base 2; cross-lane max over the 4 lane groups
//   O^T[64 dim x 16 col] += V^T[64 dim x 16 tok] . P^T[16 tok x 16 col]
//     4 dim blocks x mfma_f32_16x16x16f16, with P split into fp16 hi + lo parts so
//     the product keeps ~22 bits of P (an f32 query is split the same way for QK).
// K operands come straight from the page (row `tok`, 8 channels per lane); V operands
// come straight from the transposed V page (channel row, 4 slots per lane). LDS is only
// used to merge the waves' softmax states.
//
// Combine across splits (reference kernels.cu:806-850), exact algebra in base 2:
//   M = max m_s, L = sum l_s 2^(m_s - M), out = sum o_s 2^(m_s - M) / L.
// A request that fits in one split is written directly by its only workgroup. Otherwise
// every split writes its partial (o, m, l) with agent-coherent stores, waits for them to
// complete, and bumps a per-(request, kv head) counter; the workgroup that brings the counter to the number of active splits
// resets it to zero and performs the combine. Counters therefore read zero between
// launches: the workspace must be zeroed once when it is allocated, and one workspace
// serves one launch at a time (calls of any batch size may share it: the counters sit
// at a fixed place at its start).
#include "common.hpp"
#include "generic_attend.hpp"

#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace crucible {
namespace {

struct DecodeArgs {
    // The first 64 bytes hold what the prologue's unit check and first page loads need
    // besides the preloaded arguments (one scalar fetch).
    half_t* k_pool;              // written only by the fused append
    half_t* v_pool;
    PoolAddr addr;
    int32_t table_stride;
    int max_pages;               // ceil(max_seq / 16) <= table_stride
    int split_shift;             // a split covers 1 << split_shift pages
    int max_seq;
    int n_kv_head;
    int n_rep;
    // the rest
    const void* q;
    void* out;
    const void* k_new;           // fused append: [batch][kv_dim] rows (f32 or fp16)
    const void* v_new;
    float* po;                   // [batch][n_head][n_splits][64]
    float* pm;                   // [batch][n_head][n_splits]
    float* pl;                   // [batch][n_head][n_splits]
    uint32_t* counters;          // [batch * n_kv_head] x counter_stride; nullptr: combine in a second kernel
    int counter_stride;          // u32 between two units' counters (kCounterPad where they fit)
    int32_t q_row_stride;        // elements between query rows (n_head * 64)
    uint32_t po_bytes;           // size of po (buffer-resource bound)
    int kv_new_f16;
    int n_head;
    int n_splits;
    int out_f16;
    float scale_log2;            // (1/sqrt(64)) * log2(e)
    // fused RoPE (the qkv entry point): rotate q and the appended K row at positions[b]
    const float* rope_cos;       // [rope_max_pos][32]
    const float* rope_sin;
    int rope_max_pos;
    int kv_new_stride;           // elements between k_new (and v_new) rows
    int out_row_stride;          // elements between output rows (n_head * 64)
    // Passed to decode_kernel again as its leading (preloaded) arguments, which the kernel
    // copies over these: kept last, so that no scalar fetch of the fields above carries them.
    int lens_stride;             // 1: per-request lengths; 0: one length in params
    int lens_off;                // 0, or CRUCIBLE_PARAM_SEQ for a params buffer
    int batch;
    const int32_t* tables;       // nullptr: contiguous cache (page = pos >> 4)
    const int32_t* lens;         // request b's length is lens[b * lens_stride + lens_off]
    const int32_t* positions;    // fused append: row b goes to position positions[b]
    int32_t* plan;               // compact order's unit plan (kPlanUnits entries); nullptr: none
};


#ifdef CRUCIBLE_STAMPS
// Phase stamps, compiled only into the diagnostic libcrucible_attn_stamps.so (built from
// this file with -DCRUCIBLE_STAMPS; the product library has none of this). Thread 0 of each
// workgroup of decode_kernel records s_memrealtime (the chip-wide constant-rate clock)
// when it reaches the end of a phase, in row `workgroup id` of g_decode_stamps; the last
// slot holds what the workgroup served. stamp_after first waits for every memory
// operation its wave has in flight, so the phase's loads or stores are complete; that wait
// also holds back loads the product overlaps with the phase, so a stamped launch runs a
// little longer than the product's.
constexpr int kStampRows = 8192;
enum StampSlot {
    kStampStart,      // kernel entry
    kStampUnit,       // the workgroup's unit known (plan entry and lengths in, or searched)
    kStampPrologue,   // page ids in, the wave's K/V loads issued
    kStampLoads,      // wave 0's K/V pages resident
    kStampCompute,    // wave 0's QK, softmax and PV products issued
    kStampMerged,     // every wave past the LDS merge barrier
    kStampPublished,  // split partial acknowledged (or, for one split, the output stored)
    kStampCounted,    // split counter returned
    kStampCombined,   // the combining workgroup's output stored
    kStampMeta,       // b | g << 16 | s << 24 | n_active << 32 | last << 48 | kind << 52
    kStampSlots
};
__device__ uint64_t g_decode_stamps[kStampRows][kStampSlots];

__device__ __forceinline__ unsigned stamp_row() {
    return blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
}

__device__ __forceinline__ void stamp_store(int slot, uint64_t t) {
    if (threadIdx.x == 0 && stamp_row() < kStampRows) g_decode_stamps[stamp_row()][slot] = t;
}

__device__ __forceinline__ void stamp_now(int slot) {
    asm volatile("" ::: "memory");
    stamp_store(slot, __builtin_amdgcn_s_memrealtime());
}

__device__ __forceinline__ void stamp_after(int slot) {
    // only thread 0's wave stores stamps; the other waves do not wait
    if (threadIdx.x < 64) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    stamp_now(slot);
}

__device__ __forceinline__ void stamp_meta(int b, int g, int s, int n_active, int last, int kind) {
    if (threadIdx.x == 0 && stamp_row() < kStampRows)
        g_decode_stamps[stamp_row()][kStampMeta] =
            (uint64_t)(b & 0xffff) | (uint64_t)(g & 0xff) << 16 | (uint64_t)(s & 0xff) << 24 |
            (uint64_t)(n_active & 0xffff) << 32 | (uint64_t)(last & 1) << 48 |
            (uint64_t)(kind & 0xf) << 52;
}
// The entry time is taken into a scalar at entry and stored with the next stamp (a
// divergent store at the kernel's first instruction upsets the preloaded arguments).
#define CRUCIBLE_STAMP_TAKE(var) const uint64_t var = __builtin_amdgcn_s_memrealtime()
#define CRUCIBLE_STAMP_STORE(slot, var) stamp_store(slot, var)
#define CRUCIBLE_STAMP_NOW(slot) stamp_now(slot)
#define CRUCIBLE_STAMP_AFTER(slot) stamp_after(slot)
#define CRUCIBLE_STAMP_META(...) stamp_meta(__VA_ARGS__)
#else
#define CRUCIBLE_STAMP_TAKE(var) ((void)0)
#define CRUCIBLE_STAMP_STORE(slot, var) ((void)0)
#define CRUCIBLE_STAMP_NOW(slot) ((void)0)
#define CRUCIBLE_STAMP_AFTER(slot) ((void)0)
#define CRUCIBLE_STAMP_META(...) ((void)0)
#endif

__device__ __forceinline__ int request_len(const DecodeArgs& a, int b) {
    const int len = a.lens[b * a.lens_stride + a.lens_off];
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

// Partials cross workgroups on different XCDs, each with its own L2. They are written and
// read as agent-scope atomics (write-through stores and L2-coherent loads), so no L2
// writeback or invalidate is needed around the counter that orders them.
__device__ __forceinline__ void store_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float load_coherent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Merge the partials of splits [0, n_active) for query head hh, dims 4*d4 .. 4*d4+3.
// Loads are issued CW splits at a time so the merge costs n_active / CW round trips. CW is
// 16 for launches with more than 8 splits (batch 1 at ctx 1024: 16 splits, one round trip
// instead of two) and 8 otherwise: the wider form's registers slow the common case.
template <int CW>
__device__ __forceinline__ void combine_partials(const DecodeArgs& a, int b, int hh, int d4,
                                                 int n_active) {
    const int64_t slot0 = ((int64_t)b * a.n_head + hh) * a.n_splits;
    const __amdgpu_buffer_rsrc_t po_rsrc = make_rsrc(a.po, a.po_bytes);
    float M = -INFINITY;
    float L = 0.0f;
    float4_t o = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < n_active; s0 += CW) {
        float mv[CW], lv[CW];
        float4_t ov[CW];
#pragma unroll
        for (int j = 0; j < CW; ++j) {
            if (s0 + j < n_active) {
                const int64_t slot = slot0 + s0 + j;
                mv[j] = load_coherent(a.pm + slot);
                lv[j] = load_coherent(a.pl + slot);
                ov[j] = __builtin_bit_cast(
                    float4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                  po_rsrc, (uint32_t)(slot * kHeadDim + 4 * d4) * 4u, 0,
                                  kPolicyCoherent));
            } else {
                mv[j] = -INFINITY;
                lv[j] = 0.0f;
                ov[j] = float4_t{0.f, 0.f, 0.f, 0.f};
            }
        }
        float mx = M;
#pragma unroll
        for (int j = 0; j < CW; ++j) mx = fmaxf(mx, mv[j]);
        const float sc = fast_exp2(M - mx);  // M = -inf on the first pass: sc = 0, L = o = 0
        L *= sc;
        o = o * sc;
#pragma unroll
        for (int j = 0; j < CW; ++j) {
            if (lv[j] > 0.0f) {
                const float w = fast_exp2(mv[j] - mx);
                L += lv[j] * w;
                o += ov[j] * w;
            }
        }
        M = mx;
    }
    store_out4(a, (int64_t)b * a.out_row_stride + (int64_t)hh * kHeadDim + 4 * d4, o * (1.0f / L));
}

// RoPE of one (i, i + 32) pair (ops.rs:124-135): lo*c - hi*s, lo*s + hi*c, each product
// and difference rounded on its own as in the reference (no contraction).
__device__ __forceinline__ void rope_pair(float& lo, float& hi, float c, float s) {
#pragma clang fp contract(off)
    const float a = lo * c - hi * s;
    const float b = lo * s + hi * c;
    lo = a;
    hi = b;
}

// cos / sin of channels 8*grp .. 8*grp+7 at position pos: the pairs this lane's query and
// K operand slots hold (channel d and d + 32 sit in one lane).
struct RopeCS {
    float c[8], s[8];
};

__device__ __forceinline__ RopeCS load_rope(const DecodeArgs& a, int pos, int grp) {
    RopeCS r;
    const int p = min(max(pos, 0), a.rope_max_pos - 1);
    const float4_t* cp = reinterpret_cast<const float4_t*>(a.rope_cos + (int64_t)p * 32 + 8 * grp);
    const float4_t* sp = reinterpret_cast<const float4_t*>(a.rope_sin + (int64_t)p * 32 + 8 * grp);
    const float4_t c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        r.c[j] = c0[j];
        r.c[4 + j] = c1[j];
        r.s[j] = s0[j];
        r.s[4 + j] = s1[j];
    }
    return r;
}

// New K/V values of the appended row for this lane's operand slots, rounded to fp16
// (RNE, the conversion the standalone append kernel uses). K: lanes of column `slot`
// take channels 8*grp..+7 and 32+8*grp..+7 of kv head g; V: lanes of group slot >> 2
// take channels 16*db + col.
struct NewRow {
    half8_t k0, k1;
    half_t v[4];
};

// The appended row as loaded. Every lane loads its K channels 8*grp..+7 and 32+8*grp..+7
// and its V channels 16*db + col (db < 4) of kv head g, whatever its column, and the f32 and
// fp16 forms use the same instructions at dtype-dependent byte offsets: four 16-byte loads
// (fp16 rows load their two 16-byte pieces twice) and four 4-byte loads (for fp16, the
// aligned word that holds the value). No branch, no lane mask, no zero-filled register, so
// the loads issue ahead of the page loads without a wait; with a branch on the dtype the
// compiler converted the values inside it and waited for them before the page loads.
struct RawRow {
    u32x4_t k[4];
    uint32_t v[4];
};

__device__ __forceinline__ RawRow load_row_raw(const DecodeArgs& a, int b, int g, int col,
                                               int grp) {
    RawRow r;
    const int elt = a.kv_new_f16 ? 2 : 4;
    const char* k = static_cast<const char*>(a.k_new) + ((int64_t)b * a.kv_new_stride + g * kHeadDim) * elt;
    const char* v = static_cast<const char*>(a.v_new) + ((int64_t)b * a.kv_new_stride + g * kHeadDim) * elt;
    // f32: channels 8grp..+3, 8grp+4..+7, 32+8grp..+3, 32+8grp+4..+7; fp16: 8grp..+7, 32+8grp..+7
    const int k0 = 8 * grp * elt;
    const int k2 = (32 + 8 * grp) * elt;
    const int k1 = a.kv_new_f16 ? k0 : k0 + 16;
    const int k3 = a.kv_new_f16 ? k2 : k2 + 16;
    r.k[0] = *reinterpret_cast<const u32x4_t*>(k + k0);
    r.k[1] = *reinterpret_cast<const u32x4_t*>(k + k1);
    r.k[2] = *reinterpret_cast<const u32x4_t*>(k + k2);
    r.k[3] = *reinterpret_cast<const u32x4_t*>(k + k3);
#pragma unroll
    for (int db = 0; db < 4; ++db)
        r.v[db] = *reinterpret_cast<const uint32_t*>(v + (((16 * db + col) * elt) & ~3));
    return r;
}

// Rotate (ROPE, f32 rows) and round the loaded row to fp16.
template <bool ROPE>
__device__ __forceinline__ NewRow finish_row(const DecodeArgs& a, const RawRow& raw, int col,
                                             const RopeCS& rc) {
    NewRow r;
    if (a.kv_new_f16) {
        r.k0 = __builtin_bit_cast(half8_t, raw.k[0]);
        r.k1 = __builtin_bit_cast(half8_t, raw.k[2]);
#pragma unroll
        for (int db = 0; db < 4; ++db)
            r.v[db] = __builtin_bit_cast(half_t, (uint16_t)(raw.v[db] >> ((col & 1) * 16)));
    } else {
        float4_t k4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) k4[i] = __builtin_bit_cast(float4_t, raw.k[i]);
        if constexpr (ROPE) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float lo0 = k4[0][j], hi0 = k4[2][j], lo1 = k4[1][j], hi1 = k4[3][j];
                rope_pair(lo0, hi0, rc.c[j], rc.s[j]);
                rope_pair(lo1, hi1, rc.c[4 + j], rc.s[4 + j]);
                k4[0][j] = lo0;
                k4[2][j] = hi0;
                k4[1][j] = lo1;
                k4[3][j] = hi1;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            r.k0[j] = (half_t)k4[0][j];
            r.k0[4 + j] = (half_t)k4[1][j];
            r.k1[j] = (half_t)k4[2][j];
            r.k1[4 + j] = (half_t)k4[3][j];
            r.v[j] = (half_t)__builtin_bit_cast(float, raw.v[j]);
        }
    }
    return r;
}

// Store the appended row's kv-head-g slice into its page: the bytes
// cache_store_rows_paged writes for that slice.
__device__ __forceinline__ void store_new_row(const DecodeArgs& a, const NewRow& r, int64_t base,
                                              int g, int col, int grp, int slot) {
    if (col == slot) {
        half_t* kp = a.k_pool + base + (int64_t)slot * a.addr.kv_dim + g * kHeadDim + 8 * grp;
        *reinterpret_cast<half8_t*>(kp) = r.k0;
        *reinterpret_cast<half8_t*>(kp + 32) = r.k1;
    }
    if (grp == (slot >> 2)) {
        half_t* vp = a.v_pool + base + (int64_t)(g * kHeadDim + col) * kPageTokens + slot;
#pragma unroll
        for (int db = 0; db < 4; ++db) vp[db * 16 * kPageTokens] = r.v[db];
    }
}

// Max of a lane's 8 scores (v_max3 chains; fmaxf would add a canonicalising v_max per
// operand). The inputs are VALU results, which the hardware interlocks.
__device__ __forceinline__ float max8(const float (&v)[8]) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3\n\t"
        "v_max3_f32 %0, %0, %4, %5\n\t"
        "v_max3_f32 %0, %0, %6, %7\n\t"
        "v_max_f32 %0, %0, %8"
        : "=&v"(r)
        : "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]), "v"(v[6]),
          "v"(v[7]));
    return r;
}

constexpr int kOrderSplit = 0;
constexpr int kOrderRequest = 1;
constexpr int kOrderCompact = 2;
constexpr int kCompactPerLane = 4;    // requests per lane in the compact order's search
constexpr int kCompactMaxBatch = 64 * kCompactPerLane;

// The compact order's search: the unit workgroup blockIdx.x serves. Units are split k <
// n_active of every (request, kv head) that attends, plus one append-only unit where the
// appended row lies in a split past the attended ones, numbered in (k, request, kv head)
// order. Lane L holds requests L + 64 q, q < NQ (batch <= 64 NQ): their lengths and
// positions come in one round of vector loads. Returns false (uniformly) when the id is
// past the last unit.
struct CompactUnit {
    int k, g, lane, set, len, pos, n_active, split_append;
};

// Lane L's requests L + 64 q: raw lengths (0 past the batch) and append positions (-1).
template <int NQ, bool APPEND>
__device__ __forceinline__ void compact_load(const DecodeArgs& a, int lane, int (&lv)[NQ],
                                             int (&pv)[NQ]) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int rq = lane + 64 * q;
        lv[q] = 0;
        pv[q] = -1;
        if (rq < a.batch) {
            lv[q] = a.lens[rq * a.lens_stride + a.lens_off];
            if constexpr (APPEND) pv[q] = a.positions[rq];
        }
    }
}

template <int NQ, bool APPEND>
__device__ __forceinline__ bool compact_search(const DecodeArgs& a, int lane, const int (&lv)[NQ],
                                               const int (&pvl)[NQ], CompactUnit& u) {
    int lc[NQ], na[NQ], sap[NQ], un[NQ], pv[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        pv[q] = pvl[q];
        lc[q] = lv[q] < a.max_seq ? lv[q] : a.max_seq;  // never index past the table
        const int np = lc[q] > 0 ? (lc[q] + kPageMask) >> kPageShift : 0;
        na[q] = (np + (1 << a.split_shift) - 1) >> a.split_shift;
        sap[q] = (APPEND && pv[q] >= 0 && pv[q] < (a.max_pages << kPageShift))
                     ? pv[q] >> (kPageShift + a.split_shift) : -1;
        un[q] = na[q] + (sap[q] >= na[q] ? 1 : 0);
    }
    int k = 0, base = 0;
    uint64_t mask[NQ];
    for (;;) {  // at most n_splits + 1 rounds: a request has at most n_splits units
        int cnt = 0;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            mask[q] = __ballot(un[q] > k);
            cnt += __popcll(mask[q]);
        }
        cnt *= a.n_kv_head;
        if (cnt == 0 || k > a.n_splits) return false;
        if ((int)blockIdx.x < base + cnt) break;
        base += cnt;
        ++k;
    }
    const int j = (int)blockIdx.x - base;
    int r = j / a.n_kv_head;  // rank of the request among those with a unit k
    u.k = k;
    u.g = j - r * a.n_kv_head;
    // the r-th set bit over the masks in request order: mask q covers requests 64 q ..
    int qs = 0;
#pragma unroll
    for (int q = 0; q < NQ - 1; ++q) {
        const int c = __popcll(mask[q]);
        if (qs == q && r >= c) {
            r -= c;
            qs = q + 1;
        }
    }
    uint64_t mq = mask[0];
    int lcq = lc[0], pvq = pv[0], naq = na[0], sapq = sap[0];
#pragma unroll
    for (int q = 1; q < NQ; ++q)
        if (qs == q) {
            mq = mask[q];
            lcq = lc[q];
            pvq = pv[q];
            naq = na[q];
            sapq = sap[q];
        }
    const uint32_t rank = __builtin_amdgcn_mbcnt_hi(
        (uint32_t)(mq >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mq, 0u));
    const int bl = __builtin_ctzll(__ballot(((mq >> lane) & 1) && (int)rank == r));
    u.lane = bl;
    u.set = qs;
    u.len = __builtin_amdgcn_readlane(lcq, bl);
    u.pos = __builtin_amdgcn_readlane(pvq, bl);
    u.n_active = __builtin_amdgcn_readlane(naq, bl);
    u.split_append = __builtin_amdgcn_readlane(sapq, bl);
    return true;
}

template <int NQ, bool APPEND>
__device__ __forceinline__ bool compact_find(const DecodeArgs& a, int lane, CompactUnit& u) {
    int lv[NQ], pv[NQ];
    compact_load<NQ, APPEND>(a, lane, lv, pv);
    return compact_search<NQ, APPEND>(a, lane, lv, pv, u);
}

// The unit plan of the compact order. Every launch of a decode step sees the same lengths,
// positions and tables, and so the same units; the search above costs a round trip for the
// lengths before the one for the page ids. Entry i of the plan (in the workspace) records
// what workgroup i found: its unit, the page ids of every wave and the lengths and
// positions it was computed from. A later launch loads its entry in the same round trip as
// the lengths and, if the recorded lengths, positions and geometry equal the current ones,
// takes the unit and page ids from it; it still loads the page ids from the table beside
// the K/V loads and reissues those loads if any id changed, so a table rewritten between
// launches is always honoured. Otherwise it searches and rewrites its entry. Entry i is
// read and written only by workgroup i of a launch (read before it is written), and a
// launch sees the previous launch's entries (ordered on the stream); the entry is read
// through the scalar cache, which is never asked for it again in the same launch.
// The recorded page ids are loaded from before they are checked, so an entry is taken only
// for the same table and the same two pools (their addresses are part of the geometry): the
// ids were read from that table, and a table holds page ids of the pools it is used with.
// (Only a pool freed and allocated again smaller at the same address, with a table at its
// old address, escapes the check; the header says so.)
// Layout (int32): [0] id + 1 (0: never written), [1..11] geometry, [12] kind << 31 | split
// << 7 | request (kind 0: past the last unit, 1: a unit), [13..15] kv head, length,
// position; [32..63] page ids, PAGES per wave; [64..127] raw lengths; [128..191] positions
// (batch <= 64). The unit and geometry fit in the entry's first 64 bytes, one scalar line.
constexpr int kPlanUnits = 2048;
constexpr int kPlanEntryInts = 192;
constexpr int kPlanIds = 32;
constexpr int kPlanLens = 64;
constexpr int kPlanPos = 128;
constexpr size_t kPlanBytes = (size_t)kPlanUnits * kPlanEntryInts * sizeof(int32_t);
constexpr int kPlanMaxBatch = 64;

constexpr int kPlanGeo = 11;
constexpr int kPlanKind = 1 + kPlanGeo;
constexpr int kPlanHead = 16;  // [0] id + 1, [1..11] geometry, [12] kind|s|b, [13..15] g len pos
static_assert(kPlanKind + 4 == kPlanHead, "the unit and geometry fill one 64-byte line");

// What a plan entry's unit depends on besides the lengths and positions: the launch shape
// (the kernel's append flag and pages and waves per split included), the table's address,
// so that the recorded page ids were read from this table, and the pools' addresses, so
// that they are page ids of these pools.
template <int PAGES, int WAVES, bool APPEND>
__device__ __forceinline__ void plan_geometry(const DecodeArgs& a, int (&g)[kPlanGeo]) {
    // packed exactly where the fields fit (plan_fits checks the ranges)
    g[0] = a.batch | a.split_shift << 7 | a.lens_stride << 12 | a.lens_off << 13 |
           ((APPEND ? 1 : 0) | PAGES << 1 | WAVES << 4) << 21;
    g[1] = a.n_kv_head;
    g[2] = a.max_pages;
    g[3] = a.max_seq;
    g[4] = a.table_stride;
    const uint64_t t = (uintptr_t)a.tables;  // a preloaded argument: no wait for the block
    g[5] = (int)(uint32_t)t;
    g[6] = (int)(uint32_t)(t >> 32);
    // From the argument block, which the check waits for anyway (plan_fits, g[1..4]).
    const uint64_t kp = (uintptr_t)a.k_pool, vp = (uintptr_t)a.v_pool;
    g[7] = (int)(uint32_t)kp;
    g[8] = (int)(uint32_t)(kp >> 32);
    g[9] = (int)(uint32_t)vp;
    g[10] = (int)(uint32_t)(vp >> 32);
}

// Whether plan_geometry packs this launch exactly: batch <= 64, split_shift < 32, lens
// stride 0 or 1, lens offset < 256.
__device__ __forceinline__ bool plan_fits(const DecodeArgs& a) {
    return a.batch <= kPlanMaxBatch && a.split_shift < 32 && (a.lens_stride & ~1) == 0 &&
           a.lens_off >= 0 && a.lens_off < 256;
}

// ORDER: how workgroup ids map to (split, kv head, request): kOrderSplit, grid (split,
// kv head, request); kOrderRequest, grid (kv head, request, split); kOrderCompact, a 1-D
// grid over the units that have work, found from the lengths (batch <= 256).
// ROPE (with QF32 and APPEND): rotate q and the appended K row at the append position.
// CW: splits merged per round trip by the combining workgroup (combine_partials).
template <int PAGES, int WAVES, bool QF32, bool APPEND, bool PAGED, int ORDER, bool ROPE,
          int CW = 8>
__global__ __launch_bounds__(WAVES * 64) void decode_kernel(
    const int32_t* __restrict__ tables, const int32_t* __restrict__ lens,
    const int32_t* __restrict__ positions, int batch, int lens_stride, int lens_off,
    int32_t* plan, DecodeArgs a) {
    // The leading arguments repeat what the prologue's first loads need (they are also in
    // `a`): the library is built with kernarg preloading, so they arrive in SGPRs and the
    // length / plan / page-id loads issue without waiting for the argument block.
    a.tables = tables;
    a.lens = lens;
    a.positions = positions;
    a.batch = batch;
    a.lens_stride = lens_stride;
    a.lens_off = lens_off;
    a.plan = plan;
    CRUCIBLE_STAMP_TAKE(t_start);
    static_assert(!ROPE || (QF32 && APPEND), "RoPE is fused for f32 rows with the append");
    __shared__ float4_t s_acc[WAVES][16][17];  // [wave][col][dim/4], padded
    __shared__ float s_m[WAVES][16];
    __shared__ float s_l[WAVES][16];
    __shared__ int s_last;

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;
    const int grp = lane >> 4;

    // Which (split s, kv head g, request b) this workgroup serves, its page ids, the
    // request's length and its append position.
    int s, g, b, len, pos = -1;
    int pid[PAGES] = {};  // this wave's page ids, through the scalar cache
    int u_begin, u_end;   // the unit's logical pages
    typedef const __attribute__((address_space(4))) int32_t* const_i32_ptr;
    bool planned = false;  // unit and page ids taken from the plan (compact order)
    if constexpr (ORDER == kOrderCompact) {
        // Workgroup i serves the i-th unit (compact_find), so the units take the lowest
        // workgroup ids and a launch whose units fit the CUs gets one CU per unit; the ids
        // past the last unit return at once. The page ids follow the lengths in a second
        // round trip, unless the unit plan (batch <= 64, paged pools) holds this
        // workgroup's unit for the current lengths: then one round trip loads both.
        CompactUnit u;
        bool found;
        if (a.batch <= kPlanMaxBatch) {
            int lv[1], pv[1];
            compact_load<1, APPEND>(a, lane, lv, pv);
            // only preloaded values here: the entry's loads must not wait for the argument
            // block (plan_fits reads it, at the check below)
            const bool use_plan = PAGED && a.plan != nullptr && blockIdx.x < kPlanUnits;
            int eh[kPlanHead] = {};
            int epid[PAGES] = {};
            int snap_l = 0, snap_p = -1;
            if (use_plan) {  // uniform; issued beside the length loads
                const int32_t* e = a.plan + (size_t)blockIdx.x * kPlanEntryInts;
                const const_i32_ptr es = (const_i32_ptr)e;
#pragma unroll
                for (int j = 0; j < kPlanHead; ++j) eh[j] = es[j];
#pragma unroll
                for (int i = 0; i < PAGES; ++i) epid[i] = es[kPlanIds + wave * PAGES + i];
                snap_l = e[kPlanLens + lane];
                if constexpr (APPEND) snap_p = e[kPlanPos + lane];
            }
            int geo[kPlanGeo];
            plan_geometry<PAGES, WAVES, APPEND>(a, geo);
            bool ok = use_plan && eh[0] == (int)blockIdx.x + 1 && plan_fits(a);
#pragma unroll
            for (int j = 0; j < kPlanGeo; ++j) ok = ok && eh[1 + j] == geo[j];
            const bool lane_same = lane >= a.batch || (snap_l == lv[0] && snap_p == pv[0]);
            planned = ok && __ballot(!lane_same) == 0;
            if (planned) {
                found = eh[kPlanKind] < 0;  // the kind bit is the sign bit
                b = eh[kPlanKind] & 127;
                s = (eh[kPlanKind] >> 7) & 0xffffff;
                g = eh[kPlanKind + 1];
                len = eh[kPlanKind + 2];
                if constexpr (APPEND) pos = eh[kPlanKind + 3];
#pragma unroll
                for (int i = 0; i < PAGES; ++i) pid[i] = epid[i];
            } else {
                found = compact_search<1, APPEND>(a, lane, lv, pv, u);
                if (found) {
                    g = u.g;
                    b = u.lane;
                    len = u.len;
                    if constexpr (APPEND) pos = u.pos;
                    s = u.k < u.n_active ? u.k : u.split_append;
                    if constexpr (PAGED) {
                        const const_i32_ptr row =
                            (const_i32_ptr)(a.tables + (int64_t)b * a.table_stride);
                        const int i0 = (s << a.split_shift) + wave * PAGES;
#pragma unroll
                        for (int i = 0; i < PAGES; ++i) {
                            pid[i] = row[min(i0 + i, a.max_pages - 1)];
                            asm volatile("" : "+s"(pid[i]));  // issued here, not behind a branch
                        }
                    }
                }
                if (use_plan) {
                    // Record the unit for the next launch (vector stores: this entry is
                    // read again only by a later launch).
                    int32_t* e = a.plan + (size_t)blockIdx.x * kPlanEntryInts;
                    if (wave == 0) {
                        int v = 0;
                        if (lane == 0) v = (int)blockIdx.x + 1;
#pragma unroll
                        for (int j = 0; j < kPlanGeo; ++j)
                            if (lane == 1 + j) v = geo[j];
                        if (lane == kPlanKind)
                            v = found ? (int)(0x80000000u | (uint32_t)s << 7 | (uint32_t)b) : 0;
                        if (found) {
                            if (lane == kPlanKind + 1) v = g;
                            if (lane == kPlanKind + 2) v = len;
                            if (lane == kPlanKind + 3) v = pos;
                        }
                        if (lane < kPlanHead) e[lane] = v;
                        if (lane < a.batch) {
                            e[kPlanLens + lane] = lv[0];
                            e[kPlanPos + lane] = pv[0];
                        }
                    }
                    if (found) {
                        int v = 0;
#pragma unroll
                        for (int i = 0; i < PAGES; ++i)
                            if (lane == i) v = pid[i];
                        if (lane < PAGES) e[kPlanIds + wave * PAGES + lane] = v;
                    }
                }
            }
        } else {
            found = compact_find<kCompactPerLane, APPEND>(a, lane, u);
            if (found) {
                g = u.g;
                b = u.lane + 64 * u.set;
                len = u.len;
                if constexpr (APPEND) pos = u.pos;
                s = u.k < u.n_active ? u.k : u.split_append;
                // The page ids are uniform per wave: scalar loads (the table in the
                // constant address space: nothing writes it during the launch), which do
                // not queue behind the vector loads of workgroups already streaming pages
                // on this CU.
                if constexpr (PAGED) {
                    const const_i32_ptr row =
                        (const_i32_ptr)(a.tables + (int64_t)b * a.table_stride);
                    const int i0 = (s << a.split_shift) + wave * PAGES;
#pragma unroll
                    for (int i = 0; i < PAGES; ++i) {
                        pid[i] = row[min(i0 + i, a.max_pages - 1)];
                        asm volatile("" : "+s"(pid[i]));  // issued here, not behind a branch
                    }
                }
            }
        }
        if (!found) {  // uniform: no unit for this workgroup
            CRUCIBLE_STAMP_META(0, 0, 0, 0, 0, 2);
            return;
        }
    } else {
        // Grid (kv head, request, split), request-major: every request's first splits are
        // dispatched before any later split, and the later ones (often past the request's
        // end) queue last; or (split, kv head, request). No integer division on the way to
        // the loads. The page ids, the length and the append position are independent
        // scalar loads (one round trip through the scalar cache). Table indices are
        // clamped into the table, so every address is in bounds (ids of pages past the
        // request's end are never used).
        s = ORDER == kOrderRequest ? blockIdx.z : blockIdx.x;
        g = ORDER == kOrderRequest ? blockIdx.x : blockIdx.y;
        b = ORDER == kOrderRequest ? blockIdx.y : blockIdx.z;
        const int len_raw = ((const_i32_ptr)a.lens)[b * a.lens_stride + a.lens_off];
        if constexpr (PAGED) {
            const const_i32_ptr row = (const_i32_ptr)(a.tables + (int64_t)b * a.table_stride);
            const int i0 = (s << a.split_shift) + wave * PAGES;
#pragma unroll
            for (int i = 0; i < PAGES; ++i) pid[i] = row[min(i0 + i, a.max_pages - 1)];
        }
        if constexpr (APPEND) pos = ((const_i32_ptr)a.positions)[b];
        // Pin the loads here, so that none is sunk behind a branch on the length (which
        // would make it a second, dependent round trip).
        int lr = len_raw;
        asm volatile("" : "+s"(lr));
#pragma unroll
        for (int i = 0; i < PAGES; ++i) asm volatile("" : "+s"(pid[i]));
        if constexpr (APPEND) asm volatile("" : "+s"(pos));
        len = lr < a.max_seq ? lr : a.max_seq;  // never index past the table
    }
    CRUCIBLE_STAMP_NOW(kStampUnit);
    u_begin = s << a.split_shift;
    u_end = u_begin + (1 << a.split_shift);
    const int bg = b * a.n_kv_head + g;

    // Query operand: B[k = channel][col = head], 8 channels per lane per MFMA.
    const int h = g * a.n_rep + col;
    half8_t qh0 = {}, qh1 = {}, ql0 = {}, ql1 = {};
    float qx0[8] = {}, qx1[8] = {};  // ROPE: f32 query channels d and d + 32, rotated later
    if (col < a.n_rep) {
        const int64_t qoff = (int64_t)b * a.q_row_stride + (int64_t)h * kHeadDim + 8 * grp;
        if constexpr (ROPE) {
            const float* qp = static_cast<const float*>(a.q) + qoff;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                qx0[j] = qp[j];
                qx1[j] = qp[32 + j];
            }
        } else if constexpr (QF32) {
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

    const int wp0 = u_begin + wave * PAGES;
    int64_t page[PAGES];
#pragma unroll
    for (int i = 0; i < PAGES; ++i)
        page[i] = PAGED ? (int64_t)pid[i] : (int64_t)(wp0 + i);
    int apos = -1;  // position of the row this workgroup appends, or -1
    if (APPEND && pos >= 0 && pos < (a.max_pages << kPageShift) &&
        (pos >> kPageShift) >= u_begin && (pos >> kPageShift) < u_end)
        apos = pos;
    const int n_pages = len > 0 ? (len + kPageMask) >> kPageShift : 0;
    const bool attend = u_begin < n_pages;
    if (!attend && apos < 0) {
        CRUCIBLE_STAMP_META(b, g, s, 0, 0, 3);
        return;
    }
    // index of the appended row's page among this wave's pages (wave-uniform), or -1
    const int aidx = (apos >= 0 && (apos >> kPageShift) >= wp0 && (apos >> kPageShift) < wp0 + PAGES)
                         ? (apos >> kPageShift) - wp0 : -1;
    const int aslot = apos & kPageMask;
    // RoPE of this request's position: cos/sin of the lane's channel pairs (the query and
    // the appended K row use the same ones)
    RopeCS rc{};
    if constexpr (ROPE) rc = load_rope(a, pos, grp);
    // A planned unit's page ids against the table: the table's ids, loaded now (scalar
    // loads, beside the K/V loads issued with the plan's ids); true if any differs, with
    // pid and page then holding the table's.
    auto table_changed = [&]() -> bool {
        const const_i32_ptr row = (const_i32_ptr)(a.tables + (int64_t)b * a.table_stride);
        const int i0 = (s << a.split_shift) + wave * PAGES;
        bool changed = false;
#pragma unroll
        for (int i = 0; i < PAGES; ++i) {
            const int t = row[min(i0 + i, a.max_pages - 1)];
            changed = changed || t != pid[i];
            pid[i] = t;
            page[i] = (int64_t)t;
        }
        return changed;
    };
    if (!attend) {
        // append only: the row lies past the attended length
        if (PAGED && planned) (void)table_changed();
        if (aidx >= 0) {
            const NewRow nr = finish_row<ROPE>(a, load_row_raw(a, b, g, col, grp), col, rc);
#pragma unroll
            for (int i = 0; i < PAGES; ++i)
                if (i == aidx) store_new_row(a, nr, block_base(a.addr, page[i]), g, col, grp, aslot);
        }
        CRUCIBLE_STAMP_META(b, g, s, 0, 0, 1);
        return;
    }
    const int n_active = (n_pages + (1 << a.split_shift) - 1) >> a.split_shift;
    const int wp_end = min(min(wp0 + PAGES, u_end), n_pages);

    // The appended row's loads go out first (wave-uniform branch), then every load of this
    // wave's pages, before any arithmetic: the row is needed only when the pages are in.
    RawRow raw;
    if (APPEND && aidx >= 0) raw = load_row_raw(a, b, g, col, grp);
    // Every slot loads (no branch per page): a slot past the wave's pages reads its first
    // page again, which is in bounds, and is never used. Conditional loads made the compiler
    // merge registers between the two paths, which waited for the first page's K before the
    // second page's loads went out: two round trips instead of one. A wave without pages
    // loads nothing (uniform branch).
    half8_t ka[PAGES][2];
    half4_t va[PAGES][4];
    const int kv_dim = a.addr.kv_dim;
    auto load_pages = [&]() {
#pragma unroll
        for (int i = 0; i < PAGES; ++i) {
            const int64_t base = block_base(a.addr, wp0 + i < wp_end ? page[i] : page[0]);
            const half_t* kp = a.k_pool + base + (int64_t)col * kv_dim + g * kHeadDim + 8 * grp;
            ka[i][0] = *reinterpret_cast<const half8_t*>(kp);
            ka[i][1] = *reinterpret_cast<const half8_t*>(kp + 32);
            const half_t* vp = a.v_pool + base + (int64_t)(g * kHeadDim + col) * kPageTokens + 4 * grp;
#pragma unroll
            for (int db = 0; db < 4; ++db)
                va[i][db] = *reinterpret_cast<const half4_t*>(vp + db * 16 * kPageTokens);
        }
    };
    if (wp0 < wp_end) load_pages();
    // A planned unit checks its page ids while the pages load; if the table changed since
    // the plan was made (wave-uniform), the pages load again from the table's ids.
    if (PAGED && planned && table_changed() && wp0 < wp_end) load_pages();
    CRUCIBLE_STAMP_STORE(kStampStart, t_start);
    CRUCIBLE_STAMP_NOW(kStampPrologue);
    CRUCIBLE_STAMP_AFTER(kStampLoads);
    if constexpr (ROPE) {
        // rotate the query, then split it into fp16 hi + lo as the plain f32 path does
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            rope_pair(qx0[j], qx1[j], rc.c[j], rc.s[j]);
            qh0[j] = (half_t)qx0[j];
            qh1[j] = (half_t)qx1[j];
            ql0[j] = (half_t)(qx0[j] - (float)qh0[j]);
            ql1[j] = (half_t)(qx1[j] - (float)qh1[j]);
        }
    }
    if (APPEND && aidx >= 0) {
        // The appended row replaces what the page held in this wave's operands and is
        // written to the page for later steps.
        const NewRow nr = finish_row<ROPE>(a, raw, col, rc);
#pragma unroll
        for (int i = 0; i < PAGES; ++i) {
            if (i == aidx) {
                if (wp0 + i < wp_end) {
                    if (col == aslot) {
                        ka[i][0] = nr.k0;
                        ka[i][1] = nr.k1;
                    }
                    if (grp == (aslot >> 2)) {
#pragma unroll
                        for (int db = 0; db < 4; ++db) va[i][db][aslot & 3] = nr.v[db];
                    }
                }
                store_new_row(a, nr, block_base(a.addr, page[i]), g, col, grp, aslot);
            }
        }
    }

    // V operands that must not reach the PV products as they are: slots past the wave's
    // pages (a re-read of its first page) and the keys at or past the end of the last page
    // (unwritten slots may hold NaN, and 0 * NaN would poison the product) are zeroed here,
    // once, by uniform branches.
#pragma unroll
    for (int i = 0; i < PAGES; ++i) {
        const int p = wp0 + i;
        if (p >= wp_end) {
#pragma unroll
            for (int db = 0; db < 4; ++db) va[i][db] = half4_t{0, 0, 0, 0};
        } else if (p == n_pages - 1 && (len & kPageMask)) {
            const int tok0 = p * kPageTokens + 4 * grp;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    va[i][db][r] = (tok0 + r < len) ? va[i][db][r] : (half_t)0.0f;
        }
    }

    // Pages go through the softmax and the PV product in pairs. S^T of the two pages leaves
    // lane group grp with keys 4grp..+3 of the first page and of the second; those 8 values
    // are the k range 8grp..+7 of one 32-key PV step (mfma 16x16x32), whose V^T operand is
    // the lane's two 8-byte page quarters side by side. So a pair costs one max, one rescale
    // and 4 dim blocks x (hi, lo) PV products, half the products of a page at a time. Scores
    // stay unscaled (the scale is positive), folded into the exponent's FMA.
    const float scale = a.scale_log2;
    float m = -INFINITY;  // running max of the raw scores
    float l = 0.0f;
    float4_t acc[4] = {};
#pragma unroll
    for (int i = 0; i < PAGES; i += 2) {
        const int p = wp0 + i;
        if (p < wp_end) {
            const bool two = PAGES > 1 && p + 1 < wp_end;
            float4_t s0 = {}, s1 = {};
            s0 = mfma_16x16x32(ka[i][0], qh0, s0);
            s0 = mfma_16x16x32(ka[i][1], qh1, s0);
            if constexpr (QF32) {
                s0 = mfma_16x16x32(ka[i][0], ql0, s0);
                s0 = mfma_16x16x32(ka[i][1], ql1, s0);
            }
            if constexpr (PAGES > 1) {
                s1 = mfma_16x16x32(ka[i + 1][0], qh0, s1);
                s1 = mfma_16x16x32(ka[i + 1][1], qh1, s1);
                if constexpr (QF32) {
                    s1 = mfma_16x16x32(ka[i + 1][0], ql0, s1);
                    s1 = mfma_16x16x32(ka[i + 1][1], ql1, s1);
                }
            }
            // visible keys of the pair for this lane group: s0[r] is key 4grp + r of page p,
            // s1[r] key 4grp + r of page p + 1
            const int lim = min(len, (p + (two ? 2 : 1)) * kPageTokens) - p * kPageTokens - 4 * grp;
            float sv[8];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sv[r] = (r < lim) ? s0[r] : -INFINITY;
                sv[4 + r] = (kPageTokens + r < lim) ? s1[r] : -INFINITY;
            }
            const float tm = group_max4(max8(sv));
            const float mn = fmaxf(m, tm);  // finite: the pair's first page has a visible key
            const float mu = mn * scale;
            float pv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) pv[j] = fast_exp2(__builtin_fmaf(sv[j], scale, -mu));
            const float alpha = fast_exp2(__builtin_fmaf(m, scale, -mu));  // m = -inf: 0
            l = l * alpha + (((pv[0] + pv[1]) + (pv[2] + pv[3])) + ((pv[4] + pv[5]) + (pv[6] + pv[7])));
            m = mn;
            u32x4_t hw, lw;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float q4[4] = {pv[4 * h], pv[4 * h + 1], pv[4 * h + 2], pv[4 * h + 3]};
                hw[2 * h] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(q4[0], q4[1]));
                hw[2 * h + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(q4[2], q4[3]));
                uint32_t lo01, lo23;
                split_lo4(q4, hw[2 * h], hw[2 * h + 1], lo01, lo23);
                lw[2 * h] = lo01;
                lw[2 * h + 1] = lo23;
            }
            const half8_t ph = __builtin_bit_cast(half8_t, hw);
            const half8_t pl = __builtin_bit_cast(half8_t, lw);
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const half4_t vb = PAGES > 1 ? va[i + (PAGES > 1)][db] : half4_t{0, 0, 0, 0};
                const half8_t v = __builtin_shufflevector(va[i][db], vb, 0, 1, 2, 3, 4, 5, 6, 7);
                if (i > 0) acc[db] = acc[db] * alpha;  // the first pair starts from zero
                acc[db] = mfma_16x16x32(v, ph, acc[db]);
                acc[db] = mfma_16x16x32(v, pl, acc[db]);
            }
        }
    }
    m *= scale;  // the wave merge and the partials work in log2-scaled units
    l = group_sum4(l);
    CRUCIBLE_STAMP_NOW(kStampCompute);

    // Merge the waves' states: acc[db][r] = O^T[16*db + 4*grp + r][col].
    if (grp == 0) {
        s_m[wave][col] = m;
        s_l[wave][col] = l;
    }
#pragma unroll
    for (int db = 0; db < 4; ++db) s_acc[wave][col][4 * db + grp] = acc[db];
    __syncthreads();
    CRUCIBLE_STAMP_NOW(kStampMerged);

    const int t = threadIdx.x;
    const int ccol = t >> 4;  // query head within the group
    const int d4 = t & 15;    // dims 4*d4 .. 4*d4+3
    const bool owner = ccol < a.n_rep;
    const int hh = g * a.n_rep + ccol;
    if (owner) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) M = fmaxf(M, s_m[w][ccol]);
        float L = 0.0f;
        float4_t o = {};
        // Branch-free, so all the LDS reads issue together: a wave without pages has
        // m = -inf, l = 0 and acc = 0, so its weight is 0 and it adds exact zeros (wave 0
        // holds the split's first page, so M is finite).
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float wgt = fast_exp2(s_m[w][ccol] - M);
            L += s_l[w][ccol] * wgt;
            o += s_acc[w][ccol][d4] * wgt;
        }
        if (n_active == 1) {
            store_out4(a, (int64_t)b * a.out_row_stride + (int64_t)hh * kHeadDim + 4 * d4, o * (1.0f / L));
        } else {
            const int64_t slot = ((int64_t)b * a.n_head + hh) * a.n_splits + s;
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(u32x4_t, o), make_rsrc(a.po, a.po_bytes),
                (uint32_t)(slot * kHeadDim + 4 * d4) * 4u, 0, kPolicyCoherent);
            if (d4 == 0) {
                store_coherent(a.pm + slot, M);
                store_coherent(a.pl + slot, L);
            }
            // The partial is published once these stores are acknowledged: wait for them
            // before the workgroup barrier that precedes the counter increment.
            __builtin_amdgcn_s_waitcnt(0);
        }
    }
    CRUCIBLE_STAMP_AFTER(kStampPublished);
    if (n_active == 1 || a.counters == nullptr) {  // uniform across the workgroup
        CRUCIBLE_STAMP_META(b, g, s, n_active, n_active == 1, 0);
        return;
    }

    __syncthreads();
    if (t == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&a.counters[bg * a.counter_stride], 1u,
                                                     __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        const int last = prev == (uint32_t)(n_active - 1);
        if (last)  // ready for the next launch
            __hip_atomic_store(&a.counters[bg * a.counter_stride], 0u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        s_last = last;
        CRUCIBLE_STAMP_AFTER(kStampCounted);
        CRUCIBLE_STAMP_META(b, g, s, n_active, last, 0);
    }
    __syncthreads();
    if (!s_last) return;
    if (owner) combine_partials<CW>(a, b, hh, d4, n_active);
    CRUCIBLE_STAMP_AFTER(kStampCombined);
}

// Second-pass combine for callers that own the partials without a counter
// (attention_split): one workgroup per (request, kv head).
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeArgs a) {
    const int b = blockIdx.x / a.n_kv_head;
    const int g = blockIdx.x % a.n_kv_head;
    const int len = request_len(a, b);
    if (len <= 0) return;
    const int n_pages = (len + kPageMask) >> kPageShift;
    const int n_active = (n_pages + (1 << a.split_shift) - 1) >> a.split_shift;
    if (n_active <= 1) return;
    const int ccol = threadIdx.x >> 4;
    if (ccol >= a.n_rep) return;
    combine_partials<8>(a, b, g * a.n_rep + ccol, threadIdx.x & 15, n_active);
}

// ---------------------------------------------------------------- head_dim other than 64
// One workgroup per (request, query head) through attend_generic (generic_attend.hpp).
// ROPE (the qkv entry, f32 rows): q's pairs (i, i + hd/2) are rotated at positions[b], as
// crucible_rope_split_qkv rotates them.
template <bool QF32>
__global__ __launch_bounds__(kGenericThreads) void decode_generic_kernel(DecodeArgs a, int hd) {
    __shared__ GenericLds lds;
    const int b = blockIdx.x;
    const int h = blockIdx.y;
    const int len = request_len(a, b);
    if (len <= 0) return;  // inactive request: output untouched
    const int half = hd >> 1;
    const int64_t qoff = (int64_t)b * a.q_row_stride + (int64_t)h * hd;
    if (a.rope_cos) {
        const float* qp = static_cast<const float*>(a.q) + qoff;
        const int pos = min(max(a.positions[b], 0), a.rope_max_pos - 1);
        for (int i = threadIdx.x; i < half; i += kGenericThreads) {
            float lo = qp[i], hi = qp[i + half];
            rope_pair(lo, hi, a.rope_cos[(int64_t)pos * half + i], a.rope_sin[(int64_t)pos * half + i]);
            lds.q[i] = lo;
            lds.q[i + half] = hi;
        }
    } else {
        for (int d = threadIdx.x; d < hd; d += kGenericThreads)
            lds.q[d] = QF32 ? static_cast<const float*>(a.q)[qoff + d]
                            : (float)static_cast<const half_t*>(a.q)[qoff + d];
    }
    __syncthreads();
    GenericKeys ks{};
    ks.k_pool = a.k_pool;
    ks.v_pool = a.v_pool;
    ks.addr = a.addr;
    ks.table = a.tables ? a.tables + (int64_t)b * a.table_stride : nullptr;
    ks.g = h / a.n_rep;
    ks.hd = hd;
    ks.astart = INT32_MAX;
    const int64_t ooff = (int64_t)b * a.out_row_stride + (int64_t)h * hd;
    attend_generic(lds, ks, len, a.scale_log2, [&](int d, float v) {
        if (a.out_f16)
            static_cast<half_t*>(a.out)[ooff + d] = (half_t)v;
        else
            static_cast<float*>(a.out)[ooff + d] = v;
    });
}

// The qkv entry's two appends for head_dim other than 64: row b's K (rotated at
// positions[b] when RoPE tables are given) and its V, f32 rows of stride kv_new_stride,
// rounded to fp16 and stored at positions[b] as crucible_rope_split_qkv followed by
// crucible_cache_store_rows_paged stores them (a row whose position lies outside its table
// is skipped). One thread per (row, kv head, pair).
__global__ __launch_bounds__(256) void append_rope_generic_kernel(DecodeArgs a, int hd) {
    const int half = hd >> 1;
    const int64_t per_row = (int64_t)a.n_kv_head * half;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)a.batch * per_row) return;
    const int b = (int)(i / per_row);
    const int r = (int)(i - (int64_t)b * per_row);
    const int g = r / half;
    const int e = r - g * half;
    const int pos = a.positions[b];
    if (pos < 0 || (pos >> kPageShift) >= a.table_stride) return;
    const int64_t base = block_base(a.addr, a.tables[(int64_t)b * a.table_stride + (pos >> kPageShift)]);
    const int slot = pos & kPageMask;
    const int c = g * hd + e;  // channel of the pair's first element
    const float* kr = static_cast<const float*>(a.k_new) + (int64_t)b * a.kv_new_stride;
    const float* vr = static_cast<const float*>(a.v_new) + (int64_t)b * a.kv_new_stride;
    float lo = kr[c], hi = kr[c + half];
    if (a.rope_cos) {
        const int p = min(pos, a.rope_max_pos - 1);
        rope_pair(lo, hi, a.rope_cos[(int64_t)p * half + e], a.rope_sin[(int64_t)p * half + e]);
    }
    const int kv_dim = a.addr.kv_dim;
    a.k_pool[base + (int64_t)slot * kv_dim + c] = (half_t)lo;
    a.k_pool[base + (int64_t)slot * kv_dim + c + half] = (half_t)hi;
    a.v_pool[base + (int64_t)c * kPageTokens + slot] = (half_t)vr[c];
    a.v_pool[base + (int64_t)(c + half) * kPageTokens + slot] = (half_t)vr[c + half];
}

struct DecodeShape {
    int pages;  // pages per wave
    int waves;  // waves per workgroup
};

// Pages per wave and waves per workgroup. A split covers pages * waves pages: larger
// splits mean fewer partials to merge, smaller ones more workgroups in flight.
DecodeShape decode_shape(int64_t batch, int64_t n_kv_head, int64_t max_pages) {
    // page-units = (request, kv head, page) triples the grid is sized for
    const int64_t units = batch * n_kv_head * max_pages;
    DecodeShape sh{1, 8};                 // 8-page splits: few requests, short contexts
    if (units > 2048) sh = {2, 8};        // 16-page splits (e.g. b16 x 3 kv heads x 2048)
    if (units > 8192) sh = {4, 8};        // 32-page splits, 4 pages a wave (b16 x 12 x 2048)
    if (units > 32768) sh = {4, 4};       // 16-page splits, 4 pages a wave (b64 x 12 x 2048)
    if (const int v = tuning(CRUCIBLE_TUNE_DECODE_PAGES); v > 0) sh.pages = v;
    if (const int v = tuning(CRUCIBLE_TUNE_DECODE_WAVES); v > 0) sh.waves = v;
    return sh;
}

// The combine width: 16 splits per round trip where a launch can have more than 8, unless
// CRUCIBLE_TUNE_DECODE_COMBINE_WIDTH says otherwise (the merge loops over any count).
bool wide_combine(const DecodeArgs& a) {
    const int v = tuning(CRUCIBLE_TUNE_DECODE_COMBINE_WIDTH);
    return v > 0 ? v == 16 : a.n_splits > 8;
}

// The decode kernel's arguments: the preloaded prologue values, then the block.
#define DECODE_ARGS(a) (a).tables, (a).lens, (a).positions, (a).batch, (a).lens_stride, (a).lens_off, (a).plan, (a)

template <bool QF32, bool APPEND, bool PAGED, bool ROPE = false>
bool launch_shape(const DecodeArgs& a, DecodeShape sh, int order, dim3 grid,
                  hipStream_t stream) {
    // The 16-wide combine only where a launch can have more than 8 splits.
#define CRUCIBLE_DECODE_ORDER(P, W, O)                                                         \
    if (wide_combine(a))                                                                        \
        hipLaunchKernelGGL((decode_kernel<P, W, QF32, APPEND, PAGED, O, ROPE, 16>), grid,       \
                           dim3(W * 64), 0, stream, DECODE_ARGS(a));                                         \
    else                                                                                        \
        hipLaunchKernelGGL((decode_kernel<P, W, QF32, APPEND, PAGED, O, ROPE>), grid,           \
                           dim3(W * 64), 0, stream, DECODE_ARGS(a));
#define CRUCIBLE_DECODE_CASE(P, W)                                                             \
    if (sh.pages == P && sh.waves == W) {                                                       \
        if (order == kOrderCompact) {                                                           \
            CRUCIBLE_DECODE_ORDER(P, W, kOrderCompact)                                          \
        } else if (order == kOrderRequest) {                                                    \
            CRUCIBLE_DECODE_ORDER(P, W, kOrderRequest)                                          \
        } else {                                                                                \
            hipLaunchKernelGGL((decode_kernel<P, W, QF32, APPEND, PAGED, kOrderSplit, ROPE>),   \
                               grid, dim3(W * 64), 0, stream, DECODE_ARGS(a));                               \
        }                                                                                       \
        return true;                                                                            \
    }
    CRUCIBLE_DECODE_CASE(1, 4)
    CRUCIBLE_DECODE_CASE(2, 4)
    CRUCIBLE_DECODE_CASE(4, 4)
    CRUCIBLE_DECODE_CASE(1, 8)
    CRUCIBLE_DECODE_CASE(2, 8)
    CRUCIBLE_DECODE_CASE(4, 8)
#undef CRUCIBLE_DECODE_CASE
#undef CRUCIBLE_DECODE_ORDER
    return false;
}

int launch_decode(DecodeArgs a, DecodeShape sh, bool q_f32, hipStream_t stream,
                  const char* what) {
    CRUCIBLE_CHECK(a.n_splits > 0 && a.n_kv_head <= 65535 && a.batch <= 65535,
                   CRUCIBLE_ERR_INVALID, "%s: grid (%d, %d, %d) too large", what, a.n_splits,
                   a.n_kv_head, a.batch);
    // When the grid is larger than the chip (more workgroups than CUs), the compact order:
    // the units with work take the lowest workgroup ids, so while they fit each gets a CU
    // of its own instead of sharing one with an early split of another request. It costs
    // a second round trip before the pages (lengths first, then the page ids), so a grid
    // that fits the CUs keeps the request-major order: every request's first splits are
    // dispatched first (measured faster than split-major with the default shapes).
    // CRUCIBLE_TUNE_DECODE_ORDER overrides the choice; compact needs batch <= 256 (four
    // requests per lane) and falls back to request-major past it.
    const int64_t units = (int64_t)a.n_splits * a.n_kv_head * a.batch;
    int order = (units > device_cu_count() && a.batch <= kCompactMaxBatch) ? kOrderCompact
                                                                            : kOrderRequest;
    if (const int v = tuning(CRUCIBLE_TUNE_DECODE_ORDER); v >= 0)
        order = (v == kOrderCompact && a.batch > kCompactMaxBatch) ? kOrderRequest : v;
    CRUCIBLE_CHECK(units <= 0x7fffffff, CRUCIBLE_ERR_INVALID, "%s: grid of %lld too large", what,
                   (long long)units);
    const dim3 grid = order == kOrderCompact ? dim3((unsigned)units)
                      : order == kOrderRequest
                          ? dim3((unsigned)a.n_kv_head, (unsigned)a.batch, (unsigned)a.n_splits)
                          : dim3((unsigned)a.n_splits, (unsigned)a.n_kv_head, (unsigned)a.batch);
    bool launched;
    if (a.rope_cos)  // fused RoPE: f32 qkv rows with the append
        launched = launch_shape<true, true, true, true>(a, sh, order, grid, stream);
    else if (a.positions)  // the fused append exists for paged pools only
        launched = q_f32 ? launch_shape<true, true, true>(a, sh, order, grid, stream)
                         : launch_shape<false, true, true>(a, sh, order, grid, stream);
    else if (a.tables)
        launched = q_f32 ? launch_shape<true, false, true>(a, sh, order, grid, stream)
                         : launch_shape<false, false, true>(a, sh, order, grid, stream);
    else
        launched = q_f32 ? launch_shape<true, false, false>(a, sh, order, grid, stream)
                         : launch_shape<false, false, false>(a, sh, order, grid, stream);
    CRUCIBLE_CHECK(launched, CRUCIBLE_ERR_INVALID, "%s: bad decode shape %d x %d", what,
                   sh.pages, sh.waves);
    if (int rc = fail_launch(what)) return rc;
    if (a.n_splits > 1 && a.counters == nullptr) {
        hipLaunchKernelGGL(decode_combine_kernel, dim3((unsigned)(a.batch * a.n_kv_head)),
                           dim3(256), 0, stream, a);
        if (int rc = fail_launch(what)) return rc;
    }
    return CRUCIBLE_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int check_geometry(const char* what, int64_t n_head, int64_t n_kv_head, int64_t head_dim,
                   int64_t kv_dim) {
    CRUCIBLE_CHECK(n_head > 0 && n_kv_head > 0 && n_head % n_kv_head == 0, CRUCIBLE_ERR_INVALID,
                   "%s: n_head %lld must be a positive multiple of n_kv_head %lld", what,
                   (long long)n_head, (long long)n_kv_head);
    // before any product of the head counts: n_kv_head <= n_head <= 2^20 from here on
    CRUCIBLE_CHECK(n_head <= (1 << 20), CRUCIBLE_ERR_INVALID, "%s: n_head too large", what);
    CRUCIBLE_CHECK(head_dim == kHeadDim || generic_head_dim_ok(head_dim),
                   CRUCIBLE_ERR_UNSUPPORTED,
                   "%s: head_dim %lld unsupported (a multiple of 8 up to %d)", what,
                   (long long)head_dim, kGenericMaxHeadDim);
    CRUCIBLE_CHECK(head_dim != kHeadDim || n_head / n_kv_head <= 16, CRUCIBLE_ERR_UNSUPPORTED,
                   "%s: more than 16 query heads per kv head", what);
    CRUCIBLE_CHECK(kv_dim == n_kv_head * head_dim, CRUCIBLE_ERR_INVALID,
                   "%s: kv_dim %lld != n_kv_head * head_dim", what, (long long)kv_dim);
    return CRUCIBLE_OK;
}

// Workspace: a fixed region of kMaxCounters u32 combine counters (index b * n_kv_head + g,
// the same place for every batch size, so calls of different batch sizes can share one
// workspace), then the compact order's unit plan (kPlanBytes, also at a fixed place), then
// partial o, m, l for every (request, query head, split).
constexpr int64_t kMaxCounters = 65536;
constexpr size_t kCounterBytes = kMaxCounters * sizeof(uint32_t);
// Every split of a launch increments its unit's counter with an agent-scope atomic, and
// atomics to one 64-byte line queue behind each other: 16 units' counters packed in a line
// cost config 3 about 0.35 us a launch. Where the region holds them at one per line, each
// unit's counter gets a line of its own; every launch leaves its counters zero, so calls on
// one workspace may space them differently.
constexpr int kCounterPad = 16;  // u32 per 64-byte line

int counter_stride(int64_t units, int64_t capacity) {
    return units * kCounterPad <= capacity ? kCounterPad : 1;
}

// Saturating: a size past SIZE_MAX reads as SIZE_MAX, which no workspace or scratch meets,
// so an absurd shape fails the size check instead of wrapping to a small need.
size_t partial_floats(int64_t batch, int64_t n_head, int64_t n_splits) {
    if (batch < 0 || n_head < 0 || n_splits < 0) return SIZE_MAX;
    size_t r;
    if (__builtin_mul_overflow((size_t)batch, (size_t)n_head, &r) ||
        __builtin_mul_overflow(r, (size_t)n_splits, &r) ||
        __builtin_mul_overflow(r, (size_t)(kHeadDim + 2), &r))
        return SIZE_MAX;
    return r;
}

size_t workspace_need(int64_t batch, int64_t n_head, int64_t n_splits) {
    size_t r;
    if (__builtin_mul_overflow(partial_floats(batch, n_head, n_splits), sizeof(float), &r) ||
        __builtin_add_overflow(r, kCounterBytes + kPlanBytes, &r))
        return SIZE_MAX;
    return r;
}

void bind_workspace(DecodeArgs& a, void* ws) {
    a.counters = static_cast<uint32_t*>(ws);
    a.counter_stride = counter_stride((int64_t)a.batch * a.n_kv_head, kMaxCounters);
    a.plan = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + kCounterBytes);
    float* f = reinterpret_cast<float*>(static_cast<char*>(ws) + kCounterBytes + kPlanBytes);
    const size_t n = (size_t)a.batch * a.n_head * a.n_splits;
    a.po = f;
    a.pm = f + n * kHeadDim;
    a.pl = a.pm + n;
    a.po_bytes = (uint32_t)(n * kHeadDim * sizeof(float));
}

DecodeArgs common_args(const void* q, const void* k, const void* v, void* out, int out_dtype,
                       int64_t batch, int64_t n_head, int64_t n_kv_head, int64_t max_seq,
                       int64_t head_dim = kHeadDim) {
    DecodeArgs a{};
    a.q = q;
    a.k_pool = static_cast<half_t*>(const_cast<void*>(k));  // written only by the fused append
    a.v_pool = static_cast<half_t*>(const_cast<void*>(v));
    a.out = out;
    a.q_row_stride = (int32_t)(n_head * head_dim);
    a.out_row_stride = (int32_t)(n_head * head_dim);
    a.batch = (int)batch;
    a.n_head = (int)n_head;
    a.n_kv_head = (int)n_kv_head;
    a.n_rep = (int)(n_head / n_kv_head);
    a.max_seq = (int)max_seq;
    a.max_pages = (int)((max_seq + kPageMask) >> kPageShift);
    a.out_f16 = out_dtype == CRUCIBLE_F16;
    a.scale_log2 = head_dim == kHeadDim ? 0.125f * kLog2e
                                        : (float)(1.4426950408889634 / std::sqrt((double)head_dim));
    return a;
}

// head_dim other than 64: decode_generic_kernel over (request, query head). Appends, where
// the entry has them, are launched before it on the same stream.
int launch_decode_generic(const DecodeArgs& a, int hd, bool q_f32, hipStream_t stream,
                          const char* what) {
    CRUCIBLE_CHECK(a.n_head <= 65535, CRUCIBLE_ERR_INVALID, "%s: n_head %d too large", what,
                   a.n_head);
    CRUCIBLE_CHECK(aligned16(a.k_pool) && aligned16(a.v_pool), CRUCIBLE_ERR_INVALID,
                   "%s: pools must be 16-byte aligned", what);
    const dim3 grid((unsigned)a.batch, (unsigned)a.n_head);
    if (q_f32)
        hipLaunchKernelGGL(decode_generic_kernel<true>, grid, dim3(kGenericThreads), 0, stream, a, hd);
    else
        hipLaunchKernelGGL(decode_generic_kernel<false>, grid, dim3(kGenericThreads), 0, stream, a, hd);
    return fail_launch(what);
}

// The two appends of the fused entries for head_dim other than 64, f32 or fp16 rows of
// stride kv_dim: the library's own crucible_cache_store_rows_paged, so the pools get the
// bytes the separate calls store.
int append_rows_generic(const DecodeArgs& a, int kv_dtype, int64_t n_layer, int64_t layer,
                        hipStream_t stream) {
    for (int kind : {CRUCIBLE_POOL_K, CRUCIBLE_POOL_V}) {
        const bool k = kind == CRUCIBLE_POOL_K;
        if (const int rc = crucible_cache_store_rows_paged(
                k ? a.k_new : a.v_new, kv_dtype, k ? a.k_pool : a.v_pool, kind, a.tables,
                a.positions, a.batch, a.addr.kv_dim, a.table_stride, n_layer, layer,
                reinterpret_cast<crucible_stream_t>(stream)))
            return rc;
    }
    return CRUCIBLE_OK;
}

// Split the request into workgroups, bind the workspace and launch.
int decode_with_workspace(DecodeArgs& a, bool q_f32, void* workspace, size_t workspace_bytes,
                          hipStream_t stream, const char* what) {
    // the kernel moves q, pools, out and appended rows in 16-byte vectors
    CRUCIBLE_CHECK(aligned16(a.q) && aligned16(a.k_pool) && aligned16(a.v_pool) &&
                       aligned16(a.out) && aligned16(a.k_new) && aligned16(a.v_new),
                   CRUCIBLE_ERR_INVALID, "%s: q, pools, out and new rows must be 16-byte aligned",
                   what);
    const DecodeShape sh = decode_shape(a.batch, a.n_kv_head, a.max_pages);
    const int split_pages = sh.pages * sh.waves;  // a power of two
    a.split_shift = __builtin_ctz((unsigned)split_pages);
    a.n_splits = (a.max_pages + split_pages - 1) / split_pages;
    if (a.n_splits > 1) {
        CRUCIBLE_CHECK((size_t)a.batch * a.n_head * a.n_splits * kHeadDim * sizeof(float) <
                           ((size_t)1 << 31),
                       CRUCIBLE_ERR_INVALID, "%s: split partials exceed 2 GiB", what);
        CRUCIBLE_CHECK((int64_t)a.batch * a.n_kv_head <= kMaxCounters, CRUCIBLE_ERR_INVALID,
                       "%s: batch * n_kv_head exceeds %lld", what, (long long)kMaxCounters);
        const size_t need = workspace_need(a.batch, a.n_head, a.n_splits);
        CRUCIBLE_CHECK(workspace && workspace_bytes >= need, CRUCIBLE_ERR_WORKSPACE,
                       "%s: workspace needs %zu bytes, got %zu", what, need,
                       workspace ? workspace_bytes : (size_t)0);
        CRUCIBLE_CHECK(((uintptr_t)workspace & 15) == 0, CRUCIBLE_ERR_WORKSPACE,
                       "%s: workspace must be 16-byte aligned", what);
        bind_workspace(a, workspace);
    }
    return launch_decode(a, sh, q_f32, stream, what);
}

// ---------------------------------------------------------------- allocation-free form
// For callers that cannot allocate (code under graph capture, serving loops, harnesses that
// forbid hipMalloc): the split-K scratch of crucible_attention_decode_paged_append_noalloc
// lives in this file-scope device array, one copy per GPU, held until the process ends.
// Its first kScratchCounters u32 are the combine counters (zero at load, cleared again by
// a fill kernel at set-up, and left zero by every launch); the partials follow. Host code
// never passes `scratch` itself to a kernel: in host code the name is only a stand-in, so
// the device address comes from hipGetSymbolAddress, once per device.
constexpr size_t kScratchBytes = size_t(4) << 20;
constexpr int64_t kScratchCounters = 8192;
constexpr size_t kScratchCounterBytes = kScratchCounters * sizeof(uint32_t);
__device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ __launch_bounds__(256) void clear_counters_kernel(uint32_t* c, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) c[i] = 0u;
}

constexpr int kMaxDevices = 64;
struct ScratchSlot {
    std::mutex mu;
    std::atomic<void*> ptr{nullptr};
};
ScratchSlot g_scratch[kMaxDevices];

// The device address of this GPU's `scratch`, looked up (and its counters cleared on
// `stream`) the first time a device is used; nullptr with the error message set on failure,
// in which case the next call on that device tries again. Under stream capture the clear is
// recorded into the graph instead of running; that is harmless, because the counters are
// zero at load and every launch leaves them zero.
void* scratch_ptr(hipStream_t stream, const char* what) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        set_error(CRUCIBLE_ERR_LAUNCH, "%s: no current device (or more than %d)", what,
                  kMaxDevices);
        return nullptr;
    }
    ScratchSlot& slot = g_scratch[dev];
    if (void* p = slot.ptr.load(std::memory_order_acquire)) return p;
    std::lock_guard<std::mutex> lock(slot.mu);
    if (void* p = slot.ptr.load(std::memory_order_relaxed)) return p;
    void* p = nullptr;
    hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err == hipSuccess) {
        hipLaunchKernelGGL(clear_counters_kernel, dim3((kScratchCounters + 255) / 256),
                           dim3(256), 0, stream, static_cast<uint32_t*>(p),
                           (int)kScratchCounters);
        err = hipGetLastError();
    } else {
        (void)hipGetLastError();
    }
    if (err != hipSuccess) {
        set_error(CRUCIBLE_ERR_LAUNCH, "%s: device scratch unavailable on device %d: %s", what,
                  dev, hipGetErrorString(err));
        return nullptr;
    }
    slot.ptr.store(p, std::memory_order_release);
    return p;
}

}  // namespace
}  // namespace crucible

using namespace crucible;

extern "C" size_t crucible_attention_decode_workspace_bytes(int64_t batch, int64_t n_head,
                                                            int64_t max_seq) {
    if (batch <= 0 || n_head <= 0 || max_seq <= 0) return 0;
    // past the entry points' limits (max_seq and batch <= INT32_MAX) the need saturates
    if (max_seq > INT32_MAX || batch > INT32_MAX) return SIZE_MAX;
    const int64_t max_pages = (max_seq + kPageMask) >> kPageShift;
    const int64_t n_splits = (max_pages + 3) / 4;  // the smallest split: 1 page x 4 waves
    return workspace_need(batch, n_head, n_splits);
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
    CRUCIBLE_CHECK(table_stride > 0 && table_stride <= INT32_MAX && max_seq > 0 &&
                       max_seq <= table_stride * kPageTokens && max_seq <= INT32_MAX,
                   CRUCIBLE_ERR_INVALID, "%s: max_seq %lld must be in 1..table_stride*16", what,
                   (long long)max_seq);
    DecodeArgs a = common_args(q, k_pool, v_pool, out, out_dtype, batch, n_head, n_kv_head,
                               max_seq, head_dim);
    a.tables = page_tables;
    a.lens = seq_lens;
    a.lens_stride = 1;
    a.addr.kv_dim = (int32_t)kv_dim;
    CRUCIBLE_CHECK(paged_addr(n_layer, layer, kv_dim, a.addr), CRUCIBLE_ERR_INVALID,
                   "%s: page geometry of %lld layers x %lld channels overflows", what,
                   (long long)n_layer, (long long)kv_dim);
    a.table_stride = (int32_t)table_stride;
    if (head_dim != kHeadDim)
        return launch_decode_generic(a, (int)head_dim, q_dtype == CRUCIBLE_F32, stream, what);
    return decode_with_workspace(a, q_dtype == CRUCIBLE_F32, workspace, workspace_bytes, stream,
                                 what);
}

extern "C" int crucible_attention_decode_paged_append(
    const void* q, int q_dtype, const void* k_new, const void* v_new, int kv_dtype, void* k_pool,
    void* v_pool, void* out, int out_dtype, const int32_t* page_tables, const int32_t* positions,
    const int32_t* seq_lens, int64_t batch, int64_t n_head, int64_t n_kv_head, int64_t head_dim,
    int64_t table_stride, int64_t n_layer, int64_t layer, int64_t kv_dim, int64_t max_seq,
    void* workspace, size_t workspace_bytes, crucible_stream_t stream) {
    const char* what = "attention_decode_paged_append";
    CRUCIBLE_CHECK(dtype_ok(q_dtype) && dtype_ok(out_dtype) && dtype_ok(kv_dtype),
                   CRUCIBLE_ERR_INVALID, "%s: bad dtype", what);
    if (int rc = check_geometry(what, n_head, n_kv_head, head_dim, kv_dim)) return rc;
    CRUCIBLE_CHECK(batch >= 0 && batch <= INT32_MAX, CRUCIBLE_ERR_INVALID, "%s: batch %lld",
                   what, (long long)batch);
    if (batch == 0) return CRUCIBLE_OK;
    CRUCIBLE_CHECK(q && k_new && v_new && k_pool && v_pool && out && page_tables && positions &&
                       seq_lens,
                   CRUCIBLE_ERR_INVALID, "%s: null buffer", what);
    CRUCIBLE_CHECK(n_layer > 0 && layer >= 0 && layer < n_layer, CRUCIBLE_ERR_INVALID,
                   "%s: layer %lld outside n_layer %lld", what, (long long)layer,
                   (long long)n_layer);
    CRUCIBLE_CHECK(table_stride > 0 && table_stride <= INT32_MAX && max_seq > 0 &&
                       max_seq <= table_stride * kPageTokens && max_seq <= INT32_MAX,
                   CRUCIBLE_ERR_INVALID, "%s: max_seq %lld must be in 1..table_stride*16", what,
                   (long long)max_seq);
    DecodeArgs a = common_args(q, k_pool, v_pool, out, out_dtype, batch, n_head, n_kv_head,
                               max_seq, head_dim);
    a.tables = page_tables;
    a.lens = seq_lens;
    a.lens_stride = 1;
    a.positions = positions;
    a.k_new = k_new;
    a.v_new = v_new;
    a.kv_new_f16 = kv_dtype == CRUCIBLE_F16;
    a.kv_new_stride = (int32_t)kv_dim;
    a.addr.kv_dim = (int32_t)kv_dim;
    CRUCIBLE_CHECK(paged_addr(n_layer, layer, kv_dim, a.addr), CRUCIBLE_ERR_INVALID,
                   "%s: page geometry of %lld layers x %lld channels overflows", what,
                   (long long)n_layer, (long long)kv_dim);
    a.table_stride = (int32_t)table_stride;
    if (head_dim != kHeadDim) {
        if (const int rc = append_rows_generic(a, kv_dtype, n_layer, layer, stream)) return rc;
        return launch_decode_generic(a, (int)head_dim, q_dtype == CRUCIBLE_F32, stream, what);
    }
    return decode_with_workspace(a, q_dtype == CRUCIBLE_F32, workspace, workspace_bytes, stream,
                                 what);
}

extern "C" int crucible_attention_decode_paged_append_noalloc(
    const void* q, int q_dtype, const void* k_new, const void* v_new, int kv_dtype,
    void* k_pool, void* v_pool, void* out, int out_dtype, const int32_t* page_tables,
    const int32_t* positions, const int32_t* seq_lens, int64_t batch, int64_t n_head,
    int64_t n_kv_head, int64_t head_dim, int64_t table_stride, int64_t n_layer, int64_t layer,
    int64_t kv_dim, int64_t max_seq, crucible_stream_t stream) {
    const char* what = "attention_decode_paged_append_noalloc";
    CRUCIBLE_CHECK(dtype_ok(q_dtype) && dtype_ok(out_dtype) && dtype_ok(kv_dtype),
                   CRUCIBLE_ERR_INVALID, "%s: bad dtype", what);
    if (int rc = check_geometry(what, n_head, n_kv_head, head_dim, kv_dim)) return rc;
    CRUCIBLE_CHECK(batch >= 0 && batch <= INT32_MAX, CRUCIBLE_ERR_INVALID, "%s: batch %lld",
                   what, (long long)batch);
    if (batch == 0) return CRUCIBLE_OK;
    CRUCIBLE_CHECK(q && k_new && v_new && k_pool && v_pool && out && page_tables && positions &&
                       seq_lens,
                   CRUCIBLE_ERR_INVALID, "%s: null buffer", what);
    CRUCIBLE_CHECK(n_layer > 0 && layer >= 0 && layer < n_layer, CRUCIBLE_ERR_INVALID,
                   "%s: layer %lld outside n_layer %lld", what, (long long)layer,
                   (long long)n_layer);
    CRUCIBLE_CHECK(table_stride > 0 && table_stride <= INT32_MAX && max_seq > 0 &&
                       max_seq <= table_stride * kPageTokens && max_seq <= INT32_MAX,
                   CRUCIBLE_ERR_INVALID, "%s: max_seq %lld must be in 1..table_stride*16", what,
                   (long long)max_seq);
    DecodeArgs a = common_args(q, k_pool, v_pool, out, out_dtype, batch, n_head, n_kv_head,
                               max_seq, head_dim);
    a.tables = page_tables;
    a.lens = seq_lens;
    a.lens_stride = 1;
    a.positions = positions;
    a.k_new = k_new;
    a.v_new = v_new;
    a.kv_new_f16 = kv_dtype == CRUCIBLE_F16;
    a.kv_new_stride = (int32_t)kv_dim;
    a.addr.kv_dim = (int32_t)kv_dim;
    CRUCIBLE_CHECK(paged_addr(n_layer, layer, kv_dim, a.addr), CRUCIBLE_ERR_INVALID,
                   "%s: page geometry of %lld layers x %lld channels overflows", what,
                   (long long)n_layer, (long long)kv_dim);
    a.table_stride = (int32_t)table_stride;
    if (head_dim != kHeadDim) {  // the generic kernels use no scratch
        if (const int rc = append_rows_generic(a, kv_dtype, n_layer, layer, stream)) return rc;
        return launch_decode_generic(a, (int)head_dim, q_dtype == CRUCIBLE_F32, stream, what);
    }
    CRUCIBLE_CHECK(aligned16(a.q) && aligned16(a.k_pool) && aligned16(a.v_pool) &&
                       aligned16(a.out) && aligned16(a.k_new) && aligned16(a.v_new),
                   CRUCIBLE_ERR_INVALID, "%s: q, pools, out and new rows must be 16-byte aligned",
                   what);
    const DecodeShape sh = decode_shape(a.batch, a.n_kv_head, a.max_pages);
    const int split_pages = sh.pages * sh.waves;
    a.split_shift = __builtin_ctz((unsigned)split_pages);
    a.n_splits = (a.max_pages + split_pages - 1) / split_pages;
    if (a.n_splits > 1) {
        // the limits of the static scratch: counters and partials
        const size_t floats = partial_floats(a.batch, a.n_head, a.n_splits);
        const size_t partial_bytes =
            floats > SIZE_MAX / sizeof(float) ? SIZE_MAX : floats * sizeof(float);
        CRUCIBLE_CHECK((int64_t)a.batch * a.n_kv_head <= kScratchCounters &&
                           partial_bytes <= kScratchBytes - kScratchCounterBytes,
                       CRUCIBLE_ERR_WORKSPACE,
                       "%s: batch %lld x %lld kv heads at max_seq %lld needs %zu bytes of split "
                       "partials and %lld counters; the static scratch holds %zu bytes and %lld "
                       "counters (use crucible_attention_decode_paged_append with a workspace)",
                       what, (long long)batch, (long long)n_kv_head, (long long)max_seq,
                       partial_bytes, (long long)a.batch * a.n_kv_head,
                       kScratchBytes - kScratchCounterBytes, (long long)kScratchCounters);
        void* ptr = scratch_ptr(stream, what);
        if (!ptr) return CRUCIBLE_ERR_LAUNCH;
        a.counters = static_cast<uint32_t*>(ptr);
        a.counter_stride = counter_stride((int64_t)a.batch * a.n_kv_head, kScratchCounters);
        float* f = reinterpret_cast<float*>(static_cast<char*>(ptr) + kScratchCounterBytes);
        const size_t n = (size_t)a.batch * a.n_head * a.n_splits;
        a.po = f;
        a.pm = f + n * kHeadDim;
        a.pl = a.pm + n;
        a.po_bytes = (uint32_t)(n * kHeadDim * sizeof(float));
    }
    return launch_decode(a, sh, q_dtype == CRUCIBLE_F32, stream, what);
}

extern "C" int crucible_attention_decode_qkv_paged_append(
    const float* qkv, int64_t qkv_row_stride, const float* rope_cos, const float* rope_sin,
    int64_t rope_max_pos, void* k_pool, void* v_pool, void* out, int out_dtype,
    const int32_t* page_tables, const int32_t* positions, const int32_t* seq_lens, int64_t batch,
    int64_t n_head, int64_t n_kv_head, int64_t head_dim, int64_t table_stride, int64_t n_layer,
    int64_t layer, int64_t kv_dim, int64_t max_seq, void* workspace, size_t workspace_bytes,
    crucible_stream_t stream) {
    const char* what = "attention_decode_qkv_paged_append";
    CRUCIBLE_CHECK(dtype_ok(out_dtype), CRUCIBLE_ERR_INVALID, "%s: bad dtype", what);
    if (int rc = check_geometry(what, n_head, n_kv_head, head_dim, kv_dim)) return rc;
    CRUCIBLE_CHECK(batch >= 0 && batch <= INT32_MAX, CRUCIBLE_ERR_INVALID, "%s: batch %lld",
                   what, (long long)batch);
    if (batch == 0) return CRUCIBLE_OK;
    CRUCIBLE_CHECK(qkv && k_pool && v_pool && out && page_tables && positions && seq_lens,
                   CRUCIBLE_ERR_INVALID, "%s: null buffer", what);
    CRUCIBLE_CHECK(qkv_row_stride >= n_head * head_dim + 2 * kv_dim && qkv_row_stride % 4 == 0 &&
                       qkv_row_stride <= INT32_MAX,
                   CRUCIBLE_ERR_INVALID,
                   "%s: qkv_row_stride %lld must hold q, k and v and be a multiple of 4", what,
                   (long long)qkv_row_stride);
    CRUCIBLE_CHECK(n_layer > 0 && layer >= 0 && layer < n_layer, CRUCIBLE_ERR_INVALID,
                   "%s: layer %lld outside n_layer %lld", what, (long long)layer,
                   (long long)n_layer);
    CRUCIBLE_CHECK(table_stride > 0 && table_stride <= INT32_MAX && max_seq > 0 &&
                       max_seq <= table_stride * kPageTokens && max_seq <= INT32_MAX,
                   CRUCIBLE_ERR_INVALID, "%s: max_seq %lld must be in 1..table_stride*16", what,
                   (long long)max_seq);
    CRUCIBLE_CHECK((rope_cos == nullptr) == (rope_sin == nullptr), CRUCIBLE_ERR_INVALID,
                   "%s: rope_cos and rope_sin go together", what);
    CRUCIBLE_CHECK(!rope_cos || (rope_max_pos >= max_seq && rope_max_pos <= INT32_MAX &&
                                 aligned16(rope_cos) && aligned16(rope_sin)),
                   CRUCIBLE_ERR_INVALID,
                   "%s: rope tables must cover max_seq positions (16-byte aligned)", what);
    DecodeArgs a = common_args(qkv, k_pool, v_pool, out, out_dtype, batch, n_head, n_kv_head,
                               max_seq, head_dim);
    a.q_row_stride = (int32_t)qkv_row_stride;
    a.tables = page_tables;
    a.lens = seq_lens;
    a.lens_stride = 1;
    a.positions = positions;
    a.k_new = qkv + n_head * head_dim;
    a.v_new = qkv + n_head * head_dim + kv_dim;
    a.kv_new_f16 = 0;
    a.kv_new_stride = (int32_t)qkv_row_stride;
    a.rope_cos = rope_cos;
    a.rope_sin = rope_sin;
    a.rope_max_pos = (int)rope_max_pos;
    a.addr.kv_dim = (int32_t)kv_dim;
    CRUCIBLE_CHECK(paged_addr(n_layer, layer, kv_dim, a.addr), CRUCIBLE_ERR_INVALID,
                   "%s: page geometry of %lld layers x %lld channels overflows", what,
                   (long long)n_layer, (long long)kv_dim);
    a.table_stride = (int32_t)table_stride;
    if (head_dim != kHeadDim) {
        const int64_t threads = batch * n_kv_head * (head_dim / 2);
        CRUCIBLE_CHECK(threads <= (int64_t)INT32_MAX * 256, CRUCIBLE_ERR_INVALID, "%s: too many rows",
                       what);
        hipLaunchKernelGGL(append_rope_generic_kernel, dim3((unsigned)((threads + 255) / 256)),
                           dim3(256), 0, stream, a, (int)head_dim);
        if (const int rc = fail_launch(what)) return rc;
        return launch_decode_generic(a, (int)head_dim, true, stream, what);
    }
    return decode_with_workspace(a, true, workspace, workspace_bytes, stream, what);
}

// The decode kernel an entry point would launch for this shape, as rocprof names it
// (template arguments PAGES, WAVES, QF32, APPEND, PAGED, ORDER, ROPE, CW), following the
// same choices as the launch path (shape, grid order, combine width, overrides).
extern "C" int crucible_attention_decode_kernel_name(int64_t batch, int64_t n_head,
                                                     int64_t n_kv_head, int64_t max_seq,
                                                     int q_dtype, int entry, char* buf,
                                                     size_t n) {
    // the entry points' own limits (batch and max_seq up to INT32_MAX, n_head up to 2^20, a
    // positive multiple of n_kv_head)
    if (!buf || n == 0 || batch <= 0 || batch > INT32_MAX || n_head <= 0 || n_head > (1 << 20) ||
        n_kv_head <= 0 || n_head % n_kv_head != 0 || max_seq <= 0 || max_seq > INT32_MAX ||
        entry < 0 || entry > 2) {
        set_error(CRUCIBLE_ERR_INVALID, "decode_kernel_name: bad arguments");
        return CRUCIBLE_ERR_INVALID;
    }
    const int64_t max_pages = (max_seq + kPageMask) >> kPageShift;
    const bool append = entry != 0;
    const bool rope = entry == 2;
    const bool qf32 = rope || q_dtype == CRUCIBLE_F32;
    const DecodeShape sh = decode_shape(batch, n_kv_head, max_pages);
    const int pages = sh.pages;
    const int waves = sh.waves;
    const int n_splits = (int)((max_pages + pages * waves - 1) / (pages * waves));
    const int64_t units = (int64_t)n_splits * n_kv_head * batch;
    int order = (units > device_cu_count() && batch <= kCompactMaxBatch) ? kOrderCompact
                                                                        : kOrderRequest;
    if (const int v = tuning(CRUCIBLE_TUNE_DECODE_ORDER); v >= 0)
        order = (v == kOrderCompact && batch > kCompactMaxBatch) ? kOrderRequest : v;
    const int wv = tuning(CRUCIBLE_TUNE_DECODE_COMBINE_WIDTH);
    const int cw = order == kOrderSplit ? 8 : (wv > 0 ? wv : (n_splits > 8 ? 16 : 8));
    std::snprintf(buf, n, "decode_kernel<%d, %d, %s, %s, true, %d, %s, %d>", pages, waves,
                  qf32 ? "true" : "false", append ? "true" : "false", order,
                  rope ? "true" : "false", cw);
    return CRUCIBLE_OK;
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
    CRUCIBLE_CHECK(max_seq > 0 && max_seq <= INT32_MAX, CRUCIBLE_ERR_INVALID,
                   "%s: max_seq %lld", what, (long long)max_seq);
    // the last position's element index, layer_base + max_seq * cache_stride, fits int64
    // (max_seq * cache_stride < 2^59 after the checks above)
    CRUCIBLE_CHECK(layer_base >= 0 && layer_base <= INT64_MAX - max_seq * cache_stride,
                   CRUCIBLE_ERR_INVALID, "%s: layer_base %lld", what, (long long)layer_base);
    DecodeArgs a = common_args(q, k_cache, v_cache, out, out_dtype, 1, n_head, n_kv_head,
                               max_seq, head_dim);
    a.lens = params;
    a.lens_off = kParamSeq;
    a.addr.kv_dim = (int32_t)cache_stride;
    a.addr.page_stride = kPageTokens * cache_stride;
    a.addr.layer_off = layer_base;
    if (head_dim != kHeadDim)
        return launch_decode_generic(a, (int)head_dim, q_dtype == CRUCIBLE_F32, stream, what);
    return decode_with_workspace(a, q_dtype == CRUCIBLE_F32, workspace, workspace_bytes, stream,
                                 what);
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
    CRUCIBLE_CHECK(capacity > 0 && capacity <= INT32_MAX, CRUCIBLE_ERR_INVALID,
                   "%s: capacity %lld", what, (long long)capacity);
    CRUCIBLE_CHECK(layer_base >= 0 && layer_base <= INT64_MAX - capacity * cache_stride,
                   CRUCIBLE_ERR_INVALID, "%s: layer_base %lld", what, (long long)layer_base);
    DecodeArgs a = common_args(q, k_cache, v_cache, out, out_dtype, 1, n_head, n_kv_head,
                               capacity, head_dim);
    a.lens = params;
    a.lens_off = kParamSeq;
    a.addr.kv_dim = (int32_t)cache_stride;
    a.addr.page_stride = kPageTokens * cache_stride;
    a.addr.layer_off = layer_base;
    // head_dim other than 64: the generic kernel writes the output in one pass (the partial
    // buffers are left as they are)
    if (head_dim != kHeadDim)
        return launch_decode_generic(a, (int)head_dim, q_dtype == CRUCIBLE_F32, stream, what);
    // 128-position chunks as in the reference (gpu.rs:37 ATTN_CHUNK): 4 waves x 2 pages,
    // partials in the caller's buffers, combined by a second kernel.
    const DecodeShape sh{2, 4};
    a.split_shift = 3;  // 8 pages
    a.n_splits = (int)((capacity + 127) / 128);
    a.po = partial_o;
    a.pm = partial_m;
    a.pl = partial_l;
    a.counters = nullptr;
    CRUCIBLE_CHECK((size_t)n_head * a.n_splits * kHeadDim * sizeof(float) < ((size_t)1 << 31),
                   CRUCIBLE_ERR_INVALID, "%s: split partials exceed 2 GiB", what);
    a.po_bytes = (uint32_t)((size_t)n_head * a.n_splits * kHeadDim * sizeof(float));
    return launch_decode(a, sh, q_dtype == CRUCIBLE_F32, stream, what);
}

#ifdef CRUCIBLE_STAMPS
// Diagnostic build only: copy the first `rows` rows of the phase stamps (*slots u64 each,
// in StampSlot order) to `host`, then zero them on the device if `clear`. The clock's rate
// in kHz goes to *clock_khz. Synchronous: it waits for the device first.
extern "C" int crucible_debug_decode_stamps(uint64_t* host, int64_t rows, int clear,
                                            int* clock_khz, int* slots) {
    using namespace crucible;
    const char* what = "crucible_debug_decode_stamps";
    CRUCIBLE_CHECK(rows >= 0 && rows <= kStampRows && (rows == 0 || host) && clock_khz && slots,
                   CRUCIBLE_ERR_INVALID, "%s: %lld rows (at most %d)", what, (long long)rows,
                   kStampRows);
    *slots = kStampSlots;
    int dev = 0;
    void* p = nullptr;
    const size_t bytes = (size_t)rows * kStampSlots * sizeof(uint64_t);
    const bool ok =
        hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(clock_khz, hipDeviceAttributeWallClockRate, dev) == hipSuccess &&
        hipDeviceSynchronize() == hipSuccess &&
        (rows == 0 || hipMemcpyFromSymbol(host, HIP_SYMBOL(g_decode_stamps), bytes, 0,
                                          hipMemcpyDeviceToHost) == hipSuccess) &&
        (!clear || (hipGetSymbolAddress(&p, HIP_SYMBOL(g_decode_stamps)) == hipSuccess &&
                    hipMemset(p, 0, sizeof(g_decode_stamps)) == hipSuccess &&
                    hipDeviceSynchronize() == hipSuccess));
    CRUCIBLE_CHECK(ok, CRUCIBLE_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(hipGetLastError()));
    return CRUCIBLE_OK;
}
#endif
