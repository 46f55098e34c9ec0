// Causal prefill attention for gfx950: flash-style tiles on MFMA (fp16 in, fp32 acc).
//
// Reference semantics (engine/kernels/kernels.cu:1844-1948 reference prefill, and
// 2100-2276 for the segment-descriptor form): query row r at absolute position pos_r
// attends to keys [0, pos_r] of its own sequence through that sequence's page table;
// head h reads kv head h / (n_head / n_kv_head); scores are scaled by 1/sqrt(64).
//
// One kernel serves every reference prefill entry point; they differ only in how a
// query row finds its (table, position):
//   SEGMENTS  {packed_start, chunk_len, absolute_start, table_index} per request
//             (attention_prefill_tiled, gpu.rs:1606-1751)
//   OWNERS    owners[r], positions[r] per row (attention_prefill_packed, gpu.rs:1551-1604)
//   PARAMS    one table, position params[5] + r (attention_prefill_paged, gpu.rs:1502-1549)
//   CONTIG    contiguous cache, position pos_offset + r (attention_prefill, gpu.rs:1886-1934)
//
// Workgroup = 8 waves: 4 slots = (4 / HPW) row slices x HPW query heads of one GQA
// group, so the HPW heads that share a kv head share every K/V tile staged in LDS, and
// two waves per slot that take alternate 64-key tiles (their online-softmax states merge
// at the end). A slot owns QB blocks of 16 query rows for one head. Per 64-key tile and
// 16-row block, the wave that owns the tile computes:
//   S^T[64 key x 16 q] = K[64 x 64] . Q^T        8x mfma_f32_16x16x32_f16
//   online softmax per query column (base 2), causal mask by absolute position (skipped
//     for tiles wholly below the diagonal), lazy rescaling of the accumulators
//   O^T[64 dim x 16 q] += V^T[64 x 64 key] . P^T 16x mfma_f32_16x16x32_f16, with P
//     split into fp16 hi + lo parts so the product keeps ~22 bits of P (an f32 query
//     is split the same way for QK^T)
// The transposed V pages are copied into LDS as-is (no transpose on the way), and the
// P^T operand is exactly the register layout the S^T product leaves behind.
// Tiles stream into a ring of KB LDS buffers with direct-to-LDS loads
// (global_load_lds_dwordx4, no register staging), a pair of tiles or two ahead of the
// pair being computed, so HBM latency overlaps the MFMA work; 16-byte chunks of each 128-byte LDS
// row are XOR-swizzled by row so the operand reads stay (almost) free of bank conflicts.
// A wave skips tiles that lie wholly above the causal diagonal of its rows (the
// workgroup still loads up to its last row).
//
// Rows of a workgroup are processed in runs of one owner (table). SEGMENTS, PARAMS and
// CONTIG tiles are always a single run; an OWNERS tile that straddles two requests
// makes two passes, each masking the rows of the other request.
#include "common.hpp"
#include "generic_attend.hpp"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <type_traits>

namespace crucible {
namespace {

enum RowMode { kSegments = 0, kOwners = 1, kParams = 2, kContig = 3 };

constexpr int kKeyTile = 64;

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0], expcnt[6:4] = 7 (no wait), lgkmcnt[11:8])
constexpr int kWaitVm0Lgkm0 = 0x0070;
constexpr int kWaitVm4Lgkm0 = 0x0074;
constexpr int kWaitVm8Lgkm0 = 0x0078;
constexpr int kThreads = 512;  // 8 waves: 4 row/head slots x 2 tile parities

#ifdef CRUCIBLE_STAMPS
// Phase stamps of the 16-row LDS kernel (prefill_kernel), compiled only into the
// diagnostic libcrucible_attn_stamps.so. Thread 0 of each workgroup (wave 0: key half 0 of
// the first slot) records s_memrealtime at the end of each phase in row `workgroup id`
// (in the persistent form, the tile's list position; a tile's kPStart is then the time its
// workgroup began it: the kernel's entry for its first tile), and the time its wave spent
// in the tile loop's waits for key tiles (the wait for its own tile loads plus the barrier
// that makes every wave's loads visible).
constexpr int kPStampRows = 8192;
enum PStampSlot {
    kPStart,      // kernel entry
    kPRows,       // rows of the tile resolved (after the first barrier)
    kPFirst,      // first pair of key tiles in LDS (after the loop's first barrier)
    kPLoop,       // tile loop done
    kPMerged,     // key halves merged
    kPWritten,    // output stored (acknowledged)
    kPWait,       // ticks waited for key tiles inside the loop
    kPMeta,       // grid tile | request << 16 | x << 32 | pairs << 48
    kPSlots
};
__device__ uint64_t g_prefill_stamps[kPStampRows][kPSlots];

__device__ __forceinline__ unsigned pstamp_row() {
    return blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
}
__device__ __forceinline__ void pstamp_store(unsigned row, int slot, uint64_t v) {
    if (threadIdx.x == 0 && row < kPStampRows) g_prefill_stamps[row][slot] = v;
}
__device__ __forceinline__ uint64_t pstamp_clock() {
    asm volatile("" ::: "memory");
    return __builtin_amdgcn_s_memrealtime();
}
#define CRUCIBLE_PSTAMP_CLOCK() pstamp_clock()
#define CRUCIBLE_PSTAMP(slot, v) pstamp_store(pstamp_id, slot, v)
#define CRUCIBLE_PSTAMP_AFTER(slot)                                  \
    do {                                                             \
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory"); \
        pstamp_store(pstamp_id, slot, pstamp_clock());               \
    } while (0)
// The register-direct kernel (prefill_direct_kernel) uses the same rows, with slots
// kPRows = rows resolved and the query and first key tile's loads issued, kPFirst = wave
// 0's first key tile resident, kPLoop = wave 0's key tiles done, kPMerged = the waves'
// states merged (after the barrier), kPWritten = output stored; kPWait is 0 and the meta
// word's top field the row tile's number of key tiles. Only wave 0 waits for its memory
// operations at a stamp, so the other waves' loads stay in flight as in the product.
#define CRUCIBLE_PSTAMP_AFTER_W0(slot)                                      \
    do {                                                                    \
        if (threadIdx.x < 64) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory"); \
        pstamp_store(pstamp_id, slot, pstamp_clock());                      \
    } while (0)
#else
__device__ __forceinline__ unsigned pstamp_row() { return 0; }
#define CRUCIBLE_PSTAMP_AFTER_W0(slot) ((void)0)
#define CRUCIBLE_PSTAMP_CLOCK() uint64_t(0)
#define CRUCIBLE_PSTAMP(slot, v) ((void)0)
#define CRUCIBLE_PSTAMP_AFTER(slot) ((void)0)
#endif
constexpr float kLazyLog2 = 8.0f;  // running-max slack (log2 units) before a rescale

// Hand-written instructions and the hazards the compiler cannot see. The compiler inserts
// wait states after the instructions it emits, but an asm block is opaque to it: a block
// that reads MFMA results, the result of a transcendental op, or writes what an MFMA reads
// must supply the wait states itself. CDNA does not interlock MFMA results for VALU reads
// (an 8-pass 16x16x32 result needs about 10 wait states), a VALU read of a v_exp_f32
// result needs 1, a VALU write read by an MFMA needs 2, and v_permlane*_swap needs 2 around
// its VALU neighbours. Missing ones do not fault: the read returns the register's previous
// value, depending on how the other waves' issue fell, so results vary in the last bits
// from launch to launch (a wrong running max only changes the softmax's rounding).
//
// Column max of a lane's 16 scores, then over its 4 lane groups (lanes L, L ^ 16, L ^ 32,
// L ^ 48): v_max3 chains, then v_permlane16_swap / v_permlane32_swap of the value with
// itself (one operand ends with v[L], the other with v[L ^ 16], resp. v[L ^ 32]) and a max.
// It is asm because fmaxf on MFMA results costs a canonicalising v_max per operand, and
// this compiler's permlane swap builtins return the first operand in both halves. The
// block opens with 16 wait states for the MFMA results it reads.
__device__ __forceinline__ float tile_max(const float4_t (&st)[4]) {
    float r, t;
    asm("s_nop 7\n\ts_nop 7\n\t"
        "v_max3_f32 %0, %2, %3, %4\n\t"
        "v_max3_f32 %0, %0, %5, %6\n\t"
        "v_max3_f32 %0, %0, %7, %8\n\t"
        "v_max3_f32 %0, %0, %9, %10\n\t"
        "v_max3_f32 %0, %0, %11, %12\n\t"
        "v_max3_f32 %0, %0, %13, %14\n\t"
        "v_max3_f32 %0, %0, %15, %16\n\t"
        "v_max_f32 %0, %0, %17\n\t"
        "v_mov_b32 %1, %0\n\t"
        "s_nop 1\n\t"
        "v_permlane16_swap_b32 %0, %1\n\t"
        "s_nop 1\n\t"
        "v_max_f32 %0, %0, %1\n\t"
        "v_mov_b32 %1, %0\n\t"
        "s_nop 1\n\t"
        "v_permlane32_swap_b32 %0, %1\n\t"
        "s_nop 1\n\t"
        "v_max_f32 %0, %0, %1"
        : "=&v"(r), "=&v"(t)
        : "v"(st[0][0]), "v"(st[0][1]), "v"(st[0][2]), "v"(st[0][3]), "v"(st[1][0]),
          "v"(st[1][1]), "v"(st[1][2]), "v"(st[1][3]), "v"(st[2][0]), "v"(st[2][1]),
          "v"(st[2][2]), "v"(st[2][3]), "v"(st[3][0]), "v"(st[3][1]), "v"(st[3][2]),
          "v"(st[3][3]));
    return r;
}

// Key order of the LDS form's S^T products. Row m of key block kb (the MFMA's M index, lane group
// m >> 2 holds rows 4 (m >> 2) .. +3) is key
//   key(kb, m) = 32 (kb >> 1) + 8 (m >> 2) + 4 (kb & 1) + (m & 3)
// of the 64-key tile, so after blocks 2 ks and 2 ks + 1 the lanes of group grp hold the
// scores of keys 32 ks + 8 grp .. +7: eight consecutive keys, which is the k range that
// lane group supplies to the PV product (k = 8 grp .. +7 of a 32-key step). Its V^T
// operand is then 16 contiguous bytes of a channel row, one read instead of two 8-byte
// halves joined by register moves. The softmax does not depend on the order of keys.
__device__ __forceinline__ int tile_key(int kb, int m) {
    return 32 * (kb >> 1) + 8 * (m >> 2) + 4 * (kb & 1) + (m & 3);
}

// One lane's 16 scores of a 64-key tile, st[kb][r] = S^T[key(kb, 4 grp + r)][q = col],
// kept unscaled: the scale (> 0) is folded into the exponent, so the max needs none.

// Causal mask: key(kb, 4 grp + r) = 8 grp + 32 (kb >> 1) + 4 (kb & 1) + r of the tile is
// visible iff 32 (kb >> 1) + 4 (kb & 1) + r <= lim, where lim = pos - kbase - 8 grp for a
// row in the run and -1 (nothing visible) otherwise. Written as selects so that it
// compiles to a compare and a select per score.
__device__ __forceinline__ void mask_tile(float4_t (&st)[4], int lim) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            st[kb][r] = (32 * (kb >> 1) + 4 * (kb & 1) + r <= lim) ? st[kb][r] : -INFINITY;
}

// The same mask in the plain block order of the register-direct form, whose K rows come
// from global memory page by page (key block kb = page kb of the tile, st[kb][r] = key
// 16 kb + 4 grp + r): visible iff 16 kb + r <= lim, lim = pos - kbase - 4 grp.
__device__ __forceinline__ void mask_tile_blocks(float4_t (&st)[4], int lim) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) st[kb][r] = (16 * kb + r <= lim) ? st[kb][r] : -INFINITY;
}

// P = exp2(s * scale - mu) (one FMA and one exp per score), split into fp16 P = hi + lo
// (hi truncates, lo = RNE(p - hi): exact to about 2^-22 relative), as the hi/lo
// operands of the PV product: pb/pl[0] hold keys 0..31 of the tile, [1] keys 32..63, in
// the B-operand layout the S^T product leaves (lane group grp: keys 32 ks + 8 grp .. +7
// in the LDS form, see tile_key; keys 4 grp .. +3 of each 16-key block in the direct
// form). Returns the lane's sum of P.
//
//
// P16 (the single-operand precision): P is one fp16 operand, p rounded to nearest even
// (v_cvt_pk_f16_f32), about 2^-12 relative per element, and pl is left untouched; the PV
// product then takes one MFMA per dim block and key half instead of two. l still sums the
// unrounded p, so the rounding errors of the weights stay unbiased.
template <bool P16 = false>
__device__ __forceinline__ float tile_p(const float4_t (&st)[4], float scale, float mu,
                                        half8_t (&pb)[2], half8_t (&pl)[2]) {
    typedef float float2_t __attribute__((ext_vector_type(2)));
    typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
    u32x4_t hw[2], lw[2];
    float part[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        float pf[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) pf[r] = fast_exp2(__builtin_fmaf(st[kb][r], scale, -mu));
        part[kb] = (pf[0] + pf[1]) + (pf[2] + pf[3]);
        if constexpr (P16) {
            hw[kb >> 1][(kb & 1) * 2] = __builtin_bit_cast(
                uint32_t, __builtin_convertvector((float2_t{pf[0], pf[1]}), half2_t));
            hw[kb >> 1][(kb & 1) * 2 + 1] = __builtin_bit_cast(
                uint32_t, __builtin_convertvector((float2_t{pf[2], pf[3]}), half2_t));
        } else {
            const uint32_t h01 =
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(pf[0], pf[1]));
            const uint32_t h23 =
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(pf[2], pf[3]));
            uint32_t lo01, lo23;
            split_lo4(pf, h01, h23, lo01, lo23);
            hw[kb >> 1][(kb & 1) * 2] = h01;
            hw[kb >> 1][(kb & 1) * 2 + 1] = h23;
            lw[kb >> 1][(kb & 1) * 2] = lo01;
            lw[kb >> 1][(kb & 1) * 2 + 1] = lo23;
        }
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        pb[ks] = __builtin_bit_cast(half8_t, hw[ks]);
        if constexpr (!P16) pl[ks] = __builtin_bit_cast(half8_t, lw[ks]);
    }
    return (part[0] + part[1]) + (part[2] + part[3]);
}

// Zeroes the keys at or past the run's end in a V^T operand quarter: element r is key
// k0 + r, kept iff k0 + r < hist_end. Only the last tile of a run needs it (the pages
// there may hold anything, NaN included, and 0 * NaN would poison the product).
__device__ __forceinline__ half4_t zero_tail(half4_t v, int k0, int hist_end) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
        if (k0 + r >= hist_end) v[r] = (half_t)0.0f;
    return v;
}

struct PrefillArgs {
    const void* q;
    const half_t* k_pool;
    const half_t* v_pool;
    void* out;
    const int32_t* tables;     // nullptr in CONTIG mode
    const int32_t* segments;   // SEGMENTS
    const int32_t* owners;     // OWNERS
    const int32_t* positions;  // OWNERS
    const int32_t* params;     // PARAMS
    PoolAddr addr;
    int64_t table_stride;
    int64_t pos_offset;        // CONTIG
    int64_t rows;              // OWNERS / PARAMS / CONTIG
    int mode;
    int n_head;
    int n_kv_head;
    int n_rep;
    int max_seq;
    int out_f16;
    float scale_log2;
    // Longest-first grid: 1-D over (row level, request, x), the last row tiles (the longest
    // causal key ranges) of every request first; 0: grid (x, row tile, request).
    int heavy_first;
    int grid_x;       // heavy_first: x extent (heads or head groups)
    int grid_tiles;   // heavy_first: row tiles
    int grid_reqs;    // heavy_first: requests
    // Hybrid (SEGMENTS, register-direct form only): keys at or past a segment's
    // absolute_start come from the chunk's own rows, cur_k / cur_v [packed row][kv_dim] f32.
    int hybrid;
    const float* cur_k;
    const float* cur_v;
};

// (x, row tile, request) of this workgroup. In the longest-first order, row level v
// (tile grid_tiles - 1 - v) of every request is dispatched before level v + 1: a causal
// row tile's work grows with its index, so the longest-running workgroups start first
// instead of waiting for a free CU at the end. Each level is rotated by one request, so
// a request's tiles alternate over the XCDs (workgroups go to the 8 XCDs round-robin by
// id) instead of all landing on the same ones.
struct WgPos {
    int x;
    int64_t tile;
    int64_t req;
};

// Longest-first id -> (x, row tile, request).
__device__ __forceinline__ WgPos wg_pos(const PrefillArgs& a, uint32_t id) {
    // 32-bit arithmetic: the launcher keeps the ids below 2^31
    const uint32_t per_level = (uint32_t)a.grid_x * (uint32_t)a.grid_reqs;
    const uint32_t level = id / per_level;
    const uint32_t rem =
        (uint32_t)(((uint64_t)(id - level * per_level) + (uint64_t)level * a.grid_x) % per_level);
    return {(int)(rem % (uint32_t)a.grid_x), (int64_t)a.grid_tiles - 1 - level,
            (int64_t)(rem / (uint32_t)a.grid_x)};
}

__device__ __forceinline__ WgPos wg_pos(const PrefillArgs& a) {
    if (!a.heavy_first) return {(int)blockIdx.x, (int64_t)blockIdx.y, (int64_t)blockIdx.z};
    return wg_pos(a, blockIdx.x);
}

// Row `local` of the grid tile: its packed row (-1 = none), owner (table) and absolute
// position, by the entry point's row mode.
__device__ __forceinline__ void tile_row(const PrefillArgs& a, int64_t req, int64_t local,
                                         int& row, int& owner, int& pos) {
    row = -1;
    owner = 0;
    pos = 0;
    if (a.mode == kSegments) {
        const int32_t* seg = a.segments + 4 * req;
        if (local < seg[1]) {
            row = (int)(seg[0] + local);
            pos = (int)(seg[2] + local);
            owner = seg[3];
        }
    } else if (local < a.rows) {
        row = (int)local;
        if (a.mode == kOwners) {
            owner = a.owners[local];
            pos = a.positions[local];
        } else if (a.mode == kParams) {
            pos = (int)(a.params[kParamPrefillPos] + local);
        } else {
            pos = (int)(a.pos_offset + local);
        }
    }
    if (pos < 0 || pos >= a.max_seq) row = -1;  // outside the table: never read
}

// The persistent form's list of row tiles with rows, longest-first: level v (row tile
// grid_tiles - 1 - v) of every request that has that tile, in request order, x fastest
// within a request. Request r has n_r = min(ceil(len_r / R), grid_tiles) tiles, the
// non-persistent grid's coverage, so it holds levels grid_tiles - n_r .. grid_tiles - 1,
// and every level from the first one held (start) on holds at least one request. The
// launcher keeps grid_tiles <= 64, so one lane per level holds the list position where
// that level begins.
struct CompactList {
    int4 seg;          // lane r < grid_reqs: segment r
    int first_level;   // lane r: grid_tiles - n_r
    int start;         // first level any request holds
    int span;          // levels held: grid_tiles - start
    uint32_t begin;    // lane i < span: list position of level start + i's first tile
    uint32_t n_list;   // tiles in the list
};

// Wave 0 alone loads the segments (every wave of every workgroup reading the same few
// lines would queue on one L2 channel) and hands them to the other waves through s_seg.
// The sums and the minimum over the requests are scalar loops over readlane (no LDS
// round trips).
template <int R>
__device__ __forceinline__ CompactList compact_list(const PrefillArgs& a, int wave, int lane,
                                                    int4* s_seg) {
    CompactList c;
    typedef const __attribute__((address_space(1))) int32_t* global_i32_ptr;
    global_i32_ptr segs = (global_i32_ptr)a.segments;
    int n_req = a.grid_reqs;
    asm volatile("" : "+s"(segs), "+s"(n_req));  // both kernel arguments load together
    if (wave == 0 && lane < n_req) {
        const global_i32_ptr sp = segs + 4 * lane;
        s_seg[lane] = int4{sp[0], sp[1], sp[2], sp[3]};
    }
    __syncthreads();
    c.seg = lane < n_req ? s_seg[lane] : int4{0, 0, 0, 0};
    const int len = c.seg.y;
    const int n = len > 0 ? min((len + R - 1) / R, a.grid_tiles) : 0;
    c.first_level = a.grid_tiles - n;
    int lo = a.grid_tiles;
    uint32_t total = 0;
    for (int r = 0; r < n_req; ++r) {
        const int f = __builtin_amdgcn_readlane(c.first_level, r);
        lo = min(lo, f);
        total += (uint32_t)(a.grid_tiles - f);
    }
    c.start = lo;
    c.span = a.grid_tiles - lo;
    c.n_list = total * (uint32_t)a.grid_x;
    // tiles at levels below start + lane: request r holds max(0, start + lane - first_r)
    // of them (grid_x each)
    uint32_t below = 0;
    for (int r = 0; r < n_req; ++r)
        below += (uint32_t)max(0, lo + lane - __builtin_amdgcn_readlane(c.first_level, r));
    c.begin = below * (uint32_t)a.grid_x;
    return c;
}

// (x, row tile, request) at list position k < n_list: the level is the last one that
// begins at or before k (begin grows strictly with the level), then the (j / grid_x)-th
// request holding that level.
__device__ __forceinline__ WgPos compact_pos(const PrefillArgs& a, const CompactList& c,
                                             uint32_t k, int lane) {
    const uint32_t gx = (uint32_t)a.grid_x;
    const uint64_t started = __ballot(lane < c.span && c.begin <= k);
    const int li = __builtin_popcountll(started) - 1;  // level start + li (begin[0] = 0)
    const int v = c.start + li;
    const uint32_t j = k - (uint32_t)__builtin_amdgcn_readlane((int)c.begin, li);
    const uint64_t held = __ballot(lane < a.grid_reqs && c.first_level <= v);
    const uint32_t nth = j / gx;
    const uint32_t before = __builtin_amdgcn_mbcnt_hi(
        (uint32_t)(held >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)held, 0u));
    const uint64_t pick = __ballot(((held >> lane) & 1) && before == nth);
    // (k < n_list always finds one; a position past it would get row tile -1: no rows)
    if (pick == 0 || li < 0 || v >= a.grid_tiles) return {0, -1, 0};
    return {(int)(j - nth * gx), (int64_t)a.grid_tiles - 1 - v, (int64_t)__builtin_ctzll(pick)};
}

// `tables` is passed on its own, read-only and unaliased, so the page-id loads of the
// tile loop compile to scalar loads (lgkmcnt) that never wait on the in-flight tiles.
// KB: LDS ring depth in key tiles (4 or 6): KB / 2 - 1 pairs of tiles load ahead.
// P16: P as one fp16 operand (tile_p), one PV MFMA per dim block and key half.
// PERSIST (segment rows, at most 64 requests and 64 row tiles a request): the grid is the
// resident workgroups, not the tiles. Each workgroup loads all the segments once and from
// their lengths lists the row tiles that hold rows, in the longest-first order
// (compact_list, compact_pos); workgroup w of G then serves list positions w, 2G - 1 - w,
// 2G + w, 4G - 1 - w, ... (each round in the other direction, so the workgroups with the
// heaviest tiles of one round get the lightest of the next, or none). Tiles without rows
// cost nothing, no workgroup waits for a free slot, and nothing is shared between
// workgroups. Every tile's arithmetic is the non-persistent kernel's, so the outputs are
// the same bits.
template <int HPW, int QB, bool QF32, int KB, bool P16, bool PERSIST>
__global__ __launch_bounds__(kThreads) void prefill_kernel(PrefillArgs a,
                                                      const int32_t* __restrict__ tables) {
    constexpr int RS = 4 / HPW;          // row slices per workgroup
    constexpr int WROWS = 16 * QB;       // rows per wave
    constexpr int R = RS * WROWS;        // rows per workgroup

    // ring of key tiles, 128-byte rows whose 16-byte chunks are XOR-swizzled by row
    __shared__ half_t s_k[KB][kKeyTile][64];   // [buf][key][dim]
    __shared__ half_t s_v[KB][64][kKeyTile];   // [buf][dim][key]
    __shared__ int s_owner[R];
    __shared__ int s_pos[R];
    __shared__ int s_row[R];
    __shared__ uint64_t s_mask[2];
    __shared__ int4 s_seg[PERSIST ? 64 : 1];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int col = lane & 15;
    const int grp = lane >> 4;
    // Waves w and w + 4 own the same rows and head (slot w & 3) and split every key tile:
    // wave w takes keys 0..31 of each tile, wave w + 4 keys 32..63. Two waves per SIMD
    // then interleave their MFMA/softmax chains; their states merge at the end.
    const int kh = wave >> 2;   // key half
    const int slot = wave & 3;
    const int rs = slot / HPW;
    const int hi = slot % HPW;

    [[maybe_unused]] const uint64_t t_kernel = CRUCIBLE_PSTAMP_CLOCK();
    // PERSIST: lane r holds segment r and its number of row tiles; n_list tiles in all
    [[maybe_unused]] CompactList cl{};
    if constexpr (PERSIST) cl = compact_list<R>(a, wave, lane, s_seg);

    for (int round = 0;; ++round) {
        [[maybe_unused]] uint32_t k = 0;  // PERSIST: this tile's list position
        if constexpr (PERSIST) {
            const uint32_t G = gridDim.x, w = blockIdx.x;
            k = (round & 1) ? (uint32_t)(round + 1) * G - 1 - w : (uint32_t)round * G + w;
            if (k >= cl.n_list) break;  // uniform; every later round's position is larger
        }
        // a tile's start: the kernel's entry for the first, else the end of the previous tile
        [[maybe_unused]] const uint64_t t_entry = round == 0 ? t_kernel : CRUCIBLE_PSTAMP_CLOCK();
        [[maybe_unused]] uint64_t t_wait = 0;
        [[maybe_unused]] const unsigned pstamp_id = PERSIST ? k : pstamp_row();

        const WgPos wp = PERSIST ? compact_pos(a, cl, k, lane) : wg_pos(a);
        const int groups_per_kv = a.n_rep / HPW;
        const int g = wp.x / groups_per_kv;
        const int h = g * a.n_rep + (wp.x % groups_per_kv) * HPW + hi;

        // ---- rows of this tile: (packed row, owner, absolute position); -1 = none
        int row = -1, owner = 0, pos = 0;
        if constexpr (PERSIST) {
            // the request's segment from the lane that holds it (wp.req is wave-uniform)
            const int r = (int)wp.req;
            const int s0 = __builtin_amdgcn_readlane(cl.seg.x, r);
            const int s1 = __builtin_amdgcn_readlane(cl.seg.y, r);
            const int s2 = __builtin_amdgcn_readlane(cl.seg.z, r);
            const int s3 = __builtin_amdgcn_readlane(cl.seg.w, r);
            if (tid < R) {
                const int64_t local = wp.tile * R + tid;
                if (local >= 0 && local < s1) {
                    row = (int)(s0 + local);
                    pos = (int)(s2 + local);
                    owner = s3;
                }
                if (pos < 0 || pos >= a.max_seq) row = -1;
                s_row[tid] = row;
                s_owner[tid] = owner;
                s_pos[tid] = pos;
            }
        } else if (tid < R) {
            tile_row(a, wp.req, wp.tile * R + tid, row, owner, pos);
            s_row[tid] = row;
            s_owner[tid] = owner;
            s_pos[tid] = pos;
        }
        // valid-row masks of rows 0..63 and 64..127 (R <= 128, so waves 0 and 1 cover them)
        const uint64_t vmask = __ballot(tid < R && row >= 0);
        if (wave < 2 && lane == 0) s_mask[wave] = vmask;
        __syncthreads();
        const uint64_t mask0 = s_mask[0];
        const uint64_t mask1 = R > 64 ? s_mask[1] : 0;
        if (mask0 == 0 && mask1 == 0) {  // uniform: no row of this tile is valid
            if constexpr (!PERSIST) {
                return;
            } else {
                __syncthreads();  // every wave has read the masks before the next tile's rows
                continue;
            }
        }
        CRUCIBLE_PSTAMP(kPStart, t_entry);
        CRUCIBLE_PSTAMP(kPRows, CRUCIBLE_PSTAMP_CLOCK());

        // ---- per-lane query state for each 16-row block (the query rows load after the first
        // run's leading tiles are issued, below, so the two round trips overlap)
        const int64_t ld_q = (int64_t)a.n_head * kHeadDim;
        half8_t qh[QB][2], ql[QB][2];
        float m[QB], l[QB];
        float4_t acc[QB][4];
        int my_row[QB], my_pos[QB];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            const int ri = rs * WROWS + qb * 16 + col;
            my_row[qb] = s_row[ri];
            my_pos[qb] = s_pos[ri];
            m[qb] = -INFINITY;
            l[qb] = 0.0f;
#pragma unroll
            for (int db = 0; db < 4; ++db) acc[qb][db] = float4_t{0.f, 0.f, 0.f, 0.f};
            qh[qb][0] = qh[qb][1] = ql[qb][0] = ql[qb][1] = half8_t{};
        }
        auto load_queries = [&]() {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                if (my_row[qb] < 0) continue;
                const int64_t off = (int64_t)my_row[qb] * ld_q + (int64_t)h * kHeadDim + 8 * grp;
                if constexpr (QF32) {
                    const float* qp = static_cast<const float*>(a.q) + off;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const float x0 = qp[j], x1 = qp[32 + j];
                        qh[qb][0][j] = (half_t)x0;
                        qh[qb][1][j] = (half_t)x1;
                        ql[qb][0][j] = (half_t)(x0 - (float)qh[qb][0][j]);
                        ql[qb][1][j] = (half_t)(x1 - (float)qh[qb][1][j]);
                    }
                } else {
                    const half_t* qp = static_cast<const half_t*>(a.q) + off;
                    qh[qb][0] = *reinterpret_cast<const half8_t*>(qp);
                    qh[qb][1] = *reinterpret_cast<const half8_t*>(qp + 32);
                }
            }
        };

        const int kv_dim = a.addr.kv_dim;
        typedef const __attribute__((address_space(4))) int32_t* const_i32_ptr;

        // ---- runs of one owner (the values come from LDS: readfirstlane makes the compiler
        // treat them as the wave-uniform values they are, so page ids load as scalars)
        // Segment, params and contiguous tiles hold one run of consecutive positions: its
        // rows are the span of valid rows, read off the masks. Owner tiles may hold several
        // runs (one per request) and are scanned row by row.
        const int first_valid = mask0 ? __builtin_ctzll(mask0) : 64 + __builtin_ctzll(mask1);
        const int last_valid = mask1 ? 127 - __builtin_clzll(mask1) : 63 - __builtin_clzll(mask0);
        const int wlo = rs * WROWS, whi = rs * WROWS + WROWS;
        // Wave w stages page w >> 1 of every tile: K rows 8 (w & 1) .. +7 and V^T dims
        // 32 (w & 1) .. +31 of that page (below), so each wave needs one page id per tile.
        const int my_page = wave >> 1;
        bool first_run = true;
#ifdef CRUCIBLE_STAMPS
        bool first_pair_stamp = true;
        int stamp_pairs = 0;
#endif
        int r0 = a.mode == kOwners ? 0 : first_valid;
        while (r0 < R) {
            int r1, owner, hist_end, wave_last;
            if (a.mode != kOwners) {
                r1 = last_valid + 1;
                owner = s_owner[r0];
                hist_end = s_pos[last_valid] + 1;
                const int lo = max(r0, wlo), hi = min(r1, whi);
                wave_last = lo < hi ? s_pos[hi - 1] : -1;
            } else {
                // next run start: first valid row at or after r0
                while (r0 < R && s_row[r0] < 0) ++r0;
                if (r0 >= R) break;
                owner = s_owner[r0];
                r1 = r0 + 1;
                while (r1 < R && s_row[r1] >= 0 && s_owner[r1] == owner) ++r1;
                hist_end = 0;
                for (int r = r0; r < r1; ++r) hist_end = max(hist_end, s_pos[r] + 1);
                // this wave's last visible key within the run
                wave_last = -1;
                for (int r = max(r0, wlo); r < min(r1, whi); ++r)
                    wave_last = max(wave_last, s_pos[r]);
            }
            r0 = __builtin_amdgcn_readfirstlane(r0);
            r1 = __builtin_amdgcn_readfirstlane(r1);
            owner = __builtin_amdgcn_readfirstlane(owner);
            hist_end = __builtin_amdgcn_readfirstlane(hist_end);
            wave_last = __builtin_amdgcn_readfirstlane(wave_last);

            // Page ids go through the scalar cache (constant address space): the tables are
            // never written during a launch, and scalar loads (lgkmcnt) never wait on the
            // in-flight tile loads the way vector loads (vmcnt) would. Without a table
            // (contiguous cache) the page index is the id; the load then reads a harmless word
            // of the pool, so it needs no branch.
            const bool paged = tables != nullptr;
            const const_i32_ptr table =
                paged ? (const_i32_ptr)(tables + (int64_t)owner * a.table_stride)
                      : (const_i32_ptr)a.k_pool;
            const int n_tiles = (hist_end + kKeyTile - 1) / kKeyTile;
            const int last_page = (hist_end - 1) >> kPageShift;
            // This wave's page of tile t; pages past the run's last one are clamped to it (in
            // bounds; their keys are zeroed or masked later).
            auto page_of = [&](int t) -> int64_t {
                const int idx = min(4 * t + my_page, last_page);
                const int id = table[paged ? idx : 0];
                return paged ? (int64_t)id : (int64_t)idx;
            };

            // Issue tile t into ring buffer t % KB: 2 direct-to-LDS loads per thread.
            auto issue = [&](int t, int64_t page) {
                const int buf = t % KB;
                const int64_t base = block_base(a.addr, page);
                // K: wave w covers keys 8w .. 8w+7 of the tile; lane L puts chunk
                // (L & 7) ^ (row & 7) of its row at chunk position L & 7.
                {
                    const int row = 8 * wave + (lane >> 3);
                    const int c = (lane & 7) ^ (row & 7);
                    const half_t* src = a.k_pool + base + (int64_t)(row & kPageMask) * kv_dim +
                                        g * kHeadDim + 8 * c;
                    lds_dma16(src, lds_offset(&s_k[buf][8 * wave][0]));
                }
                // V^T, page-major: buffer `buf` holds the tile's 4 pages, each [64 dims][16 keys]
                // (32-byte rows, the two 8-key halves of a row swapped when bit 3 of the dim is
                // set, which keeps the operand reads free of bank conflicts). Lane L of wave w
                // moves dim 32 (w & 1) + (L >> 1), row position L & 1, of page w >> 1: the
                // wave's 64 lanes fill 1 KiB of that page in order.
                {
                    const int d = 32 * (wave & 1) + (lane >> 1);
                    const int half = (lane & 1) ^ ((d >> 3) & 1);
                    const half_t* src = a.v_pool + base +
                                        (int64_t)(g * kHeadDim + d) * kPageTokens + 8 * half;
                    lds_dma16(src, lds_offset(&s_v[buf][0][0] + my_page * 1024 + (wave & 1) * 512));
                }
            };

            bool in_run[QB];
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                const int ri = rs * WROWS + qb * 16 + col;
                in_run[qb] = my_row[qb] >= 0 && ri >= r0 && ri < r1;
            }

            // Tiles go in pairs: wave w computes tile 2i + (w >> 2) of pair i, so each wave of
            // a slot runs half of the tiles and the two halves' softmax chains overlap.
            constexpr int PS = KB / 2;  // pair slots in the ring
            const int n_pairs = (n_tiles + 1) / 2;
#ifdef CRUCIBLE_STAMPS
            stamp_pairs += n_pairs;
#endif
            // the pair holding the run's last tile when that tile is partial, else none
            const int tail_pair = (hist_end % kKeyTile) ? (n_tiles - 1) / 2 : -1;
#pragma unroll
            for (int p = 0; p < PS - 1; ++p)
                if (p < n_pairs) {
                    const int64_t pa = page_of(2 * p), pb = page_of(2 * p + 1);
                    issue(2 * p, pa);
                    issue(2 * p + 1, pb);  // past n_tiles: a clamped, in-bounds load nobody reads
                }
            if (first_run) {
                // The query operands are complete before the loop, so no wait for them can land
                // inside it (where it would also wait for the tiles in flight).
                load_queries();
                __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0);
                first_run = false;
            }
            for (int ip = 0; ip < n_pairs; ++ip) {
                // Wait for this thread's loads of pair ip (later pairs may stay in flight, 4
                // loads each) and its LDS reads of pair ip - 1; the barrier then makes every
                // wave's loads visible and frees pair ip - 1's buffers for pair ip + PS - 1.
                const int ahead = min(PS - 2, n_pairs - 1 - ip);
                [[maybe_unused]] const uint64_t t_w0 = CRUCIBLE_PSTAMP_CLOCK();
                if (ahead >= 2) __builtin_amdgcn_s_waitcnt(kWaitVm8Lgkm0);
                else if (ahead == 1) __builtin_amdgcn_s_waitcnt(kWaitVm4Lgkm0);
                else __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0);
                // Keys past the run's end may hold anything, NaN included, and P = 0 there
                // would still give 0 * NaN: in the run's last tile, each thread zeroes them in
                // the V^T chunk it loaded (its own load has landed), before the barrier.
                if (ip == tail_pair) {
                    const int t = n_tiles - 1;
                    const int d = 32 * (wave & 1) + (lane >> 1);
                    const int half = (lane & 1) ^ ((d >> 3) & 1);  // keys 16 j + 8 half .. +7
                    const int nv = hist_end - (t * kKeyTile + 16 * my_page + 8 * half);
                    if (nv < 8) {
                        half8_t* chunk = reinterpret_cast<half8_t*>(
                            &s_v[t % KB][0][0] + my_page * 1024 + (wave & 1) * 512) + lane;
                        half8_t v = *chunk;
#pragma unroll
                        for (int r = 0; r < 8; ++r)
                            if (r >= nv) v[r] = (half_t)0.0f;
                        *chunk = v;
                    }
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                }
                __builtin_amdgcn_s_barrier();
#ifdef CRUCIBLE_STAMPS
                {
                    const uint64_t t_w1 = CRUCIBLE_PSTAMP_CLOCK();
                    t_wait += t_w1 - t_w0;
                    if (first_pair_stamp) {
                        CRUCIBLE_PSTAMP(kPFirst, t_w1);
                        first_pair_stamp = false;
                    }
                }
#endif
                if (ip + PS - 1 < n_pairs) {
                    const int tn = 2 * (ip + PS - 1);
                    const int64_t pa = page_of(tn), pb = page_of(tn + 1);
                    issue(tn, pa);
                    issue(tn + 1, pb);
                }
                const int t = 2 * ip + kh;
                const int kbase = t * kKeyTile;
                if (t < n_tiles && wave_last >= kbase) {
                    const int buf = t % KB;
                    // S^T blocks: st[qb][kb] = S^T[kbase + key(kb, 4 grp + r)][q = col]
                    float4_t st[QB][4];
#pragma unroll
                    for (int kb = 0; kb < 4; ++kb) {
                        const int row = tile_key(kb, col);
                        const half8_t a0 = *reinterpret_cast<const half8_t*>(
                            &s_k[buf][row][8 * (grp ^ (row & 7))]);
                        const half8_t a1 = *reinterpret_cast<const half8_t*>(
                            &s_k[buf][row][8 * ((4 + grp) ^ (row & 7))]);
#pragma unroll
                        for (int qb = 0; qb < QB; ++qb) {
                            float4_t c = {0.f, 0.f, 0.f, 0.f};
                            c = mfma_16x16x32(a0, qh[qb][0], c);
                            c = mfma_16x16x32(a1, qh[qb][1], c);
                            if constexpr (QF32) {
                                c = mfma_16x16x32(a0, ql[qb][0], c);
                                c = mfma_16x16x32(a1, ql[qb][1], c);
                            }
                            st[qb][kb] = c;
                        }
                    }
                    // Mask; a tile that every row of the wave sees whole (below the diagonal,
                    // all rows in the run) needs none.
                    bool lane_full = true;
#pragma unroll
                    for (int qb = 0; qb < QB; ++qb)
                        lane_full = lane_full && in_run[qb] && my_pos[qb] >= kbase + kKeyTile - 1;
                    if (!__all(lane_full)) {
#pragma unroll
                        for (int qb = 0; qb < QB; ++qb)
                            mask_tile(st[qb], in_run[qb] ? my_pos[qb] - kbase - 8 * grp : -1);
                    }
                    half8_t pb[QB][2];
                    half8_t pl[QB][2];  // P = hi + lo: the product keeps ~22 bits of P (not P16)
#pragma unroll
                    for (int qb = 0; qb < QB; ++qb) {
                        const float tm = tile_max(st[qb]) * a.scale_log2;  // base-2 units
                        // Lazy rescale: the running max moves only when the tile's max exceeds
                        // it by more than kLazyLog2, so P stays <= 2^kLazyLog2 and most tiles
                        // skip rescaling the accumulators. out = acc / l is unchanged.
                        const bool grow = tm > m[qb] + kLazyLog2;
                        if (__any(grow)) {
                            // alpha = 1 where the max is kept (also -inf, where m - m is NaN);
                            // 0 where it grows from -inf
                            const float alpha = grow ? fast_exp2(m[qb] - tm) : 1.0f;
                            const float mn = grow ? tm : m[qb];
                            l[qb] *= alpha;
#pragma unroll
                            for (int db = 0; db < 4; ++db) acc[qb][db] = acc[qb][db] * alpha;
                            m[qb] = mn;
                        }
                        const float mu = (m[qb] == -INFINITY) ? 0.0f : m[qb];
                        l[qb] += tile_p<P16>(st[qb], a.scale_log2, mu, pb[qb], pl[qb]);
                    }
                    // O^T[dim][q] += V^T[dim][32 keys] . P^T[32 keys][q], key halves ks = 0, 1
                    // (keys past the run's end were zeroed in LDS above). Keys 32 ks + 8 grp .. +7
                    // of dim d are half grp & 1 of page 2 ks + (grp >> 1), at row position
                    // (grp & 1) ^ (bit 3 of d), one 16-byte read.
#pragma unroll
                    for (int db = 0; db < 4; ++db) {
                        const int d = 16 * db + col;
#pragma unroll
                        for (int ks = 0; ks < 2; ++ks) {
                            const half8_t va = *reinterpret_cast<const half8_t*>(
                                &s_v[buf][0][0] + (2 * ks + (grp >> 1)) * 1024 + d * 16 +
                                8 * ((grp & 1) ^ ((d >> 3) & 1)));
#pragma unroll
                            for (int qb = 0; qb < QB; ++qb) {
                                acc[qb][db] = mfma_16x16x32(va, pb[qb][ks], acc[qb][db]);
                                if constexpr (!P16)
                                    acc[qb][db] = mfma_16x16x32(va, pl[qb][ks], acc[qb][db]);
                            }
                        }
                    }
                }
            }
            // every wave's reads of the last buffers are done before the next run reuses them
            __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0);
            __builtin_amdgcn_s_barrier();
            if (a.mode != kOwners) break;  // a single run
            r0 = r1;
        }

        CRUCIBLE_PSTAMP(kPLoop, CRUCIBLE_PSTAMP_CLOCK());
        // ---- merge the key halves: waves 4..7 hand (m, l, acc) to their partner through
        // the (now idle) ring; per lane, both hold the same query column and dims. Lane-major
        // layout keeps the exchange free of bank conflicts: acc (4 x QB x 16 x 64 floats,
        // 32 KiB at QB = 2) in the K ring, m and l in the V ring.
        static_assert(4 * QB * 16 * 64 * sizeof(float) <= sizeof(s_k), "merge buffer");
        float* s_macc = reinterpret_cast<float*>(&s_k[0][0][0]);
        float* s_ml = reinterpret_cast<float*>(&s_v[0][0][0]);
        if (kh == 1) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                float* p = s_macc + (slot * QB + qb) * 16 * 64 + lane;
#pragma unroll
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int r = 0; r < 4; ++r) p[(4 * db + r) * 64] = acc[qb][db][r];
                float* q = s_ml + (slot * QB + qb) * 2 * 64 + lane;
                q[0] = m[qb];
                q[64] = l[qb];
            }
        }
        __syncthreads();
        if (kh == 0) {
            CRUCIBLE_PSTAMP(kPMerged, CRUCIBLE_PSTAMP_CLOCK());
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                const float* p = s_macc + (slot * QB + qb) * 16 * 64 + lane;
                const float* q = s_ml + (slot * QB + qb) * 2 * 64 + lane;
                const float m1 = q[0], l1 = q[64];
                const float mx = fmaxf(m[qb], m1);
                const float mu = mx == -INFINITY ? 0.0f : mx;
                const float w0 = fast_exp2(m[qb] - mu), w1 = fast_exp2(m1 - mu);
                l[qb] = l[qb] * w0 + l1 * w1;
#pragma unroll
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[qb][db][r] = acc[qb][db][r] * w0 + p[(4 * db + r) * 64] * w1;
            }

            // ---- normalise and write: lane (q = col, grp) holds dims 16*db + 4*grp .. +3
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                const float lt = group_sum4(l[qb]);
                if (my_row[qb] < 0) continue;
                const float inv = 1.0f / lt;
                const int64_t off = (int64_t)my_row[qb] * ld_q + (int64_t)h * kHeadDim + 4 * grp;
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    const float4_t o = acc[qb][db] * inv;
                    if (a.out_f16) {
                        const half4_t hv = {(half_t)o[0], (half_t)o[1], (half_t)o[2], (half_t)o[3]};
                        *reinterpret_cast<half4_t*>(static_cast<half_t*>(a.out) + off +
                                                    16 * db) = hv;
                    } else {
                        *reinterpret_cast<float4_t*>(static_cast<float*>(a.out) + off +
                                                     16 * db) = o;
                    }
                }
            }
#ifdef CRUCIBLE_STAMPS
            CRUCIBLE_PSTAMP_AFTER(kPWritten);
            CRUCIBLE_PSTAMP(kPWait, t_wait);
            CRUCIBLE_PSTAMP(kPMeta, (uint64_t)(wp.tile & 0xffff) |
                                        (uint64_t)(wp.req & 0xffff) << 16 |
                                        (uint64_t)(wp.x & 0xffff) << 32 |
                                        (uint64_t)(stamp_pairs & 0xffff) << 48);
#endif
        }  // kh == 0
        if constexpr (!PERSIST) return;
        // The key-half-1 waves go on to the next tile's rows at once; its first barrier holds
        // them until the key-half-0 waves have read the merge buffers (in the ring) above.
    }  // rounds
}

// ---------------------------------------------------------------- 32-row waves on 32x32 MFMAs
//
// The LDS form with 32 query rows per wave (the QB = 2 shape) on v_mfma_f32_32x32x16_f16:
// the same workgroup (4 slots x 2 key-half waves), LDS ring, page staging and merge as
// prefill_kernel, with the tile's products as 32x32 blocks. A 32x32x16 MFMA holds the
// SIMD's issue port for a smaller share of its cycles than two 16x16x32 ones of the same
// work, so more of the softmax's VALU work fits beside it.
//
// Operand layouts (measured on gfx950): lane L supplies A[m = L & 31][k = 8 (L >> 5) .. +7]
// and B[k = 8 (L >> 5) .. +7][n = L & 31]; result element i of lane L is
// D[m = 8 (i >> 2) + 4 (L >> 5) + (i & 3)][n = L & 31]. Lane L serves query row L & 31 of
// its wave; the half hh = L >> 5 picks which keys (S^T) or dims (O^T) of that row it holds.
//   S^T[32 keys][32 rows] = K[32 keys][64] . Q^T[64][32 rows]     4 MFMAs per 32-key block
//   O^T[32 dims][32 rows] += V^T[32 dims][16 keys] . P^T[16 keys][32 rows]
//                                                    2 dim blocks x 4 16-key steps per tile
typedef float float16v_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float16v_t mfma_32x32x16(half8_t a, half8_t b, float16v_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Key of S^T row m within a 32-key block: m = 8 I + 4 h + r holds key 16 (I >> 1) + 8 h +
// 4 (I & 1) + r. Result element i of a lane in half hh is then key 16 (i >> 3) + 8 hh + (i & 7),
// so elements 8 s .. 8 s + 7 are keys 16 s + 8 hh .. +7: exactly the k range that lane supplies
// to the PV product of 16-key step s, read straight from the accumulator.
__device__ __forceinline__ int key32(int m) {
    return 16 * (m >> 4) + 8 * ((m >> 2) & 1) + 4 * ((m >> 3) & 1) + (m & 3);
}

// Row max of a lane's 32 scores (two 32-key blocks), then over the two halves holding the same
// row (v_permlane32_swap). Two asm blocks (operand count); the first opens with 24 wait states
// for the 32x32 MFMA results it reads, which also covers the second block's inputs.
__device__ __forceinline__ float tile_max32(const float16v_t& s0, const float16v_t& s1) {
    float r, t;
    asm("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\t"
        "v_max3_f32 %0, %1, %2, %3\n\t"
        "v_max3_f32 %0, %0, %4, %5\n\t"
        "v_max3_f32 %0, %0, %6, %7\n\t"
        "v_max3_f32 %0, %0, %8, %9\n\t"
        "v_max3_f32 %0, %0, %10, %11\n\t"
        "v_max3_f32 %0, %0, %12, %13\n\t"
        "v_max3_f32 %0, %0, %14, %15\n\t"
        "v_max_f32 %0, %0, %16"
        : "=&v"(r)
        : "v"(s0[0]), "v"(s0[1]), "v"(s0[2]), "v"(s0[3]), "v"(s0[4]), "v"(s0[5]), "v"(s0[6]),
          "v"(s0[7]), "v"(s0[8]), "v"(s0[9]), "v"(s0[10]), "v"(s0[11]), "v"(s0[12]),
          "v"(s0[13]), "v"(s0[14]), "v"(s0[15]));
    asm("v_max3_f32 %0, %0, %2, %3\n\t"
        "v_max3_f32 %0, %0, %4, %5\n\t"
        "v_max3_f32 %0, %0, %6, %7\n\t"
        "v_max3_f32 %0, %0, %8, %9\n\t"
        "v_max3_f32 %0, %0, %10, %11\n\t"
        "v_max3_f32 %0, %0, %12, %13\n\t"
        "v_max3_f32 %0, %0, %14, %15\n\t"
        "v_max3_f32 %0, %0, %16, %17\n\t"
        "v_mov_b32 %1, %0\n\t"
        "s_nop 1\n\t"
        "v_permlane32_swap_b32 %0, %1\n\t"
        "s_nop 1\n\t"
        "v_max_f32 %0, %0, %1"
        : "+v"(r), "=&v"(t)
        : "v"(s1[0]), "v"(s1[1]), "v"(s1[2]), "v"(s1[3]), "v"(s1[4]), "v"(s1[5]), "v"(s1[6]),
          "v"(s1[7]), "v"(s1[8]), "v"(s1[9]), "v"(s1[10]), "v"(s1[11]), "v"(s1[12]),
          "v"(s1[13]), "v"(s1[14]), "v"(s1[15]));
    return r;
}

// Sum of a value over the two halves holding the same row (lanes L and L ^ 32).
__device__ __forceinline__ float half_sum2(float x) {
    float t;
    asm("s_nop 0\n\t"
        "v_mov_b32 %1, %0\n\t"
        "s_nop 1\n\t"
        "v_permlane32_swap_b32 %0, %1\n\t"
        "s_nop 1\n\t"
        "v_add_f32 %0, %0, %1"
        : "+v"(x), "=&v"(t));
    return x;
}

// P of one 16-key step: p = exp2(s * scale - mu) for accumulator elements 8 s .. +7 of a
// 32-key block, as the B operand of the PV product (one fp16, RNE, under P16; else fp16 hi +
// lo as tile_p). Returns the eight values' sum.
template <bool P16>
__device__ __forceinline__ float step_p32(const float16v_t& st, int s, float scale, float mu,
                                          half8_t& pb, half8_t& pl) {
    typedef float float2_t __attribute__((ext_vector_type(2)));
    typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
    float pf[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) pf[j] = fast_exp2(__builtin_fmaf(st[8 * s + j], scale, -mu));
    u32x4_t hw, lw;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if constexpr (P16) {
            hw[j] = __builtin_bit_cast(
                uint32_t, __builtin_convertvector((float2_t{pf[2 * j], pf[2 * j + 1]}), half2_t));
        } else {
            hw[j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(pf[2 * j], pf[2 * j + 1]));
        }
    }
    if constexpr (!P16) {
        const float lo4[4] = {pf[0], pf[1], pf[2], pf[3]}, hi4[4] = {pf[4], pf[5], pf[6], pf[7]};
        uint32_t a0, a1, b0, b1;
        split_lo4(lo4, hw[0], hw[1], a0, a1);
        split_lo4(hi4, hw[2], hw[3], b0, b1);
        lw = u32x4_t{a0, a1, b0, b1};
        pl = __builtin_bit_cast(half8_t, lw);
    }
    pb = __builtin_bit_cast(half8_t, hw);
    return ((pf[0] + pf[1]) + (pf[2] + pf[3])) + ((pf[4] + pf[5]) + (pf[6] + pf[7]));
}

template <int HPW, bool QF32, int KB, bool P16>
__global__ __launch_bounds__(kThreads) void prefill32_kernel(PrefillArgs a,
                                                        const int32_t* __restrict__ tables) {
    constexpr int RS = 4 / HPW;          // row slices per workgroup
    constexpr int WROWS = 32;            // rows per wave
    constexpr int R = RS * WROWS;        // rows per workgroup

    __shared__ half_t s_k[KB][kKeyTile][64];   // [buf][key][dim], 16-byte chunks swizzled
    __shared__ half_t s_v[KB][64][kKeyTile];   // page-major V^T, as prefill_kernel
    __shared__ int s_owner[R];
    __shared__ int s_pos[R];
    __shared__ int s_row[R];
    __shared__ uint64_t s_mask[2];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int qr = lane & 31;   // the wave's query row this lane serves
    const int hh = lane >> 5;   // which half of the row's keys / dims
    const int kh = wave >> 2;   // key half: tile 2 i + kh of pair i
    const int slot = wave & 3;
    const int rs = slot / HPW;
    const int hi = slot % HPW;

    const WgPos wp = wg_pos(a);
    const int groups_per_kv = a.n_rep / HPW;
    const int g = wp.x / groups_per_kv;
    const int h = g * a.n_rep + (wp.x % groups_per_kv) * HPW + hi;

    // ---- rows of this tile: (packed row, owner, absolute position); -1 = none
    int row = -1, owner = 0, pos = 0;
    if (tid < R) {
        tile_row(a, wp.req, wp.tile * R + tid, row, owner, pos);
        s_row[tid] = row;
        s_owner[tid] = owner;
        s_pos[tid] = pos;
    }
    const uint64_t vmask = __ballot(tid < R && row >= 0);
    if (wave < 2 && lane == 0) s_mask[wave] = vmask;
    __syncthreads();
    const uint64_t mask0 = s_mask[0];
    const uint64_t mask1 = R > 64 ? s_mask[1] : 0;
    if (mask0 == 0 && mask1 == 0) return;  // uniform: no row of this tile is valid

    const int64_t ld_q = (int64_t)a.n_head * kHeadDim;
    const int ri = rs * WROWS + qr;
    const int my_row = s_row[ri];
    const int my_pos = s_pos[ri];
    float m = -INFINITY, l = 0.0f;
    float16v_t acc[2] = {};
    half8_t qh[4] = {}, ql[4] = {};
    // Q^T operand of K step t4: dims 16 t4 + 8 hh .. +7 of this lane's row
    auto load_queries = [&]() {
        if (my_row < 0) return;
        const int64_t off = (int64_t)my_row * ld_q + (int64_t)h * kHeadDim + 8 * hh;
        if constexpr (QF32) {
            const float* qp = static_cast<const float*>(a.q) + off;
#pragma unroll
            for (int t4 = 0; t4 < 4; ++t4)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float x = qp[16 * t4 + j];
                    qh[t4][j] = (half_t)x;
                    ql[t4][j] = (half_t)(x - (float)qh[t4][j]);
                }
        } else {
            const half_t* qp = static_cast<const half_t*>(a.q) + off;
#pragma unroll
            for (int t4 = 0; t4 < 4; ++t4) qh[t4] = *reinterpret_cast<const half8_t*>(qp + 16 * t4);
        }
    };

    const int kv_dim = a.addr.kv_dim;
    typedef const __attribute__((address_space(4))) int32_t* const_i32_ptr;
    const int first_valid = mask0 ? __builtin_ctzll(mask0) : 64 + __builtin_ctzll(mask1);
    const int last_valid = mask1 ? 127 - __builtin_clzll(mask1) : 63 - __builtin_clzll(mask0);
    const int wlo = rs * WROWS, whi = rs * WROWS + WROWS;
    const int my_page = wave >> 1;
    bool first_run = true;
    int r0 = a.mode == kOwners ? 0 : first_valid;
    while (r0 < R) {
        int r1, own, hist_end, wave_last;
        if (a.mode != kOwners) {
            r1 = last_valid + 1;
            own = s_owner[r0];
            hist_end = s_pos[last_valid] + 1;
            const int lo = max(r0, wlo), hi2 = min(r1, whi);
            wave_last = lo < hi2 ? s_pos[hi2 - 1] : -1;
        } else {
            while (r0 < R && s_row[r0] < 0) ++r0;
            if (r0 >= R) break;
            own = s_owner[r0];
            r1 = r0 + 1;
            while (r1 < R && s_row[r1] >= 0 && s_owner[r1] == own) ++r1;
            hist_end = 0;
            for (int r = r0; r < r1; ++r) hist_end = max(hist_end, s_pos[r] + 1);
            wave_last = -1;
            for (int r = max(r0, wlo); r < min(r1, whi); ++r) wave_last = max(wave_last, s_pos[r]);
        }
        r0 = __builtin_amdgcn_readfirstlane(r0);
        r1 = __builtin_amdgcn_readfirstlane(r1);
        own = __builtin_amdgcn_readfirstlane(own);
        hist_end = __builtin_amdgcn_readfirstlane(hist_end);
        wave_last = __builtin_amdgcn_readfirstlane(wave_last);

        const bool paged = tables != nullptr;
        const const_i32_ptr table = paged ? (const_i32_ptr)(tables + (int64_t)own * a.table_stride)
                                          : (const_i32_ptr)a.k_pool;
        const int n_tiles = (hist_end + kKeyTile - 1) / kKeyTile;
        const int last_page = (hist_end - 1) >> kPageShift;
        auto page_of = [&](int t) -> int64_t {
            const int idx = min(4 * t + my_page, last_page);
            const int id = table[paged ? idx : 0];
            return paged ? (int64_t)id : (int64_t)idx;
        };
        // the staging of prefill_kernel: wave w moves K rows 8 (w & 1) .. +7 and V^T dims
        // 32 (w & 1) .. +31 of page w >> 1
        auto issue = [&](int t, int64_t page) {
            const int buf = t % KB;
            const int64_t base = block_base(a.addr, page);
            {
                const int krow = 8 * wave + (lane >> 3);
                const int c = (lane & 7) ^ (krow & 7);
                const half_t* src = a.k_pool + base + (int64_t)(krow & kPageMask) * kv_dim +
                                    g * kHeadDim + 8 * c;
                lds_dma16(src, lds_offset(&s_k[buf][8 * wave][0]));
            }
            {
                const int d = 32 * (wave & 1) + (lane >> 1);
                const int half = (lane & 1) ^ ((d >> 3) & 1);
                const half_t* src = a.v_pool + base +
                                    (int64_t)(g * kHeadDim + d) * kPageTokens + 8 * half;
                lds_dma16(src, lds_offset(&s_v[buf][0][0] + my_page * 1024 + (wave & 1) * 512));
            }
        };

        const bool in_run = my_row >= 0 && ri >= r0 && ri < r1;
        constexpr int PS = KB / 2;
        const int n_pairs = (n_tiles + 1) / 2;
        const int tail_pair = (hist_end % kKeyTile) ? (n_tiles - 1) / 2 : -1;
#pragma unroll
        for (int p = 0; p < PS - 1; ++p)
            if (p < n_pairs) {
                const int64_t pa = page_of(2 * p), pb = page_of(2 * p + 1);
                issue(2 * p, pa);
                issue(2 * p + 1, pb);
            }
        if (first_run) {
            load_queries();
            __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0);
            first_run = false;
        }
        for (int ip = 0; ip < n_pairs; ++ip) {
            const int ahead = min(PS - 2, n_pairs - 1 - ip);
            if (ahead >= 2) __builtin_amdgcn_s_waitcnt(kWaitVm8Lgkm0);
            else if (ahead == 1) __builtin_amdgcn_s_waitcnt(kWaitVm4Lgkm0);
            else __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0);
            if (ip == tail_pair) {
                const int t = n_tiles - 1;
                const int d = 32 * (wave & 1) + (lane >> 1);
                const int half = (lane & 1) ^ ((d >> 3) & 1);
                const int nv = hist_end - (t * kKeyTile + 16 * my_page + 8 * half);
                if (nv < 8) {
                    half8_t* chunk = reinterpret_cast<half8_t*>(
                        &s_v[t % KB][0][0] + my_page * 1024 + (wave & 1) * 512) + lane;
                    half8_t v = *chunk;
#pragma unroll
                    for (int r = 0; r < 8; ++r)
                        if (r >= nv) v[r] = (half_t)0.0f;
                    *chunk = v;
                }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            }
            __builtin_amdgcn_s_barrier();
            if (ip + PS - 1 < n_pairs) {
                const int tn = 2 * (ip + PS - 1);
                const int64_t pa = page_of(tn), pb = page_of(tn + 1);
                issue(tn, pa);
                issue(tn + 1, pb);
            }
            const int t = 2 * ip + kh;
            const int kbase = t * kKeyTile;
            if (t < n_tiles && wave_last >= kbase) {
                const int buf = t % KB;
                // S^T blocks: st[kb2][i] = S^T[kbase + 32 kb2 + 16 (i >> 3) + 8 hh + (i & 7)][qr]
                float16v_t st[2];
#pragma unroll
                for (int kb2 = 0; kb2 < 2; ++kb2) {
                    const int krow = 32 * kb2 + key32(qr);
                    float16v_t c = {};
#pragma unroll
                    for (int t4 = 0; t4 < 4; ++t4) {
                        const half8_t ka = *reinterpret_cast<const half8_t*>(
                            &s_k[buf][krow][8 * ((2 * t4 + hh) ^ (krow & 7))]);
                        c = mfma_32x32x16(ka, qh[t4], c);
                        if constexpr (QF32) c = mfma_32x32x16(ka, ql[t4], c);
                    }
                    st[kb2] = c;
                }
                // causal mask (a tile every row of the wave sees whole needs none): element i
                // of block kb2 is visible iff 32 kb2 + 16 (i >> 3) + (i & 7) <= pos - kbase - 8 hh
                if (!__all(in_run && my_pos >= kbase + kKeyTile - 1)) {
                    const int lim = in_run ? my_pos - kbase - 8 * hh : -1;
#pragma unroll
                    for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
                        for (int i = 0; i < 16; ++i)
                            st[kb2][i] = (32 * kb2 + 16 * (i >> 3) + (i & 7) <= lim) ? st[kb2][i]
                                                                                      : -INFINITY;
                }
                const float tm = tile_max32(st[0], st[1]) * a.scale_log2;  // base-2 units
                // lazy rescale, as prefill_kernel
                const bool grow = tm > m + kLazyLog2;
                if (__any(grow)) {
                    const float alpha = grow ? fast_exp2(m - tm) : 1.0f;
                    const float mn = grow ? tm : m;
                    l *= alpha;
                    acc[0] = acc[0] * alpha;
                    acc[1] = acc[1] * alpha;
                    m = mn;
                }
                const float mu = (m == -INFINITY) ? 0.0f : m;
                // 16-key steps: keys 32 kb2 + 16 s .. +15 are page 2 kb2 + s of the tile; this
                // lane's V^T operand is dims d, keys 8 hh .. +7 of that page, one 16-byte read
#pragma unroll
                for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        half8_t pb, pl;
                        l += step_p32<P16>(st[kb2], s, a.scale_log2, mu, pb, pl);
                        const int pg = 2 * kb2 + s;
#pragma unroll
                        for (int db2 = 0; db2 < 2; ++db2) {
                            const int d = 32 * db2 + qr;
                            const half8_t va = *reinterpret_cast<const half8_t*>(
                                &s_v[buf][0][0] + pg * 1024 + d * 16 + 8 * (hh ^ ((d >> 3) & 1)));
                            acc[db2] = mfma_32x32x16(va, pb, acc[db2]);
                            if constexpr (!P16) acc[db2] = mfma_32x32x16(va, pl, acc[db2]);
                        }
                    }
            }
        }
        __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0);
        __builtin_amdgcn_s_barrier();
        if (a.mode != kOwners) break;
        r0 = r1;
    }

    // ---- merge the key halves through the idle ring: acc (4 slots x 64 lanes x 32 floats,
    // 32 KiB) in the K ring, m and l in the V ring, lane-major
    static_assert(4 * 32 * 64 * sizeof(float) <= sizeof(s_k), "merge buffer");
    float* s_macc = reinterpret_cast<float*>(&s_k[0][0][0]);
    float* s_ml = reinterpret_cast<float*>(&s_v[0][0][0]);
    if (kh == 1) {
        float* p = s_macc + slot * 32 * 64 + lane;
#pragma unroll
        for (int db2 = 0; db2 < 2; ++db2)
#pragma unroll
            for (int i = 0; i < 16; ++i) p[(16 * db2 + i) * 64] = acc[db2][i];
        float* q = s_ml + slot * 2 * 64 + lane;
        q[0] = m;
        q[64] = l;
    }
    __syncthreads();
    if (kh == 1) return;
    {
        const float* p = s_macc + slot * 32 * 64 + lane;
        const float* q = s_ml + slot * 2 * 64 + lane;
        const float m1 = q[0], l1 = q[64];
        const float mx = fmaxf(m, m1);
        const float mu = mx == -INFINITY ? 0.0f : mx;
        const float w0 = fast_exp2(m - mu), w1 = fast_exp2(m1 - mu);
        l = l * w0 + l1 * w1;
#pragma unroll
        for (int db2 = 0; db2 < 2; ++db2)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[db2][i] = acc[db2][i] * w0 + p[(16 * db2 + i) * 64] * w1;
    }

    // ---- normalise and write: element i of block db2 is dim 32 db2 + 8 (i >> 2) + 4 hh + (i & 3)
    const float lt = half_sum2(l);
    if (my_row < 0) return;
    const float inv = 1.0f / lt;
    const int64_t off = (int64_t)my_row * ld_q + (int64_t)h * kHeadDim + 4 * hh;
#pragma unroll
    for (int db2 = 0; db2 < 2; ++db2)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
            const float4_t o = {acc[db2][4 * i4] * inv, acc[db2][4 * i4 + 1] * inv,
                                acc[db2][4 * i4 + 2] * inv, acc[db2][4 * i4 + 3] * inv};
            const int64_t at = off + 32 * db2 + 8 * i4;
            if (a.out_f16) {
                const half4_t hv = {(half_t)o[0], (half_t)o[1], (half_t)o[2], (half_t)o[3]};
                *reinterpret_cast<half4_t*>(static_cast<half_t*>(a.out) + at) = hv;
            } else {
                *reinterpret_cast<float4_t*>(static_cast<float*>(a.out) + at) = o;
            }
        }
}

// ---------------------------------------------------------------- register-direct form
//
// Workgroup = 16 query rows of one head; its 8 waves split the causal key range, wave w
// taking the 64-key tiles w, w + 8, ... Each wave loads its tile's K rows and V^T page
// slices from the pool straight into MFMA operand registers (the decode kernel's operand
// layout): no LDS staging and no barrier per tile, so the longest row block costs one
// tile's chain per wave instead of one per tile. The 8 online-softmax states merge
// through LDS once at the end. K/V tiles are read once per 16-row block (from L2 after
// the first), against once per 64 rows in the LDS form: the direct form trades L2 reads
// for parallelism, which pays while the LDS form's grid would leave CUs idle.
constexpr int kDirectWaves = 8;

// At most 128 VGPRs (4 waves per SIMD): two 8-wave workgroups per CU, so a config-1 grid
// (384 workgroups) is resident at once instead of in two rounds.
// HYB: the hybrid instantiation (keys of the segment's own chunk from cur_k / cur_v); the
// pool-only one carries none of that code (its registers stay within the cap).
template <bool QF32, bool HYB, bool P16>
__global__ __launch_bounds__(kDirectWaves * 64, 4) void prefill_direct_kernel(
    PrefillArgs a, const int32_t* __restrict__ tables) {
    __shared__ int s_owner[16];
    __shared__ int s_pos[16];
    __shared__ int s_row[16];
    __shared__ uint64_t s_mask;
    __shared__ float s_m[kDirectWaves][16];
    __shared__ float s_l[kDirectWaves][16];
    __shared__ float4_t s_acc[kDirectWaves][4][64];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int col = lane & 15;
    const int grp = lane >> 4;
    [[maybe_unused]] const uint64_t t_entry = CRUCIBLE_PSTAMP_CLOCK();
    [[maybe_unused]] const unsigned pstamp_id = pstamp_row();
    const WgPos wp = wg_pos(a);
    const int h = wp.x;
    const int g = h / a.n_rep;

    // Rows of this tile. Outside the OWNERS mode they follow from one uniform descriptor
    // (first row, row count, first position, owner) read through the scalar cache, and
    // the valid rows are one range [lo, hi) of the tile: no LDS round trip, no barrier.
    // OWNERS tiles take their rows from per-row arrays, staged in LDS.
    uint64_t mask;
    int my_row, my_pos, d_owner = 0, d_hist = 0;
    int d_pstart = 0, d_astart = 0;  // the segment's packed_start and absolute_start (hybrid)
    if (a.mode != kOwners) {
        typedef const __attribute__((address_space(4))) int32_t* const_i32_ptr;
        int64_t row0 = 0, len = a.rows, pos0 = a.pos_offset;
        if (a.mode == kSegments) {
            const const_i32_ptr seg = (const_i32_ptr)(a.segments + 4 * wp.req);
            row0 = seg[0];
            len = seg[1];
            pos0 = seg[2];
            d_owner = seg[3];
            d_pstart = (int)row0;
            d_astart = (int)pos0;
        } else if (a.mode == kParams) {
            pos0 = ((const_i32_ptr)a.params)[kParamPrefillPos];
        }
        const int64_t base = wp.tile * 16;
        // local row base + r is valid iff r < len - base and 0 <= pos0 + base + r < max_seq
        const int64_t lo64 = max((int64_t)0, -(pos0 + base));
        const int64_t hi64 = min((int64_t)16, min(len - base, (int64_t)a.max_seq - (pos0 + base)));
        if (lo64 >= hi64) return;  // uniform: no row of this tile is valid
        const int lo = (int)lo64, hi = (int)hi64;
        mask = ((hi == 64 ? 0ull : (1ull << hi)) - 1) & ~((1ull << lo) - 1);
        const bool valid = col >= lo && col < hi;
        my_row = valid ? (int)(row0 + base + col) : -1;
        my_pos = (int)(pos0 + base + (valid ? col : lo));
        d_hist = (int)(pos0 + base + hi);  // one past the last valid row's position
    } else {
        int row = -1, owner = 0, pos = 0;
        if (tid < 16) {
            tile_row(a, wp.req, wp.tile * 16 + tid, row, owner, pos);
            s_row[tid] = row;
            s_owner[tid] = owner;
            s_pos[tid] = pos;
        }
        const uint64_t vmask = __ballot(tid < 16 && row >= 0);
        if (wave == 0 && lane == 0) s_mask = vmask;
        __syncthreads();
        mask = s_mask;
        if (mask == 0) return;  // uniform: no row of this tile is valid
        my_row = s_row[col];
        my_pos = s_pos[col];
    }
    const int64_t ld_q = (int64_t)a.n_head * kHeadDim;
    half8_t qh0 = {}, qh1 = {}, ql0 = {}, ql1 = {};
    if (my_row >= 0) {
        const int64_t off = (int64_t)my_row * ld_q + (int64_t)h * kHeadDim + 8 * grp;
        if constexpr (QF32) {
            const float* qp = static_cast<const float*>(a.q) + off;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x0 = qp[j], x1 = qp[32 + j];
                qh0[j] = (half_t)x0;
                qh1[j] = (half_t)x1;
                ql0[j] = (half_t)(x0 - (float)qh0[j]);
                ql1[j] = (half_t)(x1 - (float)qh1[j]);
            }
        } else {
            const half_t* qp = static_cast<const half_t*>(a.q) + off;
            qh0 = *reinterpret_cast<const half8_t*>(qp);
            qh1 = *reinterpret_cast<const half8_t*>(qp + 32);
        }
    }

    CRUCIBLE_PSTAMP(kPStart, t_entry);
    CRUCIBLE_PSTAMP(kPRows, CRUCIBLE_PSTAMP_CLOCK());
    [[maybe_unused]] bool first_tile_stamp = true;
    [[maybe_unused]] int stamp_tiles = 0;
    float m = -INFINITY, l = 0.0f;
    float4_t acc[4] = {};
    const int kv_dim = a.addr.kv_dim;
    const int first_valid = __builtin_ctzll(mask);
    const int last_valid = 63 - __builtin_clzll(mask);
    int r0 = a.mode == kOwners ? 0 : first_valid;
    while (r0 < 16) {
        int r1, owner_r, hist_end, wave_last;
        if (a.mode != kOwners) {
            r1 = last_valid + 1;
            owner_r = d_owner;
            hist_end = d_hist;
            wave_last = d_hist - 1;
        } else {
            while (r0 < 16 && s_row[r0] < 0) ++r0;
            if (r0 >= 16) break;
            owner_r = s_owner[r0];
            r1 = r0 + 1;
            while (r1 < 16 && s_row[r1] >= 0 && s_owner[r1] == owner_r) ++r1;
            hist_end = 0;
            for (int r = r0; r < r1; ++r) hist_end = max(hist_end, s_pos[r] + 1);
            wave_last = hist_end - 1;
        }
        r0 = __builtin_amdgcn_readfirstlane(r0);
        r1 = __builtin_amdgcn_readfirstlane(r1);
        owner_r = __builtin_amdgcn_readfirstlane(owner_r);
        hist_end = __builtin_amdgcn_readfirstlane(hist_end);
        wave_last = __builtin_amdgcn_readfirstlane(wave_last);
        const bool in_run = my_row >= 0 && col >= r0 && col < r1;

        typedef const __attribute__((address_space(4))) int32_t* const_i32_ptr;
        const_i32_ptr table = tables ? (const_i32_ptr)(tables + (int64_t)owner_r * a.table_stride)
                                     : nullptr;
        const int n_tiles = (hist_end + kKeyTile - 1) / kKeyTile;
        const int last_page = (hist_end - 1) >> kPageShift;
#ifdef CRUCIBLE_STAMPS
        stamp_tiles = max(stamp_tiles, n_tiles);
#endif

        for (int t = wave; t < n_tiles; t += kDirectWaves) {
            const int kbase = t * kKeyTile;
            if (wave_last < kbase) break;  // later tiles lie above the diagonal too
            int64_t pg[4];
            // Hybrid: a page wholly at or past the segment's absolute start holds only chunk
            // keys, which come from current_k/v below; neither its table entry nor the pool
            // is read for it, as in the reference (kernels.cu:2012-2016). Uniform per page.
            bool from_pool[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int idx = min(t * 4 + j, last_page);  // clamped: in bounds, masked later
                from_pool[j] = !HYB || idx * kPageTokens < d_astart;
                pg[j] = from_pool[j] ? block_base(a.addr, table ? (int64_t)table[idx] : (int64_t)idx)
                                     : 0;
            }
            // K operand of key block kb: key 16 kb + col (page kb of the tile), channels
            // 8 grp .. +7 and 32 + 8 grp .. +7; V^T operand of channel 16 db + col: slots
            // 4 grp .. +3 of pages 2 ks and 2 ks + 1 (keys 32 ks + 4 grp .. and +16).
            half8_t ka[4][2] = {};
            half4_t va[4][2][2] = {};
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                if (!from_pool[kb]) continue;
                const half_t* kp = a.k_pool + pg[kb] + (int64_t)col * kv_dim + g * kHeadDim + 8 * grp;
                ka[kb][0] = *reinterpret_cast<const half8_t*>(kp);
                ka[kb][1] = *reinterpret_cast<const half8_t*>(kp + 32);
            }
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf) {
                        if (!from_pool[2 * ks + hf]) continue;
                        const half_t* vp = a.v_pool + pg[2 * ks + hf] +
                                           (int64_t)(g * kHeadDim + 16 * db + col) * kPageTokens +
                                           4 * grp;
                        va[db][ks][hf] = *reinterpret_cast<const half4_t*>(vp);
                    }
            // Hybrid (gpu.rs:1691-1697, kernels.cu:2012-2016): keys at or past the segment's
            // absolute start come from the chunk's own K/V rows (packed row packed_start +
            // pos - absolute_start), rounded to fp16 as the append would store them, in
            // place of the pool's. Only keys before the row tile's last visible one are
            // read, so the rows stay inside the chunk.
            if (HYB && kbase + kKeyTile > d_astart) {
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
                    const int pos = kbase + 16 * kb + col;
                    if (pos >= d_astart && pos < hist_end) {
                        const float* kr = a.cur_k + (int64_t)(d_pstart + pos - d_astart) * kv_dim +
                                          g * kHeadDim + 8 * grp;
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            ka[kb][0][j] = (half_t)kr[j];
                            ka[kb][1][j] = (half_t)kr[32 + j];
                        }
                    }
                }
#pragma unroll
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const int pos = kbase + 32 * ks + 16 * hf + 4 * grp + r;
                                if (pos >= d_astart && pos < hist_end)
                                    va[db][ks][hf][r] = (half_t)a.cur_v[
                                        (int64_t)(d_pstart + pos - d_astart) * kv_dim +
                                        g * kHeadDim + 16 * db + col];
                            }
            }

#ifdef CRUCIBLE_STAMPS
            if (first_tile_stamp) {
                CRUCIBLE_PSTAMP_AFTER_W0(kPFirst);
                first_tile_stamp = false;
            }
#endif
            float4_t st[4];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                float4_t c = {0.f, 0.f, 0.f, 0.f};
                c = mfma_16x16x32(ka[kb][0], qh0, c);
                c = mfma_16x16x32(ka[kb][1], qh1, c);
                if constexpr (QF32) {
                    c = mfma_16x16x32(ka[kb][0], ql0, c);
                    c = mfma_16x16x32(ka[kb][1], ql1, c);
                }
                st[kb] = c;
            }
            if (!__all(in_run && my_pos >= kbase + kKeyTile - 1))
                mask_tile_blocks(st, in_run ? my_pos - kbase - 4 * grp : -1);
            const float tm = tile_max(st) * a.scale_log2;  // base-2 units
            const bool grow = tm > m + kLazyLog2;
            if (__any(grow)) {
                const float alpha = grow ? fast_exp2(m - tm) : 1.0f;
                if (grow) m = tm;
                l *= alpha;
#pragma unroll
                for (int db = 0; db < 4; ++db) acc[db] = acc[db] * alpha;
            }
            const float mu = (m == -INFINITY) ? 0.0f : m;
            half8_t pb[2], pl[2];
            l += tile_p<P16>(st, a.scale_log2, mu, pb, pl);
            if (kbase + kKeyTile > hist_end) {  // the run's last tile: zero keys past its end
#pragma unroll
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        va[db][ks][0] = zero_tail(va[db][ks][0], kbase + 32 * ks + 4 * grp, hist_end);
                        va[db][ks][1] =
                            zero_tail(va[db][ks][1], kbase + 32 * ks + 16 + 4 * grp, hist_end);
                    }
            }
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const half4_t v0 = va[db][ks][0], v1 = va[db][ks][1];
                    const half8_t vv = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                    acc[db] = mfma_16x16x32(vv, pb[ks], acc[db]);
                    if constexpr (!P16) acc[db] = mfma_16x16x32(vv, pl[ks], acc[db]);
                }
        }
        if (a.mode != kOwners) break;  // a single run
        r0 = r1;
    }

    // ---- merge the 8 waves' states (per column: m, l summed over the lane groups)
    l = group_sum4(l);
    CRUCIBLE_PSTAMP_AFTER_W0(kPLoop);
    if (grp == 0) {
        s_m[wave][col] = m;
        s_l[wave][col] = l;
    }
#pragma unroll
    for (int db = 0; db < 4; ++db) s_acc[wave][db][lane] = acc[db];
    __syncthreads();
    CRUCIBLE_PSTAMP(kPMerged, CRUCIBLE_PSTAMP_CLOCK());
#ifdef CRUCIBLE_STAMPS
    CRUCIBLE_PSTAMP(kPWait, 0);
    CRUCIBLE_PSTAMP(kPMeta, (uint64_t)(wp.tile & 0xffff) | (uint64_t)(wp.req & 0xffff) << 16 |
                                (uint64_t)(wp.x & 0xffff) << 32 |
                                (uint64_t)(stamp_tiles & 0xffff) << 48);
#endif
    if (wave >= 4 || my_row < 0) return;
    const int db = wave;  // waves 0..3 each finish one 16-dim block
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDirectWaves; ++w) M = fmaxf(M, s_m[w][col]);
    float L = 0.0f;
    float4_t o = {0.f, 0.f, 0.f, 0.f};
    // Branch-free, so all the LDS reads issue together. A wave whose keys this row cannot
    // see has m = -inf, l = 0 and acc = 0: its weight is 0 and it adds exact zeros (wave
    // 0 holds the row's first key, so M is finite).
#pragma unroll
    for (int w = 0; w < kDirectWaves; ++w) {
        const float wt = fast_exp2(s_m[w][col] - M);
        L += s_l[w][col] * wt;
        o += s_acc[w][db][lane] * wt;
    }
    o = o * (1.0f / L);
    const int64_t off = (int64_t)my_row * ld_q + (int64_t)h * kHeadDim + 16 * db + 4 * grp;
    if (a.out_f16) {
        const half4_t hv = {(half_t)o[0], (half_t)o[1], (half_t)o[2], (half_t)o[3]};
        *reinterpret_cast<half4_t*>(static_cast<half_t*>(a.out) + off) = hv;
    } else {
        *reinterpret_cast<float4_t*>(static_cast<float*>(a.out) + off) = o;
    }
    CRUCIBLE_PSTAMP_AFTER_W0(kPWritten);
}

int heads_per_wg(int n_rep) { return (n_rep % 4 == 0) ? 4 : (n_rep % 2 == 0) ? 2 : 1; }

// Workgroups of `kernel` resident at once on this device (0 if unknown).
int resident_workgroups(const void* kernel, int threads) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return per_cu * device_cu_count();
}

template <int HPW, int QB, bool QF32, bool P16>
void launch_kb(const PrefillArgs& a, int kb, dim3 grid, hipStream_t stream) {
    if (kb == 6) {
        hipLaunchKernelGGL((prefill_kernel<HPW, QB, QF32, 6, P16, false>), grid, dim3(kThreads), 0,
                           stream, a, a.tables);
        return;
    }
    // On request (the tuning key), a longest-first segment grid larger than the resident
    // workgroups runs persistent: the dispatcher hands every id, those of tiles without rows
    // included, to a freed slot on the XCD the id maps to, and each pays a workgroup's
    // launch and its own segment round trip. That pays off when most ids hold no rows (one
    // long prompt packed with many short ones); with few such ids (config 4) the dispatcher's
    // dynamic order is as good and the list costs the first tile about a microsecond, so
    // the default stays the one-workgroup-per-id grid.
    auto persistent = prefill_kernel<HPW, QB, QF32, 4, P16, true>;
    static std::atomic<int> resident{-1};  // per instantiation; the same device type throughout
    const int mode = tuning(CRUCIBLE_TUNE_PREFILL_PERSIST);  // 1: resident; n >= 2: n
    if (a.heavy_first && a.mode == kSegments && a.grid_reqs <= 64 && a.grid_tiles <= 64 &&
        mode > 0) {
        int r = mode >= 2 ? mode : resident.load(std::memory_order_relaxed);
        if (r < 0) {
            r = resident_workgroups(reinterpret_cast<const void*>(persistent), kThreads);
            resident.store(r, std::memory_order_relaxed);
        }
        if (r > 0 && grid.x > (unsigned)r) {
            hipLaunchKernelGGL(persistent, dim3((unsigned)r), dim3(kThreads), 0, stream, a,
                               a.tables);
            return;
        }
    }
    hipLaunchKernelGGL((prefill_kernel<HPW, QB, QF32, 4, P16, false>), grid, dim3(kThreads), 0,
                       stream, a, a.tables);
}

// ---------------------------------------------------------------- head_dim other than 64
// One workgroup per (query head, request) walks the request's rows (grid y, strided) through
// attend_generic (generic_attend.hpp): each row attends to keys [0, pos] of its owner, read
// through the same row modes (tile_row) and, for hybrid segments, the chunk's own K/V rows
// from the segment's absolute start.
template <bool QF32>
__global__ __launch_bounds__(kGenericThreads) void prefill_generic_kernel(PrefillArgs a, int hd,
                                                                          int64_t rows_y) {
    __shared__ GenericLds lds;
    const int h = blockIdx.x;
    const int64_t req = blockIdx.z;
    const int64_t stride = (int64_t)a.n_head * hd;
    GenericKeys ks{};
    ks.k_pool = a.k_pool;
    ks.v_pool = a.v_pool;
    ks.addr = a.addr;
    ks.g = h / a.n_rep;
    ks.hd = hd;
    ks.astart = INT32_MAX;
    if (a.hybrid && a.mode == kSegments) {
        const int32_t* seg = a.segments + 4 * req;
        ks.pstart = seg[0];
        ks.astart = seg[2];
        ks.cur_k = a.cur_k;
        ks.cur_v = a.cur_v;
    }
    for (int64_t local = blockIdx.y; local < rows_y; local += gridDim.y) {
        int row, owner, pos;
        tile_row(a, req, local, row, owner, pos);
        if (row < 0) continue;  // uniform: the same row for the whole workgroup
        const int64_t qoff = (int64_t)row * stride + (int64_t)h * hd;
        for (int d = threadIdx.x; d < hd; d += kGenericThreads)
            lds.q[d] = QF32 ? static_cast<const float*>(a.q)[qoff + d]
                            : (float)static_cast<const half_t*>(a.q)[qoff + d];
        __syncthreads();
        ks.table = a.tables ? a.tables + (int64_t)owner * a.table_stride : nullptr;
        attend_generic(lds, ks, pos + 1, a.scale_log2, [&](int d, float v) {
            if (a.out_f16)
                static_cast<half_t*>(a.out)[qoff + d] = (half_t)v;
            else
                static_cast<float*>(a.out)[qoff + d] = v;
        });
    }
}

int launch_prefill_generic(PrefillArgs a, int hd, int64_t tile_rows_total, int64_t z, bool q_f32,
                           hipStream_t stream, const char* what) {
    CRUCIBLE_CHECK(a.n_head <= INT32_MAX && z <= 65535, CRUCIBLE_ERR_INVALID,
                   "%s: grid too large", what);
    CRUCIBLE_CHECK(((uintptr_t)a.k_pool & 15) == 0 && ((uintptr_t)a.v_pool & 15) == 0,
                   CRUCIBLE_ERR_INVALID, "%s: pools must be 16-byte aligned", what);
    a.scale_log2 = (float)(1.4426950408889634 / std::sqrt((double)hd));
    const dim3 grid((unsigned)a.n_head, (unsigned)std::min<int64_t>(tile_rows_total, 65535),
                    (unsigned)z);
    if (q_f32)
        hipLaunchKernelGGL(prefill_generic_kernel<true>, grid, dim3(kGenericThreads), 0, stream, a,
                           hd, tile_rows_total);
    else
        hipLaunchKernelGGL(prefill_generic_kernel<false>, grid, dim3(kGenericThreads), 0, stream,
                           a, hd, tile_rows_total);
    return fail_launch(what);
}

template <int HPW, bool QF32, bool P16>
void launch_kb32(const PrefillArgs& a, int kb, dim3 grid, hipStream_t stream) {
    if (kb == 6)
        hipLaunchKernelGGL((prefill32_kernel<HPW, QF32, 6, P16>), grid, dim3(kThreads), 0, stream,
                           a, a.tables);
    else
        hipLaunchKernelGGL((prefill32_kernel<HPW, QF32, 4, P16>), grid, dim3(kThreads), 0, stream,
                           a, a.tables);
}

template <int HPW, int QB>
void launch_hq(const PrefillArgs& a, bool q_f32, bool p16, int kb, dim3 grid,
               hipStream_t stream) {
    // 32 rows per wave: the 32x32-MFMA kernel unless CRUCIBLE_TUNE_PREFILL_M32 = 0
    if (QB == 2 && tuning(CRUCIBLE_TUNE_PREFILL_M32) != 0) {
        if (q_f32) {
            if (p16) launch_kb32<HPW, true, true>(a, kb, grid, stream);
            else launch_kb32<HPW, true, false>(a, kb, grid, stream);
        } else {
            if (p16) launch_kb32<HPW, false, true>(a, kb, grid, stream);
            else launch_kb32<HPW, false, false>(a, kb, grid, stream);
        }
        return;
    }
    if (q_f32) {
        if (p16) launch_kb<HPW, QB, true, true>(a, kb, grid, stream);
        else launch_kb<HPW, QB, true, false>(a, kb, grid, stream);
    } else {
        if (p16) launch_kb<HPW, QB, false, true>(a, kb, grid, stream);
        else launch_kb<HPW, QB, false, false>(a, kb, grid, stream);
    }
}

// tile_rows_total: rows spanned by grid.y (max_chunk or rows); z: requests.
// The LDS form's grid for these rows: (kv-head groups, row tiles of 64 * QB / HPW rows, z).
struct LdsGrid {
    int hpw, qb;
    int64_t gx, gy;
};

LdsGrid lds_grid(const PrefillArgs& a, int64_t tile_rows_total, int64_t z) {
    LdsGrid lg;
    lg.hpw = heads_per_wg(a.n_rep);
    lg.gx = (int64_t)a.n_kv_head * (a.n_rep / lg.hpw);
    const int rs = 4 / lg.hpw;
    auto tiles = [&](int qb) { return (tile_rows_total + rs * 16 * qb - 1) / (rs * 16 * qb); };
    lg.qb = (lg.gx * tiles(2) * z * 4 >= 2048) ? 2 : 1;
    if (const int v = tuning(CRUCIBLE_TUNE_PREFILL_QB); v > 0) lg.qb = v;
    lg.gy = tiles(lg.qb);
    return lg;
}


int launch_prefill(const PrefillArgs& a_in, int64_t tile_rows_total, int64_t z, bool q_f32,
                   hipStream_t stream, const char* what) {
    PrefillArgs a = a_in;
    // Longest-first for the LDS form, whose grids exceed the resident workgroups (config 4:
    // 16.5 -> 13.3 us); the direct form's grid fits the chip and keeps the plain order
    // (config 1: 7.9 against 8.2 us longest-first).
    const int heavy = tuning(CRUCIBLE_TUNE_PREFILL_HEAVY_FIRST);  // -1: by form
    // (x, row tiles, requests) as the chosen order lays them out
    auto make_grid = [&](int64_t gx, int64_t gy, bool lds_form) {
        const int64_t n = gx * gy * z;
        a.heavy_first = (heavy < 0 ? lds_form : heavy != 0) && n <= INT32_MAX;
        a.grid_x = (int)gx;
        a.grid_tiles = (int)gy;
        a.grid_reqs = (int)z;
        return a.heavy_first ? dim3((unsigned)n) : dim3((unsigned)gx, (unsigned)gy, (unsigned)z);
    };
    const LdsGrid lg = lds_grid(a, tile_rows_total, z);
    // Precision of P in the PV product: fp16 hi + lo (about 22 bits, the default: the
    // reference validator's element gate holds unwidened) or one fp16 operand (P16, when the
    // tuning key asks for it: one PV product per block instead of two).
    const bool p16 = tuning(CRUCIBLE_TUNE_PREFILL_P16) == 1;
    // The register-direct form when the LDS form would leave CUs without a workgroup
    // (short prompts: config 1 is 96 workgroups); the LDS form, which reads each K/V tile
    // once per 64 rows instead of once per 16, when its grid fills the chip.
    int direct = lg.gx * lg.gy * z < device_cu_count();
    if (const int v = tuning(CRUCIBLE_TUNE_PREFILL_DIRECT); v >= 0) direct = v;
    if (a.hybrid) direct = 1;  // the chunk's own K/V rows: register-direct form only
    if (direct) {
        const int64_t gy = (tile_rows_total + 15) / 16;
        CRUCIBLE_CHECK(a.n_head <= INT32_MAX && gy <= 65535 && z <= 65535, CRUCIBLE_ERR_INVALID,
                       "%s: grid (%d, %lld, %lld) too large", what, a.n_head, (long long)gy,
                       (long long)z);
        const dim3 grid = make_grid(a.n_head, gy, false);
        auto go = [&](auto qf, auto hyb) {
            if (p16)
                hipLaunchKernelGGL(
                    (prefill_direct_kernel<decltype(qf)::value, decltype(hyb)::value, true>), grid,
                    dim3(kDirectWaves * 64), 0, stream, a, a.tables);
            else
                hipLaunchKernelGGL(
                    (prefill_direct_kernel<decltype(qf)::value, decltype(hyb)::value, false>), grid,
                    dim3(kDirectWaves * 64), 0, stream, a, a.tables);
        };
        if (q_f32) {
            if (a.hybrid) go(std::true_type{}, std::true_type{});
            else go(std::true_type{}, std::false_type{});
        } else {
            if (a.hybrid) go(std::false_type{}, std::true_type{});
            else go(std::false_type{}, std::false_type{});
        }
        return fail_launch(what);
    }
    const int hpw = lg.hpw, qb = lg.qb;
    const int64_t gx = lg.gx, gy = lg.gy;
    // A grid that fits the chip at one workgroup per CU affords the deeper ring (96 KiB
    // of LDS); larger grids keep two workgroups per CU.
    int kb = (gx * gy * z <= 256) ? 6 : 4;
    if (const int v = tuning(CRUCIBLE_TUNE_PREFILL_BUFS); v > 0) kb = v;
    CRUCIBLE_CHECK(gx <= INT32_MAX && gy <= 65535 && z <= 65535, CRUCIBLE_ERR_INVALID,
                   "%s: grid (%lld, %lld, %lld) too large", what, (long long)gx, (long long)gy,
                   (long long)z);
    const dim3 grid = make_grid(gx, gy, true);
    if (hpw == 4) {
        if (qb == 2) launch_hq<4, 2>(a, q_f32, p16, kb, grid, stream);
        else launch_hq<4, 1>(a, q_f32, p16, kb, grid, stream);
    } else if (hpw == 2) {
        if (qb == 2) launch_hq<2, 2>(a, q_f32, p16, kb, grid, stream);
        else launch_hq<2, 1>(a, q_f32, p16, kb, grid, stream);
    } else {
        if (qb == 2) launch_hq<1, 2>(a, q_f32, p16, kb, grid, stream);
        else launch_hq<1, 1>(a, q_f32, p16, kb, grid, stream);
    }
    return fail_launch(what);
}

int check_prefill(const char* what, int q_dtype, int out_dtype, int64_t n_head,
                  int64_t n_kv_head, int64_t head_dim, int64_t kv_dim) {
    CRUCIBLE_CHECK(dtype_ok(q_dtype) && dtype_ok(out_dtype), CRUCIBLE_ERR_INVALID,
                   "%s: bad dtype", what);
    CRUCIBLE_CHECK(n_head > 0 && n_kv_head > 0 && n_head % n_kv_head == 0, CRUCIBLE_ERR_INVALID,
                   "%s: n_head %lld must be a positive multiple of n_kv_head %lld", what,
                   (long long)n_head, (long long)n_kv_head);
    // before any product of the head counts: n_kv_head <= n_head <= 2^20 from here on
    CRUCIBLE_CHECK(n_head <= (1 << 20), CRUCIBLE_ERR_INVALID, "%s: n_head too large", what);
    CRUCIBLE_CHECK(head_dim == kHeadDim || generic_head_dim_ok(head_dim),
                   CRUCIBLE_ERR_UNSUPPORTED,
                   "%s: head_dim %lld unsupported (a multiple of 8 up to %d)", what,
                   (long long)head_dim, kGenericMaxHeadDim);
    CRUCIBLE_CHECK(kv_dim == n_kv_head * head_dim, CRUCIBLE_ERR_INVALID,
                   "%s: kv_dim %lld != n_kv_head * head_dim", what, (long long)kv_dim);
    return CRUCIBLE_OK;
}

PrefillArgs base_args(const void* q, const void* k_pool, const void* v_pool, void* out,
                      int out_dtype, int64_t n_head, int64_t n_kv_head, int64_t kv_dim,
                      int64_t max_seq) {
    PrefillArgs a{};
    a.q = q;
    a.k_pool = static_cast<const half_t*>(k_pool);
    a.v_pool = static_cast<const half_t*>(v_pool);
    a.out = out;
    a.addr.kv_dim = (int32_t)kv_dim;
    a.n_head = (int)n_head;
    a.n_kv_head = (int)n_kv_head;
    a.n_rep = (int)(n_head / n_kv_head);
    a.max_seq = (int)max_seq;
    a.out_f16 = out_dtype == CRUCIBLE_F16;
    a.scale_log2 = 0.125f * kLog2e;
    return a;
}

}  // namespace
}  // namespace crucible

using namespace crucible;

extern "C" int crucible_attention_prefill_paged(const void* q, int q_dtype, const void* k_pool,
                                                const void* v_pool, void* out, int out_dtype,
                                                const int32_t* page_table, int64_t rows,
                                                int64_t n_head, int64_t n_kv_head,
                                                int64_t head_dim, int64_t n_layer, int64_t layer,
                                                int64_t kv_dim, int64_t max_seq,
                                                const int32_t* params, crucible_stream_t stream) {
    const char* what = "attention_prefill_paged";
    if (int rc = check_prefill(what, q_dtype, out_dtype, n_head, n_kv_head, head_dim, kv_dim))
        return rc;
    CRUCIBLE_CHECK(rows >= 0 && rows <= INT32_MAX, CRUCIBLE_ERR_INVALID, "%s: rows", what);
    if (rows == 0) return CRUCIBLE_OK;
    CRUCIBLE_CHECK(q && k_pool && v_pool && out && page_table && params, CRUCIBLE_ERR_INVALID,
                   "%s: null buffer", what);
    CRUCIBLE_CHECK(n_layer > 0 && layer >= 0 && layer < n_layer, CRUCIBLE_ERR_INVALID,
                   "%s: layer %lld outside n_layer %lld", what, (long long)layer,
                   (long long)n_layer);
    CRUCIBLE_CHECK(max_seq > 0 && max_seq <= INT32_MAX, CRUCIBLE_ERR_INVALID, "%s: max_seq",
                   what);
    PrefillArgs a = base_args(q, k_pool, v_pool, out, out_dtype, n_head, n_kv_head, kv_dim, max_seq);
    a.mode = kParams;
    a.tables = page_table;
    a.params = params;
    a.rows = rows;
    CRUCIBLE_CHECK(paged_addr(n_layer, layer, kv_dim, a.addr), CRUCIBLE_ERR_INVALID,
                   "%s: page geometry of %lld layers x %lld channels overflows", what,
                   (long long)n_layer, (long long)kv_dim);
    if (head_dim != kHeadDim)
        return launch_prefill_generic(a, (int)head_dim, rows, 1, q_dtype == CRUCIBLE_F32, stream,
                                      what);
    return launch_prefill(a, rows, 1, q_dtype == CRUCIBLE_F32, stream, what);
}

extern "C" int crucible_attention_prefill_packed(
    const void* q, int q_dtype, const void* k_pool, const void* v_pool, void* out, int out_dtype,
    const int32_t* tables, const int32_t* owners, const int32_t* positions, int64_t rows,
    int64_t table_stride, int64_t n_head, int64_t n_kv_head, int64_t head_dim, int64_t n_layer,
    int64_t layer, int64_t kv_dim, int64_t max_seq, crucible_stream_t stream) {
    const char* what = "attention_prefill_packed";
    if (int rc = check_prefill(what, q_dtype, out_dtype, n_head, n_kv_head, head_dim, kv_dim))
        return rc;
    CRUCIBLE_CHECK(rows >= 0 && rows <= INT32_MAX, CRUCIBLE_ERR_INVALID, "%s: rows", what);
    if (rows == 0) return CRUCIBLE_OK;
    CRUCIBLE_CHECK(q && k_pool && v_pool && out && tables && owners && positions,
                   CRUCIBLE_ERR_INVALID, "%s: null buffer", what);
    CRUCIBLE_CHECK(n_layer > 0 && layer >= 0 && layer < n_layer, CRUCIBLE_ERR_INVALID,
                   "%s: layer %lld outside n_layer %lld", what, (long long)layer,
                   (long long)n_layer);
    CRUCIBLE_CHECK(table_stride > 0 && table_stride <= INT32_MAX && max_seq > 0 &&
                       max_seq <= table_stride * kPageTokens && max_seq <= INT32_MAX,
                   CRUCIBLE_ERR_INVALID, "%s: max_seq %lld must be in 1..table_stride*16", what,
                   (long long)max_seq);
    PrefillArgs a = base_args(q, k_pool, v_pool, out, out_dtype, n_head, n_kv_head, kv_dim, max_seq);
    a.mode = kOwners;
    a.tables = tables;
    a.owners = owners;
    a.positions = positions;
    a.rows = rows;
    a.table_stride = table_stride;
    CRUCIBLE_CHECK(paged_addr(n_layer, layer, kv_dim, a.addr), CRUCIBLE_ERR_INVALID,
                   "%s: page geometry of %lld layers x %lld channels overflows", what,
                   (long long)n_layer, (long long)kv_dim);
    if (head_dim != kHeadDim)
        return launch_prefill_generic(a, (int)head_dim, rows, 1, q_dtype == CRUCIBLE_F32, stream,
                                      what);
    return launch_prefill(a, rows, 1, q_dtype == CRUCIBLE_F32, stream, what);
}

extern "C" int crucible_attention_prefill_tiled(
    const void* q, int q_dtype, const void* k_pool, const void* v_pool, const void* current_k,
    const void* current_v, void* out, int out_dtype, const int32_t* tables,
    const int32_t* segments, int64_t requests, int64_t max_chunk, int64_t table_stride,
    int64_t n_head, int64_t n_kv_head, int64_t head_dim, int64_t n_layer, int64_t layer,
    int64_t kv_dim, int hybrid, int64_t score_capacity, crucible_stream_t stream) {
    const char* what = "attention_prefill_tiled";
    if (int rc = check_prefill(what, q_dtype, out_dtype, n_head, n_kv_head, head_dim, kv_dim))
        return rc;
    CRUCIBLE_CHECK(!hybrid || (current_k && current_v), CRUCIBLE_ERR_INVALID,
                   "%s: hybrid needs the chunk's current K/V rows", what);
    // Launch checks of gpu.rs:1680-1719.
    CRUCIBLE_CHECK(requests > 0 && max_chunk > 0 && max_chunk <= INT32_MAX && table_stride > 0 &&
                       table_stride <= INT32_MAX / kPageTokens && n_layer > 0 && layer >= 0 &&
                       layer < n_layer && requests <= 65535,
                   CRUCIBLE_ERR_INVALID, "%s: invalid launch dimensions", what);
    CRUCIBLE_CHECK(q && k_pool && v_pool && out && tables && segments, CRUCIBLE_ERR_INVALID,
                   "%s: null buffer", what);
    CRUCIBLE_CHECK(score_capacity >= 0 && score_capacity <= table_stride * kPageTokens,
                   CRUCIBLE_ERR_INVALID, "%s: score capacity exceeds the page table", what);
    const int64_t max_seq = table_stride * kPageTokens;
    CRUCIBLE_CHECK(max_seq <= INT32_MAX, CRUCIBLE_ERR_INVALID, "%s: table too large", what);
    PrefillArgs a = base_args(q, k_pool, v_pool, out, out_dtype, n_head, n_kv_head, kv_dim, max_seq);
    a.mode = kSegments;
    a.tables = tables;
    a.segments = segments;
    a.table_stride = table_stride;
    CRUCIBLE_CHECK(paged_addr(n_layer, layer, kv_dim, a.addr), CRUCIBLE_ERR_INVALID,
                   "%s: page geometry of %lld layers x %lld channels overflows", what,
                   (long long)n_layer, (long long)kv_dim);
    a.hybrid = hybrid != 0;
    a.cur_k = static_cast<const float*>(current_k);
    a.cur_v = static_cast<const float*>(current_v);
    if (head_dim != kHeadDim)
        return launch_prefill_generic(a, (int)head_dim, max_chunk, requests,
                                      q_dtype == CRUCIBLE_F32, stream, what);
    return launch_prefill(a, max_chunk, requests, q_dtype == CRUCIBLE_F32, stream, what);
}

extern "C" int crucible_attention_prefill(const void* q, int q_dtype, const void* k_cache,
                                          const void* v_cache, void* out, int out_dtype,
                                          int64_t rows, int64_t n_head, int64_t n_kv_head,
                                          int64_t head_dim, int64_t max_seq,
                                          int64_t cache_stride, int64_t layer_base,
                                          int64_t pos_offset, crucible_stream_t stream) {
    const char* what = "attention_prefill";
    if (int rc = check_prefill(what, q_dtype, out_dtype, n_head, n_kv_head, head_dim,
                               cache_stride))
        return rc;
    CRUCIBLE_CHECK(rows >= 0 && rows <= INT32_MAX, CRUCIBLE_ERR_INVALID, "%s: rows", what);
    if (rows == 0) return CRUCIBLE_OK;
    CRUCIBLE_CHECK(q && k_cache && v_cache && out, CRUCIBLE_ERR_INVALID, "%s: null buffer", what);
    CRUCIBLE_CHECK(max_seq > 0 && max_seq <= INT32_MAX && pos_offset >= 0 &&
                       pos_offset <= max_seq && rows <= max_seq - pos_offset,
                   CRUCIBLE_ERR_INVALID, "%s: rows past max_seq", what);
    // the last position's element index, layer_base + max_seq * cache_stride, fits int64
    // (max_seq * cache_stride < 2^59 after the checks above)
    CRUCIBLE_CHECK(layer_base >= 0 && layer_base <= INT64_MAX - max_seq * cache_stride,
                   CRUCIBLE_ERR_INVALID, "%s: layer_base %lld", what, (long long)layer_base);
    PrefillArgs a = base_args(q, k_cache, v_cache, out, out_dtype, n_head, n_kv_head,
                              cache_stride, max_seq);
    a.mode = kContig;
    a.rows = rows;
    a.pos_offset = pos_offset;
    a.addr.page_stride = kPageTokens * cache_stride;
    a.addr.layer_off = layer_base;
    if (head_dim != kHeadDim)
        return launch_prefill_generic(a, (int)head_dim, rows, 1, q_dtype == CRUCIBLE_F32, stream,
                                      what);
    return launch_prefill(a, rows, 1, q_dtype == CRUCIBLE_F32, stream, what);
}

#ifdef CRUCIBLE_STAMPS
// Diagnostic build only: copy the first `rows` rows of the 16-row prefill kernel's phase
// stamps (*slots u64 each, in PStampSlot order) to `host`, then zero them on the device if
// `clear`. The clock's rate in kHz goes to *clock_khz. Synchronous.
extern "C" int crucible_debug_prefill_stamps(uint64_t* host, int64_t rows, int clear,
                                             int* clock_khz, int* slots) {
    using namespace crucible;
    const char* what = "crucible_debug_prefill_stamps";
    CRUCIBLE_CHECK(rows >= 0 && rows <= kPStampRows && (rows == 0 || host) && clock_khz && slots,
                   CRUCIBLE_ERR_INVALID, "%s: %lld rows (at most %d)", what, (long long)rows,
                   kPStampRows);
    *slots = kPSlots;
    int dev = 0;
    void* p = nullptr;
    const size_t bytes = (size_t)rows * kPSlots * sizeof(uint64_t);
    const bool ok =
        hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(clock_khz, hipDeviceAttributeWallClockRate, dev) == hipSuccess &&
        hipDeviceSynchronize() == hipSuccess &&
        (rows == 0 || hipMemcpyFromSymbol(host, HIP_SYMBOL(g_prefill_stamps), bytes, 0,
                                          hipMemcpyDeviceToHost) == hipSuccess) &&
        (!clear || (hipGetSymbolAddress(&p, HIP_SYMBOL(g_prefill_stamps)) == hipSuccess &&
                    hipMemset(p, 0, sizeof(g_prefill_stamps)) == hipSuccess &&
                    hipDeviceSynchronize() == hipSuccess));
    CRUCIBLE_CHECK(ok, CRUCIBLE_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(hipGetLastError()));
    return CRUCIBLE_OK;
}
#endif
