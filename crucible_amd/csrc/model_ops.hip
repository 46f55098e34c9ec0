// Decode-step kernels around the attention path: the batched projections, RMSNorm and
// RoPE of the reference decoder (engine/src/model.rs:183-299, forward_cached), with the
// reference CPU arithmetic:
//   matvec (ops.rs:17-32): f32 operands, every product and the sum in f64, one rounding
//     to f32 at the end. The products and sums run here on the f64 MFMA
//     (v_mfma_f64_16x16x4f64) in another order; the sum stays f64, so the rounded f32
//     result is the reference's unless the two f64 sums straddle an f32 rounding
//     boundary.
//   rmsnorm (ops.rs:39-52): f64 mean of squares, scale = 1 / sqrt(mean + eps) in f64,
//     h = f32(f64(x) * scale) * w.
//   silu (ops.rs:83-85) on the gate, times up (model.rs:257-260).
//   RoPE (ops.rs:94-136): element i pairs with i + 32: lo*c - hi*s, lo*s + hi*c.
// These replace the batched GEMV and the row kernels of the reference's GPU decode step
// (kernels.cu:1539-1607 gemv_batch, :968-1047 rmsnorm/rope/swiglu batch kernels), which
// accumulate in f32; keeping the CPU reference's f64 accumulation is what makes greedy
// decoding token-identical to it.
//
// Floating-point contraction is off in this file, so each f32 operation rounds on its own
// as the reference's do.
#include "common.hpp"

#include <algorithm>
#include <cstdlib>
#include <cmath>
#include <type_traits>

#pragma clang fp contract(off)

namespace crucible {
namespace {

typedef double double4_t __attribute__((ext_vector_type(4)));

constexpr int kLinWaves = 8;               // the K range is split over the 8 waves
constexpr int kLinThreads = 64 * kLinWaves;
constexpr int kLinK = 32;                  // K per chunk: 8 per lane group, 8 MFMA steps
constexpr int kLinBatch = 8;               // chunks whose loads are in flight together
                                           // (1 for the 4-block tiles: registers, occupancy)
constexpr int kNormRegChunks = 4;          // fused-norm rows with at most this many chunks
                                           // per wave take their sums of squares from the
                                           // operand registers (no separate pass); 3 for
                                           // the 4-block tiles (registers, occupancy)

enum LinMode { kPlain = 0, kResidual = 1, kSwiGLU = 2 };

__device__ __forceinline__ double4_t mfma_f64(double a, double b, double4_t c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

struct LinArgs {
    const float* x;
    int64_t ldx;
    const float* norm_w;  // fused RMSNorm weight, or nullptr
    double eps;
    const half_t* w;      // [n_out][k_in]; the gate rows in SwiGLU mode
    const half_t* w2;     // SwiGLU: the up rows
    const float* resid;   // kResidual: out = resid + y
    float* out;
    int64_t ldo;
    int rows;
    int n_out;
    int k_in;
    const unsigned char* pf;  // read-only bytes the next kernel will read (or nullptr)
    int64_t pf_bytes;         // their length; whole 64-byte lines are fetched
    int pf_per;               // 64-byte lines a workgroup fetches (set by the launcher)
};

// ---------------------------------------------------------------- next-kernel prefetch
//
// A decode step's projections are short kernels, each waiting once for a cold HBM round
// trip of its weights (the step streams more bytes than the last-level cache holds, so
// they are evicted between steps). Given the next kernel's read-only operands (pf: the
// next projection's weights), each workgroup loads one 4-byte word of every 64-byte line
// of its share of them, right after it has issued its own loads, so that those lines are
// in the last-level cache when the next kernel asks. A wave's loads complete in issue
// order, so no wait for the wave's own operands (issued earlier) waits for these; the words
// are consumed by an empty asm statement at the kernel's end, which is the only wait for
// them. The loads are buffer loads whose range check drops the lines outside the
// workgroup's share (and all of them when there is no prefetch): no branch around them,
// so the compiler's count of the loads in flight stays exact.
constexpr int kPfPerThread = 4;  // at most 4 x 512 lines (128 KB) a workgroup

struct Prefetch {
    uint32_t v[kPfPerThread];
};

template <int THREADS>
__device__ __forceinline__ Prefetch prefetch_issue(const LinArgs& a) {
    const int64_t lines = a.pf_bytes >> 6;
    const int64_t l0 = ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * a.pf_per;
    int64_t n = lines - l0 < a.pf_per ? lines - l0 : a.pf_per;  // this workgroup's lines
    n = n < 0 ? 0 : n;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(a.pf + (n > 0 ? l0 * 64 : 0), (uint32_t)(n * 64));
    Prefetch p;
#pragma unroll
    for (int i = 0; i < kPfPerThread; ++i)
        p.v[i] = __builtin_amdgcn_raw_buffer_load_b32(
            r, (uint32_t)(threadIdx.x + i * THREADS) * 64u, 0, 0);
    return p;
}

__device__ __forceinline__ void prefetch_retire(const Prefetch& p) {
#pragma unroll
    for (int i = 0; i < kPfPerThread; ++i) asm volatile("" ::"v"(p.v[i]));
}

template <int NB>
struct Chunk {
    float4_t x0, x1;
    half8_t w[NB];
    float4_t n0, n1;  // fused-norm weights of the chunk's 8 k (loaded under NORM only)
};

// out tile = 16 rows x (16 * NB) columns. kSwiGLU (NB = 1): 8 output columns, whose gate
// rows fill MFMA columns 0..7 and whose up rows fill columns 8..15, so one 16-wide tile
// carries both halves of SwiGLU at the cost of 8 columns of work.
//
// f64 MFMA 16x16x4 operand layout: lane l supplies A[l & 15][kslot] and B[kslot][l & 15]
// with kslot = l >> 4, and holds D[(l >> 4) + 4 r][l & 15], r = 0..3. Lane group g
// (= l >> 4) owns k = kbeg + k0 + 8 g + j of each 32-wide chunk at MFMA step j, for A
// (the activations) and B (the weights) alike.
template <bool NORM, int MODE, int NB>
__global__ __launch_bounds__(kLinThreads) void linear_kernel(LinArgs a) {
    __shared__ double s_scale[16];
    __shared__ double s_ss[kLinWaves][16];          // per-wave sums of squares by row
    __shared__ double s_red[kLinWaves][NB][4][64];  // [wave][block][r][lane]

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int col = lane & 15;
    const int g = lane >> 4;
    const int m0 = blockIdx.y * 16;
    static_assert(MODE != kSwiGLU || NB == 1, "SwiGLU tiles are one 16-column block");
    const int n0 = blockIdx.x * (MODE == kSwiGLU ? 8 : 16 * NB);
    const int nc = a.k_in / kLinK;  // 32-wide chunks of the K range
    // Short rows (every wave holds at most RC chunks) take the norm's sums of squares
    // from the operand registers; longer ones make a separate pass first.
    constexpr int RC = NB >= 4 ? 3 : kNormRegChunks;
    const bool reg_norm = NORM && nc <= kLinWaves * RC;

    if (NORM && !reg_norm) {
        // sum of squares of row tid >> 5 over the float4s t, t + 32, ... of the row, in
        // f64; loads go out 8 at a time so their latencies overlap
        const int r = tid >> 5, t = tid & 31;
        double ss = 0.0;
        if (m0 + r < a.rows) {
            const float4_t* xr = reinterpret_cast<const float4_t*>(a.x + (int64_t)(m0 + r) * a.ldx);
            const int n4 = a.k_in / 4;
            for (int i0 = t; i0 < n4; i0 += 32 * 8) {
                float4_t v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    v[i] = (i0 + 32 * i < n4) ? xr[i0 + 32 * i] : float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < 8; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const double d = (double)v[i][e];
                        ss += d * d;
                    }
            }
        }
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 32);
        if (t == 0) s_scale[r] = 1.0 / sqrt(ss / (double)a.k_in + a.eps);
        __syncthreads();
    }

    // The residual each output thread adds is requested now, so its round trip overlaps
    // the product instead of following it (out may alias resid: only this thread touches
    // the element).
    constexpr int kOut = 256 * NB;
    constexpr int kOutPer = (kOut + kLinThreads - 1) / kLinThreads;
    float rv[kOutPer];
    if constexpr (MODE == kResidual) {
#pragma unroll
        for (int i = 0; i < kOutPer; ++i) {
            const int o = tid + i * kLinThreads;
            const int blk = o >> 8, rem = o & 255;
            const int l = rem & 63, r = rem >> 6;
            const int orow = m0 + (l >> 4) + 4 * r;
            const int on = n0 + 16 * blk + (l & 15);
            rv[i] = (o < kOut && orow < a.rows && on < a.n_out)
                        ? a.resid[(int64_t)orow * a.ldo + on] : 0.0f;
        }
    }

    // wave w takes chunks [w * nc / 8, (w + 1) * nc / 8) of the nc chunks
    const int c0 = wave * nc / kLinWaves, c1 = (wave + 1) * nc / kLinWaves;
    const int kw = (c1 - c0) * kLinK;
    const int kbeg = c0 * kLinK + 8 * g;
    const int row = m0 + col;
    const bool row_ok = row < a.rows;
    const float* xp = a.x + (int64_t)(row_ok ? row : 0) * a.ldx + kbeg;
    const float* nwp = NORM ? a.norm_w + kbeg : nullptr;
    const half_t* wp[NB];
    bool n_ok[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const half_t* base = (MODE == kSwiGLU && col >= 8) ? a.w2 : a.w;
        const int n = MODE == kSwiGLU ? n0 + (col & 7) : n0 + col + 16 * j;
        n_ok[j] = n < a.n_out;
        wp[j] = base + (int64_t)(n_ok[j] ? n : 0) * a.k_in + kbeg;
    }

    auto load = [&](int k0) {
        Chunk<NB> c;
        c.x0 = *reinterpret_cast<const float4_t*>(xp + k0);
        c.x1 = *reinterpret_cast<const float4_t*>(xp + k0 + 4);
#pragma unroll
        for (int j = 0; j < NB; ++j) c.w[j] = *reinterpret_cast<const half8_t*>(wp[j] + k0);
        if constexpr (NORM) {
            c.n0 = *reinterpret_cast<const float4_t*>(nwp + k0);
            c.n1 = *reinterpret_cast<const float4_t*>(nwp + k0 + 4);
        }
        return c;
    };

    double4_t acc[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[j] = double4_t{0.0, 0.0, 0.0, 0.0};
    Prefetch pf{};

    // One chunk into the accumulators: the activations (normalised first under NORM)
    // and the weights go to f64, 8 MFMA steps per column block.
    auto feed = [&](const Chunk<NB>& ch, int k0, double scale) {
        float xs[8] = {ch.x0[0], ch.x0[1], ch.x0[2], ch.x0[3], ch.x1[0], ch.x1[1], ch.x1[2], ch.x1[3]};
        if constexpr (NORM) {
            const float nw[8] = {ch.n0[0], ch.n0[1], ch.n0[2], ch.n0[3],
                                 ch.n1[0], ch.n1[1], ch.n1[2], ch.n1[3]};
#pragma unroll
            for (int i = 0; i < 8; ++i) xs[i] = (float)((double)xs[i] * scale) * nw[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const double av = row_ok ? (double)xs[i] : 0.0;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const double bv = n_ok[j] ? (double)(float)ch.w[j][i] : 0.0;
                acc[j] = mfma_f64(av, bv, acc[j]);
            }
        }
    };

    if (reg_norm) {
        // Every chunk of the wave loads at once; the row's sum of squares comes from
        // those registers: per lane over its chunks, then over the 4 lane groups of the
        // row, then over the waves in a fixed order.
        Chunk<NB> ch[RC];
        const int nch = c1 - c0;
#pragma unroll
        for (int c = 0; c < RC; ++c)
            if (c < nch) ch[c] = load(c * kLinK);
        pf = prefetch_issue<kLinThreads>(a);
        __builtin_amdgcn_sched_barrier(0);  // issued now, not after the waits below
        double ss = 0.0;
#pragma unroll
        for (int c = 0; c < RC; ++c) {
            if (c >= nch) break;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const double d0 = (double)ch[c].x0[i], d1 = (double)ch[c].x1[i];
                ss += d0 * d0;
                ss += d1 * d1;
            }
        }
        ss += __shfl_xor(ss, 16);
        ss += __shfl_xor(ss, 32);
        if (g == 0) s_ss[wave][col] = ss;
        __syncthreads();
        double tot = 0.0;
#pragma unroll
        for (int w = 0; w < kLinWaves; ++w) tot += s_ss[w][col];
        const double scale = 1.0 / sqrt(tot / (double)a.k_in + a.eps);
#pragma unroll
        for (int c = 0; c < RC; ++c) {
            if (c >= nch) break;
            feed(ch[c], c * kLinK, scale);
        }
    } else {
        const double scale = NORM ? s_scale[col] : 1.0;
        // Up to kLinBatch chunks load at once (the weights stream from HBM once: their
        // latency, not the MFMA, bounds these small-batch products), then feed the MFMA.
        constexpr int BATCH = NB >= 4 ? 1 : kLinBatch;
        for (int b0 = 0; b0 < kw; b0 += BATCH * kLinK) {
            Chunk<NB> ch[BATCH];
#pragma unroll
            for (int c = 0; c < BATCH; ++c)
                if (b0 + c * kLinK < kw) ch[c] = load(b0 + c * kLinK);
            if (b0 == 0) pf = prefetch_issue<kLinThreads>(a);
#pragma unroll
            for (int c = 0; c < BATCH; ++c) {
                if (b0 + c * kLinK >= kw) break;
                feed(ch[c], b0 + c * kLinK, scale);
            }
        }
    }

#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) s_red[wave][j][r][lane] = acc[j][r];
    __syncthreads();

    // fixed summation order over the waves: the result does not depend on scheduling
    if constexpr (MODE == kSwiGLU) {
        // thread (row, c) of the 16 x 8 outputs: gate at tile column c, up at c + 8
        if (tid < 128) {
            const int orow = m0 + (tid >> 3), c = tid & 7;
            const int l = 16 * ((tid >> 3) & 3) + c, r = tid >> 5;
            if (orow < a.rows && n0 + c < a.n_out) {
                double y = 0.0, u = 0.0;
#pragma unroll
                for (int w = 0; w < kLinWaves; ++w) {
                    y += s_red[w][0][r][l];
                    u += s_red[w][0][r][l + 8];
                }
                const float gf = (float)y;
                a.out[(int64_t)orow * a.ldo + n0 + c] = gf / (1.0f + expf(-gf)) * (float)u;
            }
        }
        prefetch_retire(pf);
        return;
    }
#pragma unroll
    for (int i = 0; i < kOutPer; ++i) {
        const int o = tid + i * kLinThreads;
        if (o >= kOut) break;
        const int blk = o >> 8, rem = o & 255;
        const int l = rem & 63, r = rem >> 6;
        const int orow = m0 + (l >> 4) + 4 * r;
        const int on = n0 + 16 * blk + (l & 15);
        if (orow >= a.rows || on >= a.n_out) continue;
        double y = 0.0;
#pragma unroll
        for (int w = 0; w < kLinWaves; ++w) y += s_red[w][blk][r][l];
        float* dst = a.out + (int64_t)orow * a.ldo + on;
        if constexpr (MODE == kResidual) {
            *dst = rv[i] + (float)y;
        } else {
            *dst = (float)y;
        }
    }
    prefetch_retire(pf);
}

// ---------------------------------------------------------------- 4-column tiles

// f64 MFMA 4x4x4 (four 4x4 blocks) operand layout, measured on gfx950: lane l supplies
// A[l & 15][kslot] (the 16 rows are the four blocks of 4 rows) and B[kslot][l & 3] with
// kslot = l >> 4 (the blocks share B: lanes that differ only in bits 2-3 hold the same
// weight), and holds D[4 ((l >> 2) & 3) + (l >> 4)][l & 3]. It issues every 16 cycles,
// the MAC rate of the 16x16x4 form, for a quarter of the columns: a 16-row product
// spreads over four times the workgroups.
__device__ __forceinline__ double mfma4_f64(double a, double b, double c) {
    return __builtin_amdgcn_mfma_f64_4x4x4f64(a, b, c, 0, 0, 0);
}

// out tile = 16 rows x 4 columns; in kSwiGLU mode the gate rows and the up rows of those 4
// columns are two weight groups. Same K split over the waves, chunk loads, fused norm and
// f64 contract as linear_kernel; two accumulators per group (even and odd MFMA steps)
// keep two independent chains in flight, summed in a fixed order at the end.
// At most 128 VGPRs (4 waves per SIMD): two workgroups per CU, so grids of up to 512
// workgroups (the decode step's 288 for qkv, 512 for gate/up) run in one round.
template <bool NORM, int MODE>
__global__ __launch_bounds__(kLinThreads, 4) void linear4_kernel(LinArgs a) {
    constexpr int G = MODE == kSwiGLU ? 2 : 1;  // weight groups of 4 columns
    __shared__ double s_scale[16];
    __shared__ double s_ss[kLinWaves][16];
    __shared__ double s_red[kLinWaves][G][64];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int col = lane & 15;  // A row within the tile
    const int g = lane >> 4;
    const int m0 = blockIdx.y * 16;
    const int n0 = blockIdx.x * 4;
    const int nc = a.k_in / kLinK;
    constexpr int RC = 3;  // chunks held for the register-sourced norm (k_in <= 768)
    const bool reg_norm = NORM && nc <= kLinWaves * RC;

    // Output element of threads 0..63 (the D layout); the residual is requested now.
    const int orow = m0 + 4 * ((lane >> 2) & 3) + (lane >> 4);
    const int ocol = n0 + (lane & 3);
    const bool out_ok = tid < 64 && orow < a.rows && ocol < a.n_out;
    float rv = 0.0f;
    if constexpr (MODE == kResidual)
        if (out_ok) rv = a.resid[(int64_t)orow * a.ldo + ocol];

    if (NORM && !reg_norm) {
        const int r = tid >> 5, t = tid & 31;
        double ss = 0.0;
        if (m0 + r < a.rows) {
            const float4_t* xr = reinterpret_cast<const float4_t*>(a.x + (int64_t)(m0 + r) * a.ldx);
            const int n4 = a.k_in / 4;
            for (int i0 = t; i0 < n4; i0 += 32 * 8) {
                float4_t v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    v[i] = (i0 + 32 * i < n4) ? xr[i0 + 32 * i] : float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < 8; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const double d = (double)v[i][e];
                        ss += d * d;
                    }
            }
        }
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 32);
        if (t == 0) s_scale[r] = 1.0 / sqrt(ss / (double)a.k_in + a.eps);
        __syncthreads();
    }

    const int c0 = wave * nc / kLinWaves, c1 = (wave + 1) * nc / kLinWaves;
    const int kw = (c1 - c0) * kLinK;
    const int kbeg = c0 * kLinK + 8 * g;
    const int row = m0 + col;
    const bool row_ok = row < a.rows;
    const float* xp = a.x + (int64_t)(row_ok ? row : 0) * a.ldx + kbeg;
    const float* nwp = NORM ? a.norm_w + kbeg : nullptr;
    const int wn = n0 + (lane & 3);
    const bool wn_ok = wn < a.n_out;
    const half_t* wp[G];
    wp[0] = a.w + (int64_t)(wn_ok ? wn : 0) * a.k_in + kbeg;
    if constexpr (G == 2) wp[1] = a.w2 + (int64_t)(wn_ok ? wn : 0) * a.k_in + kbeg;

    auto load = [&](int k0) {
        Chunk<G> c;
        c.x0 = *reinterpret_cast<const float4_t*>(xp + k0);
        c.x1 = *reinterpret_cast<const float4_t*>(xp + k0 + 4);
#pragma unroll
        for (int j = 0; j < G; ++j) c.w[j] = *reinterpret_cast<const half8_t*>(wp[j] + k0);
        if constexpr (NORM) {
            c.n0 = *reinterpret_cast<const float4_t*>(nwp + k0);
            c.n1 = *reinterpret_cast<const float4_t*>(nwp + k0 + 4);
        }
        return c;
    };

    double acc[G][2];
#pragma unroll
    for (int j = 0; j < G; ++j) acc[j][0] = acc[j][1] = 0.0;
    Prefetch pf{};

    auto feed = [&](const Chunk<G>& ch, int k0, double scale) {
        float xs[8] = {ch.x0[0], ch.x0[1], ch.x0[2], ch.x0[3], ch.x1[0], ch.x1[1], ch.x1[2], ch.x1[3]};
        if constexpr (NORM) {
            const float nw[8] = {ch.n0[0], ch.n0[1], ch.n0[2], ch.n0[3],
                                 ch.n1[0], ch.n1[1], ch.n1[2], ch.n1[3]};
#pragma unroll
            for (int i = 0; i < 8; ++i) xs[i] = (float)((double)xs[i] * scale) * nw[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const double av = row_ok ? (double)xs[i] : 0.0;
#pragma unroll
            for (int j = 0; j < G; ++j) {
                const double bv = wn_ok ? (double)(float)ch.w[j][i] : 0.0;
                acc[j][i & 1] = mfma4_f64(av, bv, acc[j][i & 1]);
            }
        }
    };

    if (reg_norm) {
        Chunk<G> ch[RC];
        const int nch = c1 - c0;
#pragma unroll
        for (int c = 0; c < RC; ++c)
            if (c < nch) ch[c] = load(c * kLinK);
        pf = prefetch_issue<kLinThreads>(a);
        __builtin_amdgcn_sched_barrier(0);  // issued now, not after the waits below
        double ss = 0.0;
#pragma unroll
        for (int c = 0; c < RC; ++c) {
            if (c >= nch) break;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const double d0 = (double)ch[c].x0[i], d1 = (double)ch[c].x1[i];
                ss += d0 * d0;
                ss += d1 * d1;
            }
        }
        ss += __shfl_xor(ss, 16);
        ss += __shfl_xor(ss, 32);
        if (g == 0) s_ss[wave][col] = ss;
        __syncthreads();
        double tot = 0.0;
#pragma unroll
        for (int w = 0; w < kLinWaves; ++w) tot += s_ss[w][col];
        const double scale = 1.0 / sqrt(tot / (double)a.k_in + a.eps);
#pragma unroll
        for (int c = 0; c < RC; ++c) {
            if (c >= nch) break;
            feed(ch[c], c * kLinK, scale);
        }
    } else {
        const double scale = NORM ? s_scale[col] : 1.0;
        // 8 chunks in flight for the plain products (down: all of a wave's K at once);
        // the norm and SwiGLU forms keep 3 to stay within 128 registers
        constexpr int BATCH = (NORM || G == 2) ? 3 : kLinBatch;
        for (int b0 = 0; b0 < kw; b0 += BATCH * kLinK) {
            Chunk<G> ch[BATCH];
#pragma unroll
            for (int c = 0; c < BATCH; ++c)
                if (b0 + c * kLinK < kw) ch[c] = load(b0 + c * kLinK);
            if (b0 == 0) pf = prefetch_issue<kLinThreads>(a);
#pragma unroll
            for (int c = 0; c < BATCH; ++c) {
                if (b0 + c * kLinK >= kw) break;
                feed(ch[c], b0 + c * kLinK, scale);
            }
        }
    }

#pragma unroll
    for (int j = 0; j < G; ++j) s_red[wave][j][lane] = acc[j][0] + acc[j][1];
    __syncthreads();
    if (out_ok) {
        // fixed summation order over the waves
        double y[G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
            y[j] = 0.0;
#pragma unroll
            for (int w = 0; w < kLinWaves; ++w) y[j] += s_red[w][j][lane];
        }
        float* dst = a.out + (int64_t)orow * a.ldo + ocol;
        if constexpr (MODE == kSwiGLU) {
            const float gf = (float)y[0];
            *dst = gf / (1.0f + expf(-gf)) * (float)y[G - 1];
        } else if constexpr (MODE == kResidual) {
            *dst = rv + (float)y[0];
        } else {
            *dst = (float)y[0];
        }
    }
    prefetch_retire(pf);
}

// ---------------------------------------------------------------- wide projections

constexpr int kWideDepth = 4;  // weight tiles in flight per wave
constexpr int kWideMaxIters = 16;  // tiles per workgroup (the walk is fully unrolled)

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// The vocabulary projection: tens of thousands of output columns at <= 16 rows. A
// persistent grid (one workgroup per CU and 16-row block) walks the 16-column tiles, tile
// t on workgroup t mod gridDim.x, so the activations are loaded, normalised and converted
// to f64 once per workgroup and stay in registers for every tile, and every CU gets the
// same number of tiles to within one. Weights stream through a ring of kWideDepth tiles
// in registers, kWideDepth - 1 tiles ahead of the MFMAs. Every load and store is a buffer
// access whose range check does the masking (rows and columns past the end read zeros,
// stores there are dropped), so none sits behind a branch and the compiler's wait before
// each tile's MFMAs covers that tile's loads only. Same arithmetic, operand layout and
// fixed wave order as linear_kernel. RC = chunks per wave (k_in <= 256 * RC).
template <bool NORM, int RC>
__global__ __launch_bounds__(kLinThreads) void linear_wide_kernel(LinArgs a) {
    __shared__ double s_ss[kLinWaves][16];
    __shared__ double s_red[2][kLinWaves][4][64];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int col = lane & 15;
    const int g = lane >> 4;
    const int m0 = blockIdx.y * 16;
    const int nc = a.k_in / kLinK;
    const int c0 = wave * nc / kLinWaves, c1 = (wave + 1) * nc / kLinWaves;
    const int nch = c1 - c0;  // <= RC; chunks past it read as zeros
    const int kbeg = c0 * kLinK + 8 * g;
    const int row = m0 + col;
    // Offsets are below 2^31 (the launcher checks); OR-ing in the sign bit of (limit - 1 -
    // index) moves an index at or past its limit beyond every range. Arithmetic, not a
    // select: a branch around a load would hide its count from the compiler's waits.
    auto oob = [](int index, int limit) { return (uint32_t)(limit - 1 - index) & 0x80000000u; };

    const __amdgpu_buffer_rsrc_t xr =
        make_rsrc(a.x, (uint32_t)(((int64_t)(a.rows - 1) * a.ldx + a.k_in) * 4));
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, (uint32_t)((int64_t)a.n_out * a.k_in * 2));
    const __amdgpu_buffer_rsrc_t orr =
        make_rsrc(a.out, (uint32_t)(((int64_t)(a.rows - 1) * a.ldo + a.n_out) * 4));

    float4_t xv[RC][2], nv[RC][2];
#pragma unroll
    for (int c = 0; c < RC; ++c) {
        const uint32_t off = ((uint32_t)(row * (int)a.ldx + kbeg + c * kLinK) * 4u) |
                             oob(row, a.rows) | oob(c, nch);
        xv[c][0] = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
        xv[c][1] = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16, 0, 0));
        if constexpr (NORM) {
            const __amdgpu_buffer_rsrc_t nr = make_rsrc(a.norm_w, (uint32_t)(a.k_in * 4));
            const uint32_t noff = ((uint32_t)(kbeg + c * kLinK) * 4u) | oob(c, nch);
            nv[c][0] = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(nr, noff, 0, 0));
            nv[c][1] = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(nr, noff + 16, 0, 0));
        }
    }

    const int n_tiles = (a.n_out + 15) / 16;
    // tile t's weights for this lane: row 16 t + col, this wave's chunks
    auto wload = [&](int t, half8_t (&wv)[RC]) {
        const int n = 16 * t + col;
#pragma unroll
        for (int c = 0; c < RC; ++c) {
            const uint32_t off = ((uint32_t)(n * a.k_in + kbeg + c * kLinK) * 2u) |
                                 oob(n, a.n_out) | oob(c, nch);
            wv[c] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
        }
    };
    // The first weight tiles are requested before the activations are normalised, so their
    // latency overlaps that work (one workgroup per CU: registers are not the limit).
    half8_t wb[kWideDepth][RC];
#pragma unroll
    for (int j = 0; j < kWideDepth - 1; ++j) wload(blockIdx.x + j * gridDim.x, wb[j]);
    __builtin_amdgcn_sched_barrier(0);  // keep them ahead of the wait for the activations

    double scale = 1.0;
    if constexpr (NORM) {
        double ss = 0.0;
#pragma unroll
        for (int c = 0; c < RC; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const double d0 = (double)xv[c][0][i], d1 = (double)xv[c][1][i];
                ss += d0 * d0;
                ss += d1 * d1;
            }
        ss += __shfl_xor(ss, 16);
        ss += __shfl_xor(ss, 32);
        if (g == 0) s_ss[wave][col] = ss;
        __syncthreads();
        double tot = 0.0;
#pragma unroll
        for (int w = 0; w < kLinWaves; ++w) tot += s_ss[w][col];
        scale = 1.0 / sqrt(tot / (double)a.k_in + a.eps);
    }
    double av[RC][8];
#pragma unroll
    for (int c = 0; c < RC; ++c) {
        float xs[8] = {xv[c][0][0], xv[c][0][1], xv[c][0][2], xv[c][0][3],
                       xv[c][1][0], xv[c][1][1], xv[c][1][2], xv[c][1][3]};
        if constexpr (NORM) {
            const float nw[8] = {nv[c][0][0], nv[c][0][1], nv[c][0][2], nv[c][0][3],
                                 nv[c][1][0], nv[c][1][1], nv[c][1][2], nv[c][1][3]};
#pragma unroll
            for (int i = 0; i < 8; ++i) xs[i] = (float)((double)xs[i] * scale) * nw[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) av[c][i] = (double)xs[i];
    }

    // Iteration i handles tile blockIdx.x + i * gridDim.x from ring slot i % depth. The walk
    // is unrolled whole (the launcher keeps it within kWideMaxIters tiles a workgroup):
    // straight-line code lets the compiler's wait before each tile's MFMAs count exactly
    // the loads still in flight, where a loop's back edge made it drain them all. The exit
    // is uniform across the workgroup.
#pragma unroll
    for (int i = 0; i < kWideMaxIters; ++i) {
        const int t = blockIdx.x + i * gridDim.x;
        if (t >= n_tiles) break;
        wload(t + (kWideDepth - 1) * gridDim.x, wb[(i + kWideDepth - 1) % kWideDepth]);
        double4_t acc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int c = 0; c < RC; ++c)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                acc = mfma_f64(av[c][e], (double)(float)wb[i % kWideDepth][c][e], acc);
        double* red = &s_red[i & 1][0][0][0];
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(wave * 4 + r) * 64 + lane] = acc[r];
        __syncthreads();
        // waves 0..3: output (row (l >> 4) + 4 r, column l & 15) of the tile
        const int l = tid & 63, r = (tid >> 6) & 3;
        double y = 0.0;
#pragma unroll
        for (int w = 0; w < kLinWaves; ++w) y += red[(w * 4 + r) * 64 + l];
        const int orow = m0 + (l >> 4) + 4 * r;
        const int on = 16 * t + (l & 15);
        const uint32_t off = ((uint32_t)(orow * (int)a.ldo + on) * 4u) | oob(tid, 256) |
                             oob(orow, a.rows) | oob(on, a.n_out);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, (float)y), orr, off, 0, 0);
    }
}

// ---------------------------------------------------------------- prompt-sized products

// Products over a whole prompt batch (thousands of rows; the reference's prefill runs them
// as WMMA GEMMs, kernels.cu:2402-2526) are bound by the f64 MFMA itself: a 16x16x4 step
// occupies a SIMD for 64 cycles, so 16 bytes of operands per lane every 64 cycles keep it
// busy, and no LDS staging is needed. The decode tilings (16-row tiles, the K range split
// over 8 waves, every weight read once per 16 rows) give way to output tiles: each wave
// owns RB x CB MFMA blocks (RB*16 rows x CB*16 columns) over the whole K range, so no sum
// crosses waves and each output is one wave's fixed-order f64 sum. Operands come from L2
// straight into registers, two 32-wide K chunks ahead of the MFMAs.
//
// The waves of a workgroup share their rows (and the fused norm's row scales) and take
// adjacent column ranges. Workgroup L runs on XCD L % 8; XCD x takes tiles
// [x * per_xcd, (x + 1) * per_xcd) in row-major order, so each XCD's L2 holds one slice of
// the rows plus the weights, instead of every XCD fetching every row.
constexpr int kGemmWaves = 4;
constexpr int kGemmThreads = 64 * kGemmWaves;
constexpr int kGemmMinRows = 128;  // below this the decode tilings are used

template <int RB, int CB, bool NORM>
struct GemmChunk {
    float4_t x[RB][2];
    half8_t w[CB];
    float4_t nw[NORM ? 2 : 1];  // the norm weights of the chunk's K range (NORM only)
};

template <bool NORM, int MODE, int RB, int CB>
__global__ __launch_bounds__(kGemmThreads, 2) void linear_gemm_kernel(LinArgs a, int col_tiles,
                                                                      int n_tiles, int per_xcd) {
    static_assert(MODE != kSwiGLU || CB % 2 == 0, "SwiGLU pairs each gate block with its up block");
    constexpr int ROWS = RB * 16;
    // a wave's output columns: CB blocks, or CB / 2 gate blocks beside their up blocks
    constexpr int NBLK = MODE == kSwiGLU ? CB / 2 : CB;
    __shared__ double s_scale[ROWS];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int col = lane & 15, g = lane >> 4;
    const int L = blockIdx.x;
    const int t = (L & 7) * per_xcd + (L >> 3);
    if (t >= n_tiles) return;  // uniform over the workgroup
    const int rt = t / col_tiles;
    const int m0 = rt * ROWS;
    const int n0 = ((t - rt * col_tiles) * kGemmWaves + wave) * NBLK * 16;

    if constexpr (NORM) {
        // f64 sums of squares of the workgroup's rows: TPR threads a row over interleaved
        // float4s, 8 loads in flight; rows past the end get sum 0 (their outputs are not
        // stored)
        constexpr int TPR = kGemmThreads / ROWS;
        const int r = tid / TPR, q = tid % TPR;
        const int row = m0 + r;
        double ss = 0.0;
        if (row < a.rows) {
            const float4_t* xr = reinterpret_cast<const float4_t*>(a.x + (int64_t)row * a.ldx);
            const int n4 = a.k_in / 4;
            for (int i0 = q; i0 < n4; i0 += TPR * 8) {
                float4_t v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    v[i] = (i0 + TPR * i < n4) ? xr[i0 + TPR * i] : float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < 8; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const double d = (double)v[i][e];
                        ss += d * d;
                    }
            }
        }
#pragma unroll
        for (int off = TPR / 2; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, TPR);
        if (q == 0) s_scale[r] = 1.0 / sqrt(ss / (double)a.k_in + a.eps);
        __syncthreads();
    }
    if (n0 >= a.n_out) return;

    // Lane (col, g) feeds row m0 + 16 rb + col of A and column 16 cb + col of B with
    // k = k0 + 8 g + i at MFMA step i of a 32-wide chunk. Rows and columns past the end
    // read the last valid one: an MFMA output depends only on its own row and column, and
    // those outputs are not stored.
    const float* xp[RB];
    double scale[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int row = m0 + 16 * rb + col;
        xp[rb] = a.x + (int64_t)(row < a.rows ? row : a.rows - 1) * a.ldx + 8 * g;
        scale[rb] = NORM ? s_scale[16 * rb + col] : 1.0;
    }
    const half_t* wp[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        const half_t* base = (MODE == kSwiGLU && cb >= NBLK) ? a.w2 : a.w;
        const int n = n0 + 16 * (cb % NBLK) + col;
        wp[cb] = base + (int64_t)(n < a.n_out ? n : a.n_out - 1) * a.k_in + 8 * g;
    }
    const float* nwp = NORM ? a.norm_w + 8 * g : nullptr;

    // the residual is requested first, so its round trip is long over by the epilogue
    // (out may alias resid: each element is read and written by the same lane)
    float rv[RB][NBLK][4];
    if constexpr (MODE == kResidual) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int cb = 0; cb < NBLK; ++cb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = min(m0 + 16 * rb + g + 4 * r, a.rows - 1);
                    const int n = min(n0 + 16 * cb + col, a.n_out - 1);
                    rv[rb][cb][r] = a.resid[(int64_t)row * a.ldo + n];
                }
    }

    using Chunk = GemmChunk<RB, CB, NORM>;
    auto load = [&](int k0, Chunk& c) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            c.x[rb][0] = *reinterpret_cast<const float4_t*>(xp[rb] + k0);
            c.x[rb][1] = *reinterpret_cast<const float4_t*>(xp[rb] + k0 + 4);
        }
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) c.w[cb] = *reinterpret_cast<const half8_t*>(wp[cb] + k0);
        if constexpr (NORM) {
            c.nw[0] = *reinterpret_cast<const float4_t*>(nwp + k0);
            c.nw[1] = *reinterpret_cast<const float4_t*>(nwp + k0 + 4);
        }
    };

    double4_t acc[RB][CB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = double4_t{0.0, 0.0, 0.0, 0.0};

    auto feed = [&](const Chunk& c) {
        double av[RB][8];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            float xs[8] = {c.x[rb][0][0], c.x[rb][0][1], c.x[rb][0][2], c.x[rb][0][3],
                           c.x[rb][1][0], c.x[rb][1][1], c.x[rb][1][2], c.x[rb][1][3]};
            if constexpr (NORM) {
                const float nw[8] = {c.nw[0][0], c.nw[0][1], c.nw[0][2], c.nw[0][3],
                                     c.nw[1][0], c.nw[1][1], c.nw[1][2], c.nw[1][3]};
#pragma unroll
                for (int i = 0; i < 8; ++i) xs[i] = (float)((double)xs[i] * scale[rb]) * nw[i];
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) av[rb][i] = (double)xs[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            double bv[CB];
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) bv[cb] = (double)(float)c.w[cb][i];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = mfma_f64(av[rb][i], bv[cb], acc[rb][cb]);
        }
    };

    // Two chunks in flight, reloaded in place: the loads are unconditional (the last
    // iteration re-reads the final pair, unused), so each buffer keeps its registers
    // across the loop and the wait before a feed counts only the other buffer's loads.
    // k_in is a multiple of 64.
    Chunk c0, c1;
    load(0, c0);
    __builtin_amdgcn_sched_barrier(0);  // c0's loads before c1's, as in the loop
    load(32, c1);
    __builtin_amdgcn_sched_barrier(0);
    for (int k0 = 0; k0 < a.k_in; k0 += 64) {
        feed(c0);
        __builtin_amdgcn_sched_barrier(0);
        load(min(k0 + 64, a.k_in - 64), c0);
        __builtin_amdgcn_sched_barrier(0);
        feed(c1);
        __builtin_amdgcn_sched_barrier(0);
        load(min(k0 + 96, a.k_in - 32), c1);
        __builtin_amdgcn_sched_barrier(0);
    }

    // lane (col, g) holds rows 16 rb + g + 4 r, column 16 cb + col of the wave's blocks
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < NBLK; ++cb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + 16 * rb + g + 4 * r;
                const int n = n0 + 16 * cb + col;
                if (row >= a.rows || n >= a.n_out) continue;
                float* dst = a.out + (int64_t)row * a.ldo + n;
                if constexpr (MODE == kSwiGLU) {
                    const float gf = (float)acc[rb][cb][r];
                    *dst = gf / (1.0f + expf(-gf)) * (float)acc[rb][cb + NBLK][r];
                } else if constexpr (MODE == kResidual) {
                    *dst = rv[rb][cb][r] + (float)acc[rb][cb][r];
                } else {
                    *dst = (float)acc[rb][cb][r];
                }
            }
}

// ---------------------------------------------------------------- RMSNorm rows

constexpr int kNormThreads = 256;

__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const float* __restrict__ x,
                                                               int64_t ldx,
                                                               const float* __restrict__ w,
                                                               double eps, float* out,
                                                               int64_t ldo, int n) {
    __shared__ double s_part[kNormThreads / 64];
    const float* xr = x + (int64_t)blockIdx.x * ldx;
    double ss = 0.0;
    for (int k = threadIdx.x; k < n; k += kNormThreads) {
        const double v = (double)xr[k];
        ss += v * v;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int i = 0; i < kNormThreads / 64; ++i) tot += s_part[i];
    const double scale = 1.0 / sqrt(tot / (double)n + eps);
    float* orow = out + (int64_t)blockIdx.x * ldo;
    for (int k = threadIdx.x; k < n; k += kNormThreads)
        orow[k] = (float)((double)xr[k] * scale) * w[k];
}

// ---------------------------------------------------------------- RoPE + split

// One thread per (row, head, i < 32) of the fused [q | k | v] row: q and k heads rotate,
// v heads copy. A position outside the tables yields NaN rows (no out-of-range read).
__global__ void rope_split_kernel(const float* __restrict__ qkv, int64_t ld, float* q,
                                  float* k, float* v, const float* __restrict__ cos_t,
                                  const float* __restrict__ sin_t,
                                  const int32_t* __restrict__ positions, int rows, int n_head,
                                  int n_kv_head, int head_dim, int max_pos) {
    const int heads = n_head + 2 * n_kv_head;
    const int half = head_dim >> 1;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)rows * heads * half) return;
    const int i = (int)(idx % half);
    const int head = (int)((idx / half) % heads);
    const int row = (int)((idx / half) / heads);
    const float* src = qkv + (int64_t)row * ld + (int64_t)head * head_dim;
    const float lo = src[i], hi = src[i + half];
    float* dst;
    if (head < n_head) dst = q + ((int64_t)row * n_head + head) * head_dim;
    else if (head < n_head + n_kv_head) dst = k + ((int64_t)row * n_kv_head + head - n_head) * head_dim;
    else dst = v + ((int64_t)row * n_kv_head + head - n_head - n_kv_head) * head_dim;
    if (head >= n_head + n_kv_head) {
        dst[i] = lo;
        dst[i + half] = hi;
        return;
    }
    const int pos = positions[row];
    if (pos < 0 || pos >= max_pos) {
        dst[i] = dst[i + half] = __builtin_nanf("");
        return;
    }
    const float c = cos_t[(int64_t)pos * half + i];
    const float s = sin_t[(int64_t)pos * half + i];
    dst[i] = lo * c - hi * s;
    dst[i + half] = lo * s + hi * c;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// The prefetch's lines a workgroup: the region spread evenly over the grid, at most
// kPfPerThread lines a thread.
LinArgs with_prefetch_share(LinArgs a, const dim3& grid) {
    const int64_t n_wg = (int64_t)grid.x * grid.y;
    const int64_t lines = a.pf_bytes >> 6;
    a.pf_per = (int)std::min<int64_t>((lines + n_wg - 1) / n_wg, kPfPerThread * kLinThreads);
    return a;
}

template <bool NORM, int MODE, int NB>
void launch_linear(const LinArgs& a, hipStream_t stream) {
    const int cols = MODE == kSwiGLU ? 8 : 16 * NB;
    const dim3 grid((unsigned)((a.n_out + cols - 1) / cols), (unsigned)((a.rows + 15) / 16));
    hipLaunchKernelGGL((linear_kernel<NORM, MODE, NB>), grid, dim3(kLinThreads), 0, stream,
                       with_prefetch_share(a, grid));
}

template <bool NORM, int MODE>
void launch_linear4(const LinArgs& a, hipStream_t stream) {
    const dim3 grid((unsigned)((a.n_out + 3) / 4), (unsigned)((a.rows + 15) / 16));
    hipLaunchKernelGGL((linear4_kernel<NORM, MODE>), grid, dim3(kLinThreads), 0, stream,
                       with_prefetch_share(a, grid));
}

template <bool NORM, int MODE, int RB, int CB>
void launch_gemm(const LinArgs& a, hipStream_t stream) {
    constexpr int wg_cols = (MODE == kSwiGLU ? CB / 2 : CB) * 16 * kGemmWaves;
    const int col_tiles = (a.n_out + wg_cols - 1) / wg_cols;
    const int n_tiles = col_tiles * ((a.rows + RB * 16 - 1) / (RB * 16));
    const int per_xcd = (n_tiles + 7) / 8;
    hipLaunchKernelGGL((linear_gemm_kernel<NORM, MODE, RB, CB>), dim3((unsigned)(8 * per_xcd)),
                       dim3(kGemmThreads), 0, stream, a, col_tiles, n_tiles, per_xcd);
}

// Output-tiled products for prompt-sized row counts (k_in a multiple of 64);
// CRUCIBLE_TUNE_LINEAR_TILE = 32 forces them, 4 or 16 the decode tilings.
bool use_gemm(int64_t rows, int64_t k_in) {
    if (k_in % 64 != 0) return false;
    if (const int v = tuning(CRUCIBLE_TUNE_LINEAR_TILE); v > 0) return v == 32;
    return rows >= kGemmMinRows;
}

template <int MODE>
void launch_gemm_mode(const LinArgs& a, hipStream_t stream) {
    if (a.norm_w) launch_gemm<true, MODE, 2, 2>(a, stream);
    else launch_gemm<false, MODE, 2, 2>(a, stream);
}

// 4-column tiles where 16-column tiles would leave CUs without a workgroup and no norm is
// fused (the decode step's o and down projections: 5.16 -> 4.84 and 10.2 -> 8.9 us).
// With a fused norm every workgroup loads and normalises the whole rows, and four times
// the workgroups made it slower (qkv 6.9 -> 8.8 us, gate/up 7.4 -> 11.6 us), so those keep
// 16 columns. CRUCIBLE_TUNE_LINEAR_TILE = 4 | 16 overrides the choice.
bool use_tile4(int64_t n_out, int64_t rows, int cols16, bool norm) {
    if (const int v = tuning(CRUCIBLE_TUNE_LINEAR_TILE); v > 0) return v == 4;
    return !norm && ((n_out + cols16 - 1) / cols16) * ((rows + 15) / 16) < device_cu_count();
}

int check_linear(const char* what, const float* x, int64_t ldx, const float* norm_w,
                 const void* w, int64_t n_out, int64_t k_in, const float* out, int64_t ldo,
                 int64_t rows) {
    CRUCIBLE_CHECK(x && w && out, CRUCIBLE_ERR_INVALID, "%s: null buffer", what);
    CRUCIBLE_CHECK(rows >= 0 && rows <= 16 * 65535, CRUCIBLE_ERR_INVALID, "%s: rows %lld",
                   what, (long long)rows);
    CRUCIBLE_CHECK(n_out > 0 && n_out <= INT32_MAX, CRUCIBLE_ERR_INVALID, "%s: n_out %lld",
                   what, (long long)n_out);
    CRUCIBLE_CHECK(k_in > 0 && k_in % 32 == 0 && k_in <= (1 << 20), CRUCIBLE_ERR_UNSUPPORTED,
                   "%s: k_in %lld must be a positive multiple of 32", what, (long long)k_in);
    CRUCIBLE_CHECK(ldx >= k_in && ldx % 4 == 0 && ldo >= n_out && ldx <= INT32_MAX &&
                       ldo <= INT32_MAX,
                   CRUCIBLE_ERR_INVALID, "%s: leading dimensions (ldx %lld, ldo %lld)", what,
                   (long long)ldx, (long long)ldo);
    CRUCIBLE_CHECK(aligned16(x) && aligned16(w) && (!norm_w || aligned16(norm_w)),
                   CRUCIBLE_ERR_INVALID, "%s: x, w and norm_w must be 16-byte aligned", what);
    return CRUCIBLE_OK;
}

int check_prefetch(const char* what, const void* pf, int64_t pf_bytes) {
    CRUCIBLE_CHECK(pf_bytes >= 0 && pf_bytes % 64 == 0 && (pf_bytes == 0 || pf) &&
                       ((uintptr_t)pf & 3) == 0,
                   CRUCIBLE_ERR_INVALID,
                   "%s: prefetch (%p, %lld bytes) must be 4-byte aligned, a multiple of 64 bytes",
                   what, pf, (long long)pf_bytes);
    return CRUCIBLE_OK;
}

// The prefetch region as the kernels take it: none when the tuning key turns it off.
void set_prefetch(LinArgs& a, const void* pf, int64_t pf_bytes) {
    if (tuning(CRUCIBLE_TUNE_LINEAR_PREFETCH) == 0) pf_bytes = 0;
    a.pf = pf_bytes > 0 ? static_cast<const unsigned char*>(pf) : nullptr;
    a.pf_bytes = pf_bytes;
}

int linear_f64acc(const char* what, const float* x, int64_t ldx, const float* norm_w, float eps,
                  const void* w, int64_t n_out, int64_t k_in, const float* resid, float* out,
                  int64_t ldo, int64_t rows, const void* pf, int64_t pf_bytes,
                  crucible_stream_t stream) {
    int rc = check_linear(what, x, ldx, norm_w, w, n_out, k_in, out, ldo, rows);
    if (rc == CRUCIBLE_OK) rc = check_prefetch(what, pf, pf_bytes);
    if (rc != CRUCIBLE_OK) return rc;
    if (rows == 0) return CRUCIBLE_OK;
    LinArgs a{x, ldx, norm_w, (double)eps, static_cast<const half_t*>(w), nullptr, resid, out,
              ldo, (int)rows, (int)n_out, (int)k_in};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (use_gemm(rows, k_in)) {
        if (resid) launch_gemm_mode<kResidual>(a, s);
        else launch_gemm_mode<kPlain>(a, s);
        return fail_launch(what);
    }
    set_prefetch(a, pf, pf_bytes);
    // Wide outputs (the vocabulary projection): the persistent tile walk when the K range
    // fits its registers, else 4 column blocks per workgroup so each activation fragment
    // feeds 4 MFMAs; narrow ones keep a workgroup per 16 columns.
    const bool wide = n_out >= 16 * 1024;
    const int64_t wide_rc = (k_in / kLinK + kLinWaves - 1) / kLinWaves;
    // the buffer ranges of the persistent walk are 32-bit
    const bool wide_fits = (int64_t)n_out * k_in * 2 < (1LL << 31) &&
                           ((rows - 1) * ldx + k_in) * 4 < (1LL << 31) &&
                           ((rows - 1) * ldo + n_out) * 4 < (1LL << 31);
    if (wide && !resid && wide_rc <= 4 && wide_fits) {
        a.pf = nullptr;  // the persistent walk streams its own tiles to the end
        a.pf_bytes = 0;
        const int64_t row_blocks = (rows + 15) / 16;
        const int64_t tiles = (n_out + 15) / 16;
        // one workgroup per CU (and row block), or more when a CU would need more than
        // kWideMaxIters tiles
        const int64_t cus = device_cu_count();
        const int64_t per_cu = std::max<int64_t>(1, cus / std::min<int64_t>(row_blocks, cus));
        const int64_t gx = std::min<int64_t>(
            tiles, std::max<int64_t>(per_cu, (tiles + kWideMaxIters - 1) / kWideMaxIters));
        const dim3 grid((unsigned)gx, (unsigned)row_blocks);
        auto go = [&](auto norm_tag, auto rc_tag) {
            hipLaunchKernelGGL((linear_wide_kernel<decltype(norm_tag)::value, decltype(rc_tag)::value>),
                               grid, dim3(kLinThreads), 0, s, a);
        };
        auto by_rc = [&](auto norm_tag) {
            switch (wide_rc) {
                case 1: go(norm_tag, std::integral_constant<int, 1>{}); break;
                case 2: go(norm_tag, std::integral_constant<int, 2>{}); break;
                case 3: go(norm_tag, std::integral_constant<int, 3>{}); break;
                default: go(norm_tag, std::integral_constant<int, 4>{}); break;
            }
        };
        if (norm_w) by_rc(std::true_type{});
        else by_rc(std::false_type{});
        return fail_launch(what);
    }
    if (!wide && use_tile4(n_out, rows, 16, norm_w != nullptr)) {
        if (resid) {
            if (norm_w) launch_linear4<true, kResidual>(a, s);
            else launch_linear4<false, kResidual>(a, s);
        } else {
            if (norm_w) launch_linear4<true, kPlain>(a, s);
            else launch_linear4<false, kPlain>(a, s);
        }
    } else if (resid) {
        if (norm_w) launch_linear<true, kResidual, 1>(a, s);
        else launch_linear<false, kResidual, 1>(a, s);
    } else if (norm_w) {
        if (wide) launch_linear<true, kPlain, 4>(a, s);
        else launch_linear<true, kPlain, 1>(a, s);
    } else {
        if (wide) launch_linear<false, kPlain, 4>(a, s);
        else launch_linear<false, kPlain, 1>(a, s);
    }
    return fail_launch(what);
}

int linear_swiglu_f64acc(const char* what, const float* x, int64_t ldx, const float* norm_w,
                         float eps, const void* w_gate, const void* w_up, int64_t hidden,
                         int64_t k_in, float* out, int64_t ldo, int64_t rows, const void* pf,
                         int64_t pf_bytes, crucible_stream_t stream) {
    int rc = check_linear(what, x, ldx, norm_w, w_gate, hidden, k_in, out, ldo, rows);
    if (rc == CRUCIBLE_OK) rc = check_prefetch(what, pf, pf_bytes);
    if (rc != CRUCIBLE_OK) return rc;
    CRUCIBLE_CHECK(w_up && aligned16(w_up), CRUCIBLE_ERR_INVALID,
                   "%s: w_up must be a 16-byte aligned buffer", what);
    if (rows == 0) return CRUCIBLE_OK;
    LinArgs a{x, ldx, norm_w, (double)eps, static_cast<const half_t*>(w_gate),
              static_cast<const half_t*>(w_up), nullptr, out, ldo, (int)rows, (int)hidden,
              (int)k_in};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (use_gemm(rows, k_in)) {
        launch_gemm_mode<kSwiGLU>(a, s);
        return fail_launch(what);
    }
    set_prefetch(a, pf, pf_bytes);
    if (use_tile4(hidden, rows, 8, norm_w != nullptr)) {
        if (norm_w) launch_linear4<true, kSwiGLU>(a, s);
        else launch_linear4<false, kSwiGLU>(a, s);
    } else if (norm_w) {
        launch_linear<true, kSwiGLU, 1>(a, s);
    } else {
        launch_linear<false, kSwiGLU, 1>(a, s);
    }
    return fail_launch(what);
}

}  // namespace
}  // namespace crucible

using namespace crucible;

extern "C" int crucible_linear_f64acc(const float* x, int64_t ldx, const float* norm_w, float eps,
                                      const void* w, int64_t n_out, int64_t k_in,
                                      const float* resid, float* out, int64_t ldo, int64_t rows,
                                      crucible_stream_t stream) {
    return linear_f64acc("crucible_linear_f64acc", x, ldx, norm_w, eps, w, n_out, k_in, resid,
                         out, ldo, rows, nullptr, 0, stream);
}

extern "C" int crucible_linear_f64acc_prefetch(const float* x, int64_t ldx, const float* norm_w,
                                               float eps, const void* w, int64_t n_out,
                                               int64_t k_in, const float* resid, float* out,
                                               int64_t ldo, int64_t rows, const void* prefetch,
                                               int64_t prefetch_bytes, crucible_stream_t stream) {
    return linear_f64acc("crucible_linear_f64acc_prefetch", x, ldx, norm_w, eps, w, n_out, k_in,
                         resid, out, ldo, rows, prefetch, prefetch_bytes, stream);
}

extern "C" int crucible_linear_swiglu_f64acc(const float* x, int64_t ldx, const float* norm_w,
                                             float eps, const void* w_gate, const void* w_up,
                                             int64_t hidden, int64_t k_in, float* out,
                                             int64_t ldo, int64_t rows,
                                             crucible_stream_t stream) {
    return linear_swiglu_f64acc("crucible_linear_swiglu_f64acc", x, ldx, norm_w, eps, w_gate,
                                w_up, hidden, k_in, out, ldo, rows, nullptr, 0, stream);
}

extern "C" int crucible_linear_swiglu_f64acc_prefetch(const float* x, int64_t ldx,
                                                      const float* norm_w, float eps,
                                                      const void* w_gate, const void* w_up,
                                                      int64_t hidden, int64_t k_in, float* out,
                                                      int64_t ldo, int64_t rows,
                                                      const void* prefetch,
                                                      int64_t prefetch_bytes,
                                                      crucible_stream_t stream) {
    return linear_swiglu_f64acc("crucible_linear_swiglu_f64acc_prefetch", x, ldx, norm_w, eps,
                                w_gate, w_up, hidden, k_in, out, ldo, rows, prefetch,
                                prefetch_bytes, stream);
}

extern "C" int crucible_rmsnorm_rows(const float* x, int64_t ldx, const float* w, float eps,
                                     float* out, int64_t ldo, int64_t rows, int64_t n,
                                     crucible_stream_t stream) {
    const char* what = "crucible_rmsnorm_rows";
    CRUCIBLE_CHECK(x && w && out, CRUCIBLE_ERR_INVALID, "%s: null buffer", what);
    CRUCIBLE_CHECK(rows >= 0 && rows <= INT32_MAX && n > 0 && n <= INT32_MAX && ldx >= n &&
                       ldo >= n && ldx <= INT32_MAX && ldo <= INT32_MAX,
                   CRUCIBLE_ERR_INVALID, "%s: bad shape", what);
    if (rows == 0) return CRUCIBLE_OK;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(kNormThreads), 0,
                       reinterpret_cast<hipStream_t>(stream), x, ldx, w, (double)eps, out, ldo,
                       (int)n);
    return fail_launch(what);
}

extern "C" int crucible_rope_split_qkv(const float* qkv, int64_t ld, float* q, float* k, float* v,
                                       const float* cos_table, const float* sin_table,
                                       const int32_t* positions, int64_t rows, int64_t n_head,
                                       int64_t n_kv_head, int64_t head_dim, int64_t max_pos,
                                       crucible_stream_t stream) {
    const char* what = "crucible_rope_split_qkv";
    CRUCIBLE_CHECK(qkv && q && k && v && cos_table && sin_table && positions,
                   CRUCIBLE_ERR_INVALID, "%s: null buffer", what);
    CRUCIBLE_CHECK(head_dim > 0 && head_dim % 2 == 0 && head_dim <= 4096, CRUCIBLE_ERR_UNSUPPORTED,
                   "%s: head_dim %lld unsupported (an even number up to 4096)", what,
                   (long long)head_dim);
    CRUCIBLE_CHECK(n_head > 0 && n_kv_head > 0 && n_head <= 4096 && n_kv_head <= 4096 &&
                       ld >= (n_head + 2 * n_kv_head) * head_dim && ld <= INT32_MAX &&
                       max_pos > 0 &&
                       max_pos <= INT32_MAX && rows >= 0 && rows <= (1 << 24),
                   CRUCIBLE_ERR_INVALID, "%s: bad shape", what);
    if (rows == 0) return CRUCIBLE_OK;
    const int64_t threads = rows * (n_head + 2 * n_kv_head) * (head_dim / 2);
    hipLaunchKernelGGL(rope_split_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), qkv, ld, q, k, v, cos_table,
                       sin_table, positions, (int)rows, (int)n_head, (int)n_kv_head,
                       (int)head_dim, (int)max_pos);
    return fail_launch(what);
}
