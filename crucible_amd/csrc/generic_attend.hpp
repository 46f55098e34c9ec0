// Attention of one query row for head dimensions other than 64.
//
// The reference kernels take any head_dim (kernels.cu:1741-1756, 2100-2276: loops over d in
// steps of the warp). The MFMA kernels of attn_decode.hip / attn_prefill.hip are built for
// head_dim 64, the dimension of every preset. Other dimensions (a multiple of 8 up to 256)
// run through this workgroup-level routine instead: plain wave64 code, f32 accumulation,
// fp16 K/V read from the same pool layout, online softmax in base 2.
//
// One workgroup of kGenericThreads threads attends one (query row, query head) over keys
// [0, n). Wave w takes the 64-key blocks w, w + 4, ...: lane k scores key 64 * blk + k
// (q from LDS, its K row in 16-byte loads), the wave's max and sum come from lane
// shuffles, and for the P.V product the lanes switch to dimensions (lane d holds dims d,
// d + 64, ...) and read each page's V^T rows (16 contiguous slots per dimension). The four
// wave states merge through LDS at the end.
#pragma once

#include "common.hpp"

namespace crucible {

constexpr int kGenericMaxHeadDim = 256;
constexpr int kGenericThreads = 256;
constexpr int kGenericWaves = kGenericThreads / 64;

inline bool generic_head_dim_ok(int64_t hd) {
    return hd > 0 && hd % 8 == 0 && hd <= kGenericMaxHeadDim;
}

// Where the keys of a row live.
struct GenericKeys {
    const half_t* k_pool;
    const half_t* v_pool;
    PoolAddr addr;
    const int32_t* table;  // the row's page table, or nullptr: page = position >> 4
    int g;                 // kv head
    int hd;
    // Keys at positions in [astart, n) come from the chunk's own rows cur_k / cur_v
    // ([row][kv_dim] f32; row pstart + position - astart), rounded to fp16 as the append
    // stores them (hybrid prefill). astart = INT32_MAX: none.
    int astart;
    int pstart;
    const float* cur_k;
    const float* cur_v;
};

struct GenericLds {
    alignas(16) float q[kGenericMaxHeadDim];  // the query row, f32
    alignas(16) float p[kGenericWaves][64];   // each wave's probabilities of its key block
    alignas(16) float o[kGenericWaves][kGenericMaxHeadDim];
    float m[kGenericWaves];
    float l[kGenericWaves];
};

__device__ __forceinline__ float generic_wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

__device__ __forceinline__ float generic_wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ float round_f16(float x) { return (float)(half_t)x; }

// Attention of the query row in lds.q (hd values) over keys [0, n), n >= 1, by the whole
// workgroup (every thread calls it). store(d, value) is called once for each d < hd.
// scale_log2 = log2(e) / sqrt(hd).
template <class Store>
__device__ void attend_generic(GenericLds& lds, const GenericKeys& ks, int n, float scale_log2,
                               Store store) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hd = ks.hd;
    const int kv_dim = ks.addr.kv_dim;
    const int head_off = ks.g * hd;
    float m = -INFINITY;  // running max, log2-scaled
    float l = 0.0f;
    float o[kGenericMaxHeadDim / 64] = {};
    for (int blk = wave; blk * 64 < n; blk += kGenericWaves) {
        const int key0 = blk * 64;
        // scores: lane k takes key key0 + k
        const int j = key0 + lane;
        float s2 = -INFINITY;
        if (j < n) {
            float acc = 0.0f;
            if (j >= ks.astart) {
                const float* kc = ks.cur_k + (int64_t)(ks.pstart + j - ks.astart) * kv_dim + head_off;
                for (int c = 0; c < hd; c += 4) {
                    const float4_t q4 = *reinterpret_cast<const float4_t*>(&lds.q[c]);
#pragma unroll
                    for (int t = 0; t < 4; ++t) acc = __builtin_fmaf(q4[t], round_f16(kc[c + t]), acc);
                }
            } else {
                const int64_t page = ks.table ? (int64_t)ks.table[j >> kPageShift]
                                              : (int64_t)(j >> kPageShift);
                const half_t* kr = ks.k_pool + block_base(ks.addr, page) +
                                   (int64_t)(j & kPageMask) * kv_dim + head_off;
                for (int c = 0; c < hd; c += 8) {
                    const half8_t k8 = *reinterpret_cast<const half8_t*>(kr + c);
                    const float4_t q0 = *reinterpret_cast<const float4_t*>(&lds.q[c]);
                    const float4_t q1 = *reinterpret_cast<const float4_t*>(&lds.q[c + 4]);
#pragma unroll
                    for (int t = 0; t < 4; ++t) acc = __builtin_fmaf(q0[t], (float)k8[t], acc);
#pragma unroll
                    for (int t = 0; t < 4; ++t) acc = __builtin_fmaf(q1[t], (float)k8[4 + t], acc);
                }
            }
            s2 = acc * scale_log2;
        }
        const float bm = generic_wave_max(s2);  // finite: key key0 (lane 0) is visible
        const float mn = fmaxf(m, bm);
        const float p = j < n ? fast_exp2(s2 - mn) : 0.0f;
        const float alpha = fast_exp2(m - mn);  // m = -inf on the first block: 0
        l = l * alpha + generic_wave_sum(p);
        m = mn;
        lds.p[wave][lane] = p;
        // The wave's lanes read each other's p: LDS operations of one wave complete in order,
        // so this only keeps the compiler from moving the reads above the write.
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int i = 0; i < kGenericMaxHeadDim / 64; ++i) o[i] *= alpha;
        // P.V: lane d takes dims d, d + 64, ...; 16 keys (one page) at a time
        const int kend = min(64, n - key0);
        for (int pp = 0; pp * kPageTokens < kend; ++pp) {
            const int pk = key0 + pp * kPageTokens;  // first key of the page
            // A page wholly at or past astart (hybrid) comes from cur_v alone: neither its
            // table entry nor the pool is read, as in the reference (kernels.cu:2012-2016).
            const bool from_pool = pk < ks.astart;  // uniform
            int64_t base = 0;
            if (from_pool)
                base = block_base(ks.addr, ks.table ? (int64_t)ks.table[pk >> kPageShift]
                                                    : (int64_t)(pk >> kPageShift));
            const float4_t* pw = reinterpret_cast<const float4_t*>(&lds.p[wave][pp * kPageTokens]);
            const float4_t p0 = pw[0], p1 = pw[1], p2 = pw[2], p3 = pw[3];
            const float pv[16] = {p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3],
                                  p2[0], p2[1], p2[2], p2[3], p3[0], p3[1], p3[2], p3[3]};
#pragma unroll
            for (int i = 0; i < kGenericMaxHeadDim / 64; ++i) {
                const int d = lane + 64 * i;
                if (d >= hd) break;
                half8_t v0 = {}, v1 = {};
                if (from_pool) {
                    const half_t* vr = ks.v_pool + base + (int64_t)(head_off + d) * kPageTokens;
                    v0 = *reinterpret_cast<const half8_t*>(vr);
                    v1 = *reinterpret_cast<const half8_t*>(vr + 8);
                }
                float acc = o[i];
#pragma unroll
                for (int s = 0; s < kPageTokens; ++s) {
                    const int key = pk + s;
                    float v = (float)(s < 8 ? v0[s] : v1[s - 8]);
                    if (key >= ks.astart && key < n)
                        v = round_f16(ks.cur_v[(int64_t)(ks.pstart + key - ks.astart) * kv_dim +
                                               head_off + d]);
                    // slots at or past n may hold anything (NaN included): 0 * NaN is NaN
                    acc = __builtin_fmaf(pv[s], key < n ? v : 0.0f, acc);
                }
                o[i] = acc;
            }
        }
    }
    // Merge the waves. A wave without keys has m = -inf, l = 0 and o = 0: weight 0. Wave 0
    // holds key 0, so the merged max is finite.
    if (lane == 0) {
        lds.m[wave] = m;
        lds.l[wave] = l;
    }
#pragma unroll
    for (int i = 0; i < kGenericMaxHeadDim / 64; ++i) {
        const int d = lane + 64 * i;
        if (d < hd) lds.o[wave][d] = o[i];
    }
    __syncthreads();
    for (int d = threadIdx.x; d < hd; d += kGenericThreads) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kGenericWaves; ++w) M = fmaxf(M, lds.m[w]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < kGenericWaves; ++w) {
            const float wt = fast_exp2(lds.m[w] - M);
            L += lds.l[w] * wt;
            O += lds.o[w][d] * wt;
        }
        store(d, O / L);
    }
    __syncthreads();  // lds is free for the caller's next row
}

}  // namespace crucible
