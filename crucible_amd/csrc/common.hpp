// Shared definitions for the gfx950 attention kernels and their C-ABI wrappers.
//
// Page geometry follows the reference engine exactly (engine/kernels/kernels.cu:1630-1638,
// engine/src/paged.rs:12-21): 16-token pages, page = table[pos >> 4], slot = pos & 15,
// block(page, layer) = ((page * n_layer + layer) * 16) * kv_dim elements. All offsets are
// formed in 64-bit. Inside a block, K keeps the reference order [16][kv_dim] and V is
// stored transposed, [kv_dim][16], so a V page slice is already the A operand of the PV
// matrix product.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/crucible_attn.h"

namespace crucible {

constexpr int kPageTokens = 16;
constexpr int kPageShift = 4;
constexpr int kPageMask = 15;
constexpr int kHeadDim = 64;
constexpr int kParamPrefillPos = CRUCIBLE_PARAM_PREFILL_POS;
constexpr int kParamSeq = CRUCIBLE_PARAM_SEQ;

typedef _Float16 half_t;
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- addressing

// How a kernel finds the fp16 rows of position `pos` for layer `layer`:
//   paged:      block = table[pos >> 4] * page_stride + layer_off
//   contiguous: block = (pos >> 4) * page_stride + layer_off   (table == nullptr)
// page_stride = n_layer * 16 * kv_dim (paged) or 16 * kv_dim (contiguous);
// layer_off = layer * 16 * kv_dim (paged) or layer_base (contiguous).
struct PoolAddr {
    int64_t page_stride;
    int64_t layer_off;
    int32_t kv_dim;
};

__device__ __forceinline__ int64_t block_base(const PoolAddr& a, int64_t page) {
    return page * a.page_stride + a.layer_off;
}

// ---------------------------------------------------------------- math

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Max and sum of a value over a lane's 4 lane groups (lanes L, L ^ 16, L ^ 32, L ^ 48):
// v_permlane16_swap / v_permlane32_swap of the value with a copy of itself (one operand
// ends with v[L], the other with v[L ^ 16], resp. v[L ^ 32]), then a max or an add. The
// shuffles they replace go through LDS (ds_bpermute). The swap needs 2 wait states around
// its VALU neighbours; the block opens with 1 for a v_exp_f32 result it may read. The sum
// adds the same pairs in the same grouping as two xor shuffles, (x + x^16) + (x^32 + x^48),
// so its bits do not change.
__device__ __forceinline__ float group_max4(float x) {
    float t;
    asm("s_nop 0\n\t"
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
        : "+v"(x), "=&v"(t));
    return x;
}

__device__ __forceinline__ float group_sum4(float x) {
    float t;
    asm("s_nop 0\n\t"
        "v_mov_b32 %1, %0\n\t"
        "s_nop 1\n\t"
        "v_permlane16_swap_b32 %0, %1\n\t"
        "s_nop 1\n\t"
        "v_add_f32 %0, %0, %1\n\t"
        "v_mov_b32 %1, %0\n\t"
        "s_nop 1\n\t"
        "v_permlane32_swap_b32 %0, %1\n\t"
        "s_nop 1\n\t"
        "v_add_f32 %0, %0, %1"
        : "+v"(x), "=&v"(t));
    return x;
}

// P as fp16 hi + lo (the operand pairs of the PV products): hi = v_cvt_pkrtz (round toward
// zero) of a pair of values, and lo = RNE(p - hi) from v_fma_mix{lo,hi}_f16, which take hi
// as an fp16 operand, form p - hi exactly in f32 and round once to fp16 into one half of the
// packed result (one instruction per value where the C form needs a convert, a subtract
// and half a pack). hi + lo carries p to about 2^-22 relative.
//
// It reads v_exp_f32 results (1 wait state) and an MFMA reads what it writes (2 wait
// states): the block opens with s_nop 0 and ends with s_nop 1.
__device__ __forceinline__ void split_lo4(const float (&p)[4], uint32_t h01, uint32_t h23,
                                          uint32_t& lo01, uint32_t& lo23) {
    asm("s_nop 0\n\t"
        "v_fma_mixlo_f16 %0, %2, -1.0, %4 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %0, %2, -1.0, %5 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixlo_f16 %1, %3, -1.0, %6 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %1, %3, -1.0, %7 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "s_nop 1"
        : "=&v"(lo01), "=&v"(lo23)
        : "v"(h01), "v"(h23), "v"(p[0]), "v"(p[1]), "v"(p[2]), "v"(p[3]));
}

__device__ __forceinline__ float4_t mfma_16x16x32(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float4_t mfma_16x16x16(half4_t a, half4_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// Raw buffer resource over [base, base + bytes) for 16-byte loads and stores that carry a
// cache policy (word 3 is the gfx9 raw-buffer format). Accesses past `bytes` are dropped
// (stores) or read zero (loads).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// Cache policy sc1: agent-scope coherent (write-through stores, loads that do not hit
// another XCD's stale L2 line).
constexpr int kPolicyCoherent = 16;

// Direct-to-LDS 16-byte load: every lane of the wave moves 16 bytes from `src` to
// LDS byte offset lds_base + 16 * lane (global_load_lds_dwordx4, M0 = lds_base, which
// must be wave-uniform). Issued through inline asm so the compiler does not track the
// LDS write: the caller orders it with its own s_waitcnt vmcnt + s_barrier, which lets
// several tiles stay in flight while earlier ones are read (the compiler would otherwise
// wait for every outstanding load before each LDS read). An SALU write of M0 needs one
// wait state before a load with LDS reads it (s_nop 0); the compiler adds none inside asm.
__device__ __forceinline__ void lds_dma16(const void* src, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(src), "s"(lds_base)
                 : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}

// log2(e): softmax is evaluated as 2^(s * scale * log2e - m) with m in the same units.
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- host side

void set_error(int status, const char* fmt, ...);
int fail_launch(const char* what);
// Current value of a launch-shape override (CRUCIBLE_TUNE_*), -1 for the automatic choice.
int tuning(int key);
// CUs of the current device (256 on MI355X), queried once per device: the launch-shape
// choices compare grids against it.
int device_cu_count();
// a * b * c for non-negative factors, or -1 when a factor is negative or the product does
// not fit int64 (argument validation computes sizes with it before anything uses them)
inline int64_t checked_mul(int64_t a, int64_t b, int64_t c = 1) {
    int64_t r;
    if (a < 0 || b < 0 || c < 0 || __builtin_mul_overflow(a, b, &r) ||
        __builtin_mul_overflow(r, c, &r))
        return -1;
    return r;
}
// The element offsets of a paged pool: layer `layer`'s block of page p starts at
// p * page_stride + layer_off. False when the layer is outside n_layer or a page id up to
// INT32_MAX (any int32 table entry) would not give an int64 offset.
inline bool paged_addr(int64_t n_layer, int64_t layer, int64_t kv_dim, PoolAddr& out) {
    const int64_t stride = checked_mul(n_layer, kPageTokens, kv_dim);
    if (stride <= 0 || checked_mul(stride, INT32_MAX) < 0 || layer < 0 || layer >= n_layer)
        return false;
    out.page_stride = stride;
    out.layer_off = layer * kPageTokens * kv_dim;  // below stride
    return true;
}
inline bool dtype_ok(int d) { return d == CRUCIBLE_F32 || d == CRUCIBLE_F16; }
inline bool kind_ok(int k) { return k == CRUCIBLE_POOL_K || k == CRUCIBLE_POOL_V; }

}  // namespace crucible

#define CRUCIBLE_CHECK(cond, status, ...)                 \
    do {                                                  \
        if (!(cond)) {                                    \
            ::crucible::set_error((status), __VA_ARGS__); \
            return (status);                              \
        }                                                 \
    } while (0)
