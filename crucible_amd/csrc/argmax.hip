// Greedy token selection on the device: one index per logits row.
//
// Replaces Gpu::argmax_rows (engine/src/gpu.rs:562-580, kernel kernels.cu:1215-1260) with
// the host rule it must agree with, engine/src/sampling.rs:141-150:
//     best = 0; for i: if v[i] > v[best] { best = i }
// i.e. the highest value wins, equal values resolve to the lowest index, -0.0 equals
// +0.0, a NaN never displaces anything, and a NaN at index 0 can never be displaced
// (nothing compares greater than it), so such a row returns 0.
//
// Order-independent form used here: for every non-NaN element build the 64-bit key
//     (order(v) << 32) | (0xffffffff - i)
// where order() maps floats to unsigned integers with the same ordering (and maps -0.0
// to +0.0). The maximum key is the highest value with the lowest index among ties, so a
// plain max-reduction in any order gives the host's answer; the v[0]-is-NaN case is
// checked once per row. One workgroup of 1024 threads per row; each thread keeps four
// loads in flight.
#include "common.hpp"

namespace crucible {
namespace {

constexpr int kArgmaxThreads = 1024;

__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t i) {
    if (v != v) return 0;  // NaN: never a candidate
    uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint64_t)(0xffffffffu - i);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(const float* __restrict__ x,
                                                                   int32_t* __restrict__ out,
                                                                   int64_t cols) {
    __shared__ uint64_t s_key[kArgmaxThreads / 64];
    const float* r = x + (int64_t)blockIdx.x * cols;
    const int t = threadIdx.x;
    uint64_t best = 0;
    int64_t i = t;
    for (; i + 3 * kArgmaxThreads < cols; i += 4 * kArgmaxThreads) {
        const float v0 = r[i], v1 = r[i + kArgmaxThreads], v2 = r[i + 2 * kArgmaxThreads],
                    v3 = r[i + 3 * kArgmaxThreads];
        best = max_u64(best, argmax_key(v0, (uint32_t)i));
        best = max_u64(best, argmax_key(v1, (uint32_t)(i + kArgmaxThreads)));
        best = max_u64(best, argmax_key(v2, (uint32_t)(i + 2 * kArgmaxThreads)));
        best = max_u64(best, argmax_key(v3, (uint32_t)(i + 3 * kArgmaxThreads)));
    }
    for (; i < cols; i += kArgmaxThreads) best = max_u64(best, argmax_key(r[i], (uint32_t)i));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) best = max_u64(best, __shfl_xor(best, off));
    if ((t & 63) == 0) s_key[t >> 6] = best;
    __syncthreads();
    if (t == 0) {
        uint64_t k = s_key[0];
#pragma unroll
        for (int w = 1; w < kArgmaxThreads / 64; ++w) k = max_u64(k, s_key[w]);
        const float v0 = r[0];
        // all-NaN rows (k == 0) and rows whose first element is NaN answer 0
        out[blockIdx.x] = (k == 0 || v0 != v0) ? 0 : (int32_t)(0xffffffffu - (uint32_t)k);
    }
}

}  // namespace
}  // namespace crucible

using namespace crucible;

extern "C" int crucible_argmax_rows(const float* x, int32_t* out, int64_t rows, int64_t cols,
                                    crucible_stream_t stream) {
    const char* what = "argmax_rows";
    CRUCIBLE_CHECK(rows >= 0 && rows <= INT32_MAX && cols > 0 && cols < 0xffffffffLL,
                   CRUCIBLE_ERR_INVALID, "%s: rows=%lld cols=%lld", what, (long long)rows,
                   (long long)cols);
    if (rows == 0) return CRUCIBLE_OK;
    CRUCIBLE_CHECK(x && out, CRUCIBLE_ERR_INVALID, "%s: null buffer", what);
    hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)rows), dim3(kArgmaxThreads), 0, stream,
                       x, out, cols);
    return fail_launch(what);
}
