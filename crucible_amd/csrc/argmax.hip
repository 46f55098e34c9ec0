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
// checked once per row. One workgroup of 1024 threads per row; each thread keeps up to 50
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

// Index of the row's maximum by the host rule, in thread 0 (other threads: unspecified).
// Each thread scans its columns in increasing order keeping (value, index) of its first
// maximum: a strict `>` never takes a NaN, keeps the earlier of equal values and treats
// -0.0 and +0.0 as equal, which is the host rule within the thread (a compare and two
// selects per element, where a 64-bit key per element costs about ten instructions and
// made one row's scan VALU-bound on its CU). The threads' winners then meet as 64-bit
// keys. Each pass issues all of a thread's loads at once (50: one pass covers 51,200
// columns, the 50,257-word vocabulary included, within 105 VGPRs); loads past the row end
// are predicated off.
__device__ __forceinline__ int32_t row_argmax(const float* __restrict__ r, int64_t cols) {
    __shared__ uint64_t s_key[kArgmaxThreads / 64];
    const int t = threadIdx.x;
    const int n = (int)cols;  // < 2^31 (the launchers check)
    float bv = -INFINITY;
    int bi = -1;  // no candidate yet
    constexpr int kU = 50;
    for (int i0 = t; i0 < n; i0 += kU * kArgmaxThreads) {
        float v[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int i = i0 + u * kArgmaxThreads;
            v[u] = i < n ? r[i] : -INFINITY;
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const bool take = v[u] > bv;
            bv = take ? v[u] : bv;
            bi = take ? i0 + u * kArgmaxThreads : bi;
        }
    }
    // A thread that saw nothing above -inf offers no candidate: under the host rule a -inf
    // (or NaN) element never displaces index 0, so a row whose maximum is -inf answers 0,
    // as an empty key set does below.
    uint64_t best = bi < 0 ? 0 : argmax_key(bv, (uint32_t)bi);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) best = max_u64(best, __shfl_xor(best, off));
    if ((t & 63) == 0) s_key[t >> 6] = best;
    __syncthreads();
    int32_t idx = 0;
    if (t == 0) {
        uint64_t k = s_key[0];
#pragma unroll
        for (int w = 1; w < kArgmaxThreads / 64; ++w) k = max_u64(k, s_key[w]);
        const float v0 = r[0];
        // all-NaN rows (k == 0) and rows whose first element is NaN answer 0
        idx = (k == 0 || v0 != v0) ? 0 : (int32_t)(0xffffffffu - (uint32_t)k);
    }
    return idx;
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(const float* __restrict__ x,
                                                                   int32_t* __restrict__ out,
                                                                   int64_t cols) {
    const int32_t idx = row_argmax(x + (int64_t)blockIdx.x * cols, cols);
    if (threadIdx.x == 0) out[blockIdx.x] = idx;
}

// The greedy decode step's tail, one workgroup per row (see crucible_greedy_advance).
__global__ __launch_bounds__(kArgmaxThreads) void greedy_advance_kernel(
    const float* __restrict__ logits, int64_t cols, const float* __restrict__ emb,
    int64_t n_embd, float* __restrict__ x, int64_t ldx, int32_t* __restrict__ tokens,
    int32_t* __restrict__ history, int64_t* step, int64_t max_steps,
    int32_t* __restrict__ positions, int32_t* __restrict__ lens, uint32_t* done, int rows) {
    __shared__ int32_t s_tok;
    const int row = blockIdx.x;
    const int32_t tok = row_argmax(logits + (int64_t)row * cols, cols);
    if (threadIdx.x == 0) {
        s_tok = tok;
        tokens[row] = tok;
        const int64_t st = *step;  // read before this row is counted below
        if (st >= 0 && st < max_steps) history[st * rows + row] = tok;
        positions[row] += 1;
        lens[row] += 1;
    }
    __syncthreads();
    const float* src = emb + (int64_t)s_tok * n_embd;
    float* dst = x + (int64_t)row * ldx;
    for (int64_t k = threadIdx.x; k < n_embd; k += kArgmaxThreads) dst[k] = src[k];
    if (threadIdx.x == 0) {
        // The row that completes the step advances it. Every row has read the step by then:
        // its value was used for the history store before this atomic issued. Relaxed
        // order suffices (what this launch writes reaches the next one at the kernel
        // boundary); acquire-release would write back and invalidate the whole L2 here.
        const uint32_t prev =
            __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == (uint32_t)(rows - 1)) {
            __hip_atomic_store(step, *step + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

}  // namespace
}  // namespace crucible

using namespace crucible;

extern "C" int crucible_argmax_rows(const float* x, int32_t* out, int64_t rows, int64_t cols,
                                    crucible_stream_t stream) {
    const char* what = "argmax_rows";
    CRUCIBLE_CHECK(rows >= 0 && rows <= INT32_MAX && cols > 0 && cols < 0x7fffffffLL,
                   CRUCIBLE_ERR_INVALID, "%s: rows=%lld cols=%lld", what, (long long)rows,
                   (long long)cols);
    if (rows == 0) return CRUCIBLE_OK;
    CRUCIBLE_CHECK(x && out, CRUCIBLE_ERR_INVALID, "%s: null buffer", what);
    hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)rows), dim3(kArgmaxThreads), 0, stream,
                       x, out, cols);
    return fail_launch(what);
}

extern "C" int crucible_greedy_advance(const float* logits, int64_t rows, int64_t cols,
                                       const float* emb, int64_t n_embd, float* x, int64_t ldx,
                                       int32_t* tokens, int32_t* history, int64_t* step,
                                       int64_t max_steps, int32_t* positions, int32_t* lens,
                                       uint32_t* done, crucible_stream_t stream) {
    const char* what = "greedy_advance";
    CRUCIBLE_CHECK(rows >= 0 && rows <= 65535 && cols > 0 && cols < 0x7fffffffLL &&
                       n_embd > 0 && ldx >= n_embd && ldx <= INT32_MAX && max_steps >= 0 &&
                       max_steps <= INT32_MAX,
                   CRUCIBLE_ERR_INVALID, "%s: rows=%lld cols=%lld n_embd=%lld ldx=%lld", what,
                   (long long)rows, (long long)cols, (long long)n_embd, (long long)ldx);
    if (rows == 0) return CRUCIBLE_OK;
    CRUCIBLE_CHECK(logits && emb && x && tokens && step && positions && lens && done &&
                       (history || max_steps == 0),
                   CRUCIBLE_ERR_INVALID, "%s: null buffer", what);
    hipLaunchKernelGGL(greedy_advance_kernel, dim3((unsigned)rows), dim3(kArgmaxThreads), 0,
                       stream, logits, cols, emb, n_embd, x, ldx, tokens, history, step,
                       max_steps, positions, lens, done, (int)rows);
    return fail_launch(what);
}
