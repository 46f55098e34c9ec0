/*
 * CPU oracle for the crucible attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (crucible_amd/, include/)
 * links, loads or calls this file. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, and only as the checker.
 *
 * It restates, in plain scalar C, the arithmetic of the reference engine
 * (Onwcan/crucible, Rust + CUDA) for the attention path:
 *
 *   - paged geometry           engine/kernels/kernels.cu:1630-1638, engine/src/paged.rs:12-21
 *   - KV append scatters       kernels.cu:1079-1092 (contiguous), 1646-1669 (params),
 *                              1713-1731 (rows), 2280-2292 (packed)
 *   - attention (any row)      kernels.cu:1741-1839 (decode), 1844-1948 (prefill),
 *                              engine/src/model.rs:210-235 + ops.rs:67-80 (CPU reference)
 *   - split-K partial/combine  kernels.cu:692-850
 *   - argmax                   engine/src/sampling.rs:141-150
 *   - RoPE table/apply         engine/src/ops.rs:94-136
 *   - generators               engine/src/gpu_attention_validation.rs:40-61 (xorshift,
 *                              counter hash), engine/src/main.rs:1136-1146 (probe tokens)
 *
 * Storage contract: KV pools hold IEEE fp16 bit patterns (uint16_t). The K pool
 * keeps the reference element order [page][layer][16][kv_dim]. The V pool keeps
 * the same (page, layer) blocks but stores each block transposed, [kv_dim][16],
 * so element (slot, c) of a block sits at block_base + c*16 + slot. Page and
 * slot selection -- table[pos >> 4], pos & 15 -- is the reference's, unchanged.
 *
 * Parity pins (what checks each function; see tests/):
 *   f32<->f16        numpy float16 conversion on exhaustive/edge inputs
 *   offsets/append   paged.rs geometry KATs, closed forms, append->gather round trip
 *   dense attention  torch SDPA (library), numpy textbook, uniform/one-hot closed forms
 *   ref-order f32    agrees with the f64 oracle to <= 1e-5
 *   split/combine    equals the unsplit result; chunks past the end are neutral
 *   argmax           the adversarial rows of engine/src/gpu.rs:2295-2399
 *   rope             ops.rs KATs: identity at pos 0, norm preservation
 *   generators       an independent numpy implementation (bitwise)
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, so no FMA contraction
 * changes the reference-order f32 arithmetic).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_PAGE_TOKENS 16
#define ORC_PAGE_SHIFT 4
#define ORC_PAGE_MASK 15

/* ------------------------------------------------------------------------- */
/* fp16 <-> fp32, IEEE binary16, round to nearest even                        */
/* ------------------------------------------------------------------------- */

uint16_t orc_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                     /* inf or NaN */
        if (ax == 0x7f800000u) return sign | 0x7c00u;
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) return sign | 0x7c00u; /* >= 65520 rounds to inf */
    if (ax >= 0x38800000u) {                      /* normal half: |f| >= 2^-14 */
        const uint32_t e = (ax >> 23) - 127 + 15; /* 1..30 */
        const uint32_t mant = ax & 0x7fffffu;
        uint32_t h = (e << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1; /* carry may bump e */
        return (uint16_t)(sign | h);
    }
    /* subnormal half (or zero): value = m * 2^-24, m = rne(|f| * 2^24) in 0..1024 */
    float a;
    memcpy(&a, &ax, 4);
    const float m = nearbyintf(a * 16777216.0f);
    return (uint16_t)(sign | (uint16_t)m);
}

float orc_f16_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    float v;
    if (e == 0) {
        v = ldexpf((float)m, -24);
    } else if (e == 31) {
        uint32_t bits = 0x7f800000u | (m << 13);
        memcpy(&v, &bits, 4);
    } else {
        v = ldexpf((float)(1024u + m), (int)e - 25);
    }
    uint32_t bits;
    memcpy(&bits, &v, 4);
    bits |= sign;
    memcpy(&v, &bits, 4);
    return v;
}

void orc_f32_to_f16_array(const float* src, uint16_t* dst, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_f32_to_f16(src[i]);
}

void orc_f16_to_f32_array(const uint16_t* src, float* dst, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_f16_to_f32(src[i]);
}

/* ------------------------------------------------------------------------- */
/* Paged geometry                                                             */
/* ------------------------------------------------------------------------- */

/* kernels.cu:1630-1638: ((page * n_layer + layer) * PAGE_TOKENS + slot) * kv_dim,
 * evaluated entirely in 64-bit. */
int64_t orc_paged_offset(int64_t page, int64_t slot, int64_t n_layer, int64_t layer,
                         int64_t kv_dim)
{
    return ((page * n_layer + layer) * ORC_PAGE_TOKENS + slot) * kv_dim;
}

/* Element (slot, channel c) of page `page`, layer `layer`, in a pool of kind
 * `v_kind` (0 = K, reference order; 1 = V, block-transposed). */
int64_t orc_pool_index(int v_kind, int64_t page, int64_t slot, int64_t c, int64_t n_layer,
                       int64_t layer, int64_t kv_dim)
{
    const int64_t block = orc_paged_offset(page, 0, n_layer, layer, kv_dim);
    return v_kind ? block + c * ORC_PAGE_TOKENS + slot : block + slot * kv_dim + c;
}

/* Contiguous cache of the same element order: K is [layer][cap][kv_dim], V is
 * [layer][cap/16][kv_dim][16]. `layer_base` = layer * cap * kv_dim. */
int64_t orc_contig_index(int v_kind, int64_t layer_base, int64_t pos, int64_t c, int64_t kv_dim)
{
    const int64_t block = layer_base + (pos >> ORC_PAGE_SHIFT) * ORC_PAGE_TOKENS * kv_dim;
    return v_kind ? block + c * ORC_PAGE_TOKENS + (pos & ORC_PAGE_MASK)
                  : block + (pos & ORC_PAGE_MASK) * kv_dim + c;
}

/* ------------------------------------------------------------------------- */
/* KV append: f32 rows -> fp16 pool                                           */
/* ------------------------------------------------------------------------- */

enum { ORC_STORE_ROWS = 0, ORC_STORE_PARAMS = 1, ORC_STORE_PACKED = 2, ORC_STORE_CONTIG = 3 };
#define ORC_PARAM_PREFILL_POS 5 /* kernels.cu:43, gpu.rs:78 */

/*
 * mode ROWS   (cache_store_rows_paged_f32, kernels.cu:1713-1731):
 *             page = tables[row*stride + (positions[row] >> 4)]
 * mode PARAMS (cache_store_paged_f32, kernels.cu:1646-1669):
 *             pos = params[5] + row, page = tables[pos >> 4]
 * mode PACKED (cache_store_packed_paged_f32, kernels.cu:2280-2292):
 *             page = tables[owners[row]*stride + (positions[row] >> 4)]
 * mode CONTIG (cache_store_f32, kernels.cu:1079-1092):
 *             pos = pos_offset + row, at layer_base
 * src_f16 != NULL means the rows are already fp16 bit patterns.
 */
void orc_cache_store(int mode, int v_kind, const float* src, const uint16_t* src_f16,
                     uint16_t* pool, const int32_t* tables, const int32_t* positions,
                     const int32_t* owners, const int32_t* params, int64_t rows,
                     int64_t kv_dim, int64_t table_stride, int64_t n_layer, int64_t layer,
                     int64_t layer_base, int64_t pos_offset)
{
    for (int64_t r = 0; r < rows; ++r) {
        int64_t pos = 0, page = 0;
        switch (mode) {
        case ORC_STORE_ROWS:
            pos = positions[r];
            page = tables[r * table_stride + (pos >> ORC_PAGE_SHIFT)];
            break;
        case ORC_STORE_PARAMS:
            pos = params[ORC_PARAM_PREFILL_POS] + r;
            page = tables[pos >> ORC_PAGE_SHIFT];
            break;
        case ORC_STORE_PACKED:
            pos = positions[r];
            page = tables[(int64_t)owners[r] * table_stride + (pos >> ORC_PAGE_SHIFT)];
            break;
        default:
            pos = pos_offset + r;
            break;
        }
        for (int64_t c = 0; c < kv_dim; ++c) {
            const uint16_t h = src_f16 ? src_f16[r * kv_dim + c] : orc_f32_to_f16(src[r * kv_dim + c]);
            const int64_t idx = mode == ORC_STORE_CONTIG
                ? orc_contig_index(v_kind, layer_base, pos, c, kv_dim)
                : orc_pool_index(v_kind, page, pos & ORC_PAGE_MASK, c, n_layer, layer, kv_dim);
            pool[idx] = h;
        }
    }
}

/* Gather positions [0, len) of one sequence into dense f32 rows [len][kv_dim]. */
void orc_gather(int v_kind, const uint16_t* pool, const int32_t* table, int64_t len,
                int64_t kv_dim, int64_t n_layer, int64_t layer, float* dense)
{
    for (int64_t p = 0; p < len; ++p) {
        const int64_t page = table[p >> ORC_PAGE_SHIFT];
        for (int64_t c = 0; c < kv_dim; ++c)
            dense[p * kv_dim + c] = orc_f16_to_f32(
                pool[orc_pool_index(v_kind, page, p & ORC_PAGE_MASK, c, n_layer, layer, kv_dim)]);
    }
}

/* Rewrite a V pool (block-transposed) into reference element order, or back. */
void orc_v_blocks_transpose(const uint16_t* src, uint16_t* dst, int64_t blocks, int64_t kv_dim,
                            int to_reference)
{
    const int64_t bs = ORC_PAGE_TOKENS * kv_dim;
    for (int64_t b = 0; b < blocks; ++b)
        for (int64_t s = 0; s < ORC_PAGE_TOKENS; ++s)
            for (int64_t c = 0; c < kv_dim; ++c) {
                const int64_t ref = b * bs + s * kv_dim + c;
                const int64_t vt = b * bs + c * ORC_PAGE_TOKENS + s;
                if (to_reference) dst[ref] = src[vt];
                else dst[vt] = src[ref];
            }
}

/* ------------------------------------------------------------------------- */
/* Attention                                                                  */
/* ------------------------------------------------------------------------- */

/*
 * Dense single-query attention in f64 (the mathematical definition):
 *   s_j = (q . k_j) * scale, j < len;  p = softmax(s);  o = sum_j p_j v_j.
 * k, v are [len][stride] f32 rows; q and o have head_dim entries.
 */
static void attend_one_f64(const float* q, const float* k, const float* v, int64_t len,
                           int64_t stride, int64_t head_dim, double scale, double* scores,
                           float* o, double* o64)
{
    double mx = -INFINITY;
    for (int64_t j = 0; j < len; ++j) {
        double dot = 0.0;
        for (int64_t d = 0; d < head_dim; ++d) dot += (double)q[d] * (double)k[j * stride + d];
        scores[j] = dot * scale;
        if (scores[j] > mx) mx = scores[j];
    }
    double sum = 0.0;
    for (int64_t j = 0; j < len; ++j) {
        scores[j] = exp(scores[j] - mx);
        sum += scores[j];
    }
    for (int64_t d = 0; d < head_dim; ++d) {
        double acc = 0.0;
        for (int64_t j = 0; j < len; ++j) acc += scores[j] * (double)v[j * stride + d];
        if (o) o[d] = (float)(acc / sum);
        if (o64) o64[d] = acc / sum;
    }
}

/*
 * Reference-order f32 attention, engine/src/model.rs:210-235 with
 * engine/src/ops.rs:67-80: f32 dot in ascending d, times f32 scale; softmax with
 * f32 max, f32 exp, f64 sum and f32 normalisation; PV accumulated in f32 in
 * ascending j.
 */
static void attend_one_ref_f32(const float* q, const float* k, const float* v, int64_t len,
                               int64_t stride, int64_t head_dim, float scale, float* scores,
                               float* o)
{
    for (int64_t j = 0; j < len; ++j) {
        float dot = 0.0f;
        for (int64_t d = 0; d < head_dim; ++d) dot += q[d] * k[j * stride + d];
        scores[j] = dot * scale;
    }
    float mx = -INFINITY;
    for (int64_t j = 0; j < len; ++j) mx = scores[j] > mx ? scores[j] : mx;
    double sum = 0.0;
    for (int64_t j = 0; j < len; ++j) {
        scores[j] = expf(scores[j] - mx);
        sum += (double)scores[j];
    }
    const double inv = 1.0 / sum;
    for (int64_t j = 0; j < len; ++j) scores[j] = (float)((double)scores[j] * inv);
    for (int64_t d = 0; d < head_dim; ++d) o[d] = 0.0f;
    for (int64_t j = 0; j < len; ++j)
        for (int64_t d = 0; d < head_dim; ++d) o[d] += scores[j] * v[j * stride + d];
}

/*
 * Dense causal attention over one sequence's K/V rows:
 *   q   [n_q][n_head*head_dim]   query rows
 *   k,v [n_k][n_kv_head*head_dim]
 *   lens[i] = number of visible keys for query row i (causal length)
 *   out [n_q][n_head*head_dim]
 * GQA: head h reads KV head h / (n_head / n_kv_head)  (kernels.cu:1760-1761, model.rs:215-219)
 * precise = 1 -> f64 definition; 0 -> reference-order f32.
 */
int orc_attention_dense(const float* q, const float* k, const float* v, const int32_t* lens,
                        int64_t n_q, int64_t n_k, int64_t n_head, int64_t n_kv_head,
                        int64_t head_dim, double scale, int precise, float* out)
{
    if (n_kv_head <= 0 || n_head % n_kv_head) return -1;
    const int64_t n_rep = n_head / n_kv_head;
    const int64_t kv_dim = n_kv_head * head_dim;
    int rc = 0;
    /* Rows are independent: threads split them, each with its own score buffers, and
     * every value is computed exactly as in the single-threaded loop. */
#pragma omp parallel
    {
        double* s64 = (double*)malloc(sizeof(double) * (size_t)(n_k > 0 ? n_k : 1));
        float* s32 = (float*)malloc(sizeof(float) * (size_t)(n_k > 0 ? n_k : 1));
        if (!s64 || !s32) {
#pragma omp atomic write
            rc = -2;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (int64_t i = 0; i < n_q; ++i) {
                const int64_t len = lens[i];
                if (len <= 0 || len > n_k) continue; /* inactive rows are left untouched */
                for (int64_t h = 0; h < n_head; ++h) {
                    const int64_t g = h / n_rep;
                    const float* qh = q + i * n_head * head_dim + h * head_dim;
                    float* oh = out + i * n_head * head_dim + h * head_dim;
                    if (precise)
                        attend_one_f64(qh, k + g * head_dim, v + g * head_dim, len, kv_dim,
                                       head_dim, scale, s64, oh, NULL);
                    else
                        attend_one_ref_f32(qh, k + g * head_dim, v + g * head_dim, len, kv_dim,
                                           head_dim, (float)scale, s32, oh);
                }
            }
        }
        free(s64);
        free(s32);
    }
    return rc;
}

/*
 * Paged attention, one query row per entry:
 *   row r uses table  tables[(table_index ? table_index[r] : r) * table_stride]
 *   and sees keys     [0, lens[r])   (lens[r] <= 0 -> inactive, out untouched)
 * This single definition covers decode (kernels.cu:1741-1839; lens = seq_lens),
 * packed prefill (kernels.cu:1938-1948; table_index = owners, lens = positions+1)
 * and single-sequence prefill (kernels.cu:1927-1936; lens = params[5]+row+1).
 */
int orc_attention_paged_rows(const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                             const int32_t* tables, const int32_t* table_index,
                             const int32_t* lens, int64_t rows, int64_t n_head,
                             int64_t n_kv_head, int64_t head_dim, int64_t table_stride,
                             int64_t n_layer, int64_t layer, double scale, int precise,
                             float* out)
{
    const int64_t kv_dim = n_kv_head * head_dim;
    int64_t max_len = 0;
    for (int64_t r = 0; r < rows; ++r) max_len = lens[r] > max_len ? lens[r] : max_len;
    if (max_len > table_stride * ORC_PAGE_TOKENS) return -3;
    float* kd = (float*)malloc(sizeof(float) * (size_t)(max_len * kv_dim + 1));
    float* vd = (float*)malloc(sizeof(float) * (size_t)(max_len * kv_dim + 1));
    if (!kd || !vd) { free(kd); free(vd); return -2; }
    int rc = 0;
    for (int64_t r = 0; r < rows && rc == 0; ++r) {
        const int32_t len = lens[r];
        if (len <= 0) continue;
        const int32_t* table = tables + (table_index ? (int64_t)table_index[r] : r) * table_stride;
        orc_gather(0, k_pool, table, len, kv_dim, n_layer, layer, kd);
        orc_gather(1, v_pool, table, len, kv_dim, n_layer, layer, vd);
        rc = orc_attention_dense(q + r * n_head * head_dim, kd, vd, &len, 1, len, n_head,
                                 n_kv_head, head_dim, scale, precise,
                                 out + r * n_head * head_dim);
    }
    free(kd);
    free(vd);
    return rc;
}

/*
 * Split-K partials and combine (kernels.cu:692-850), f64:
 * chunk c covers keys [c*chunk, min((c+1)*chunk, len)). A chunk starting at or past
 * len contributes the neutral partial (m=-inf, l=0, o=0). Partials are
 *   m_c = max_j s_j,  l_c = sum_j e^{s_j - m_c},  o_c = sum_j e^{s_j - m_c} v_j
 * and the combine is m = max m_c, l = sum l_c e^{m_c - m}, out = sum o_c e^{m_c-m} / l.
 */
void orc_split_partials(const float* q, const float* k, const float* v, int64_t len,
                        int64_t stride, int64_t head_dim, double scale, int64_t chunk,
                        int64_t n_chunks, double* pm, double* pl, double* po)
{
    for (int64_t c = 0; c < n_chunks; ++c) {
        const int64_t start = c * chunk;
        pm[c] = -INFINITY;
        pl[c] = 0.0;
        for (int64_t d = 0; d < head_dim; ++d) po[c * head_dim + d] = 0.0;
        if (start >= len) continue;
        const int64_t end = start + chunk < len ? start + chunk : len;
        double mx = -INFINITY;
        for (int64_t j = start; j < end; ++j) {
            double dot = 0.0;
            for (int64_t d = 0; d < head_dim; ++d) dot += (double)q[d] * (double)k[j * stride + d];
            dot *= scale;
            if (dot > mx) mx = dot;
        }
        double l = 0.0;
        for (int64_t j = start; j < end; ++j) {
            double dot = 0.0;
            for (int64_t d = 0; d < head_dim; ++d) dot += (double)q[d] * (double)k[j * stride + d];
            const double e = exp(dot * scale - mx);
            l += e;
            for (int64_t d = 0; d < head_dim; ++d) po[c * head_dim + d] += e * (double)v[j * stride + d];
        }
        pm[c] = mx;
        pl[c] = l;
    }
}

void orc_split_combine(const double* pm, const double* pl, const double* po, int64_t n_chunks,
                       int64_t head_dim, double* out)
{
    double m = -INFINITY;
    for (int64_t c = 0; c < n_chunks; ++c) m = pm[c] > m ? pm[c] : m;
    double l = 0.0;
    for (int64_t c = 0; c < n_chunks; ++c)
        if (pl[c] > 0.0) l += pl[c] * exp(pm[c] - m);
    for (int64_t d = 0; d < head_dim; ++d) {
        double acc = 0.0;
        for (int64_t c = 0; c < n_chunks; ++c)
            if (pl[c] > 0.0) acc += po[c * head_dim + d] * exp(pm[c] - m);
        out[d] = acc / l;
    }
}

/* ------------------------------------------------------------------------- */
/* Greedy selection, RoPE                                                      */
/* ------------------------------------------------------------------------- */

/* sampling.rs:141-150: best = 0; for i: if v[i] > v[best] { best = i } */
int64_t orc_argmax(const float* v, int64_t n)
{
    int64_t best = 0;
    for (int64_t i = 0; i < n; ++i)
        if (v[i] > v[best]) best = i;
    return best;
}

/* ops.rs:99-115: tables [max_seq][head_dim/2], angle computed in f64, stored f32. */
void orc_rope_table(int64_t head_dim, int64_t max_seq, double theta, float* cos_t, float* sin_t)
{
    const int64_t half = head_dim / 2;
    for (int64_t pos = 0; pos < max_seq; ++pos)
        for (int64_t i = 0; i < half; ++i) {
            const double inv_freq = pow(theta, -((double)(2 * i)) / (double)head_dim);
            const double angle = (double)pos * inv_freq;
            cos_t[pos * half + i] = (float)cos(angle);
            sin_t[pos * half + i] = (float)sin(angle);
        }
}

/* ops.rs:124-136: half-split rotation, element i pairs with i + head_dim/2. */
void orc_rope_apply(float* v, int64_t head_dim, const float* cos_t, const float* sin_t, int64_t pos)
{
    const int64_t half = head_dim / 2;
    for (int64_t i = 0; i < half; ++i) {
        const float c = cos_t[pos * half + i];
        const float s = sin_t[pos * half + i];
        const float lo = v[i];
        const float hi = v[i + half];
        v[i] = lo * c - hi * s;
        v[i + half] = lo * s + hi * c;
    }
}

/* ------------------------------------------------------------------------- */
/* Generators                                                                 */
/* ------------------------------------------------------------------------- */

/* gpu_attention_validation.rs:40-45 and main.rs:1136-1146 (xorshift64 13/7/17). */
uint64_t orc_xorshift(uint64_t* state)
{
    *state ^= *state << 13;
    *state ^= *state >> 7;
    *state ^= *state << 17;
    return *state;
}

/* main.rs:1136-1146: probe tokens from state 0x9E3779B97F4A7C15. */
void orc_probe_tokens(int64_t n, int64_t vocab, int64_t* out)
{
    uint64_t state = 0x9E3779B97F4A7C15ull;
    for (int64_t i = 0; i < n; ++i) out[i] = (int64_t)(orc_xorshift(&state) % (uint64_t)vocab);
}

/* gpu_attention_validation.rs:131-136: Fisher-Yates over 0..n with xorshift,
 * state = max(seed, 1). */
void orc_shuffle(uint64_t seed, int64_t n, int64_t* out)
{
    for (int64_t i = 0; i < n; ++i) out[i] = i;
    uint64_t state = seed ? seed : 1;
    for (int64_t i = n - 1; i >= 1; --i) {
        const int64_t j = (int64_t)(orc_xorshift(&state) % (uint64_t)(i + 1));
        const int64_t t = out[i];
        out[i] = out[j];
        out[j] = t;
    }
}

/* gpu_attention_validation.rs:47-61: counter-based value in [-1, 1). */
float orc_value(uint64_t id, uint64_t pos, uint64_t head, uint64_t dim, uint64_t salt)
{
    uint64_t v = salt ^ ((id + 1) * 0x9e3779b97f4a7c15ull) ^ ((pos + 1) * 0xbf58476d1ce4e5b9ull)
               ^ ((head + 1) * 0x94d049bb133111ebull) ^ ((dim + 1) * 0xd6e8feb86659fd93ull);
    v ^= v >> 30;
    v *= 0xbf58476d1ce4e5b9ull;
    v ^= v >> 27;
    v *= 0x94d049bb133111ebull;
    v ^= v >> 31;
    return ((float)(v >> 40) / 16777216.0f) * 2.0f - 1.0f;
}

/* splitmix64 (Steele, Lea, Flood 2014): state += golden gamma, then mix. */
uint64_t orc_splitmix64(uint64_t* state)
{
    uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

/*
 * The build's seeded N(0,1) stream: element i uses splitmix64 outputs
 * x = sm(seed, 2i+1), y = sm(seed, 2i+2) of the counter stream, i.e. the state
 * seed + k*gamma before mixing. u1 = (1 + (x >> 11)) * 2^-53 in (0, 1],
 * u2 = (y >> 11) * 2^-53 in [0, 1), z = sqrt(-2 ln u1) cos(2 pi u2) in f64,
 * rounded to f32. Element i depends only on (seed, i), so any slice can be
 * produced independently (the device generator does exactly that).
 */
void orc_normal_f32(uint64_t seed, int64_t start, int64_t n, float* out)
{
    for (int64_t i = 0; i < n; ++i) {
        uint64_t st = seed + (uint64_t)(2 * (start + i)) * 0x9e3779b97f4a7c15ull;
        const uint64_t x = orc_splitmix64(&st);
        const uint64_t y = orc_splitmix64(&st);
        const double u1 = (double)((x >> 11) + 1) * 0x1.0p-53;
        const double u2 = (double)(y >> 11) * 0x1.0p-53;
        out[i] = (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2));
    }
}

/* The same stream, rounded to fp16 (RNE of the f32 value). */
void orc_normal_f16(uint64_t seed, int64_t start, int64_t n, uint16_t* out)
{
    for (int64_t i = 0; i < n; ++i) {
        float f;
        orc_normal_f32(seed, start + i, 1, &f);
        out[i] = orc_f32_to_f16(f);
    }
}

/* orc_value over a grid: out[p][h][d] = value(id, pos0 + p, h, d, salt). */
void orc_value_grid(uint64_t id, int64_t pos0, int64_t n_pos, int64_t n_head, int64_t head_dim,
                    uint64_t salt, float* out)
{
    for (int64_t p = 0; p < n_pos; ++p)
        for (int64_t h = 0; h < n_head; ++h)
            for (int64_t d = 0; d < head_dim; ++d)
                out[(p * n_head + h) * head_dim + d] =
                    orc_value(id, (uint64_t)(pos0 + p), (uint64_t)h, (uint64_t)d, salt);
}
