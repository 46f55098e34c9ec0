/*
 * crucible_attn.h -- C ABI of the MI355X (gfx950) attention hot path.
 *
 * Drop-in boundary for the attention and KV-append methods of the reference
 * engine's GPU backend (Onwcan/crucible, engine/src/gpu.rs, `impl Gpu`). Each
 * entry point below names the method it replaces. Argument order and meaning
 * follow the reference; sizes are int64_t where the reference takes usize.
 *
 * Conventions
 *   - Every pointer is a device pointer unless stated otherwise. The caller owns
 *     every buffer; no entry point allocates device memory, synchronises, or
 *     copies host<->device. Every entry point enqueues on `stream` and returns.
 *   - Per-step values (positions, lengths, page tables, params) are read from
 *     device memory, never passed by value, so hipGraph capture of a step stays
 *     valid across replays (kernels.cu:17-35 in the reference).
 *   - Read-only metadata: page tables, seq_lens, positions, owners, segments and
 *     params are read through the scalar (constant) cache, which does not see
 *     writes made during the same launch. They must stay unchanged while a launch
 *     runs and must not overlap `out`, the pools, the workspace or any other buffer
 *     the launch writes. The library checks none of this; an overlap gives stale
 *     reads, not a fault.
 *   - Return value: CRUCIBLE_OK (0) or an error code. Argument validation
 *     happens before any launch; on error nothing is enqueued. The message of
 *     the last error on the calling thread is available from
 *     crucible_attn_last_error(). Sizes are bounded so that no offset a kernel
 *     computes can overflow int64: counts of rows, requests, positions, strides and
 *     leading dimensions at most INT32_MAX, n_head at most 2^20, and a paged pool's
 *     page stride (n_layer * 16 * kv_dim elements) such that any int32 page id gives
 *     an int64 offset.
 *   - Page geometry is the reference's: 16-token pages, page = table[pos >> 4],
 *     slot = pos & 15, and a page holds every layer. Element offsets of the
 *     (page, layer) block are ((page * n_layer + layer) * 16) * kv_dim.
 *   - Page layout (the one change the north star allows): K pools keep the
 *     reference element order inside a block, [16][kv_dim]. V pools store each
 *     block transposed, [kv_dim][16]; element (slot, c) is at block + c*16 + slot.
 *     KV pools hold IEEE fp16. Pool sizes are unchanged.
 *   - Contiguous caches (the reference's non-paged oracle path) use the same
 *     element order with pages numbered pos >> 4 inside a layer region:
 *     K [layer][cap][kv_dim], V [layer][cap/16][kv_dim][16]; `layer_base` is
 *     layer * cap * kv_dim as in the reference.
 */
#ifndef CRUCIBLE_ATTN_H
#define CRUCIBLE_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same type as HIP's hipStream_t; NULL is the default stream. */
typedef struct ihipStream_t* crucible_stream_t;

enum crucible_status {
    CRUCIBLE_OK = 0,
    CRUCIBLE_ERR_INVALID = 1,     /* argument failed validation; nothing launched */
    CRUCIBLE_ERR_UNSUPPORTED = 2, /* geometry this build does not implement */
    CRUCIBLE_ERR_WORKSPACE = 3,   /* workspace missing or smaller than required */
    CRUCIBLE_ERR_LAUNCH = 4       /* the HIP runtime rejected a launch */
};

enum crucible_dtype { CRUCIBLE_F32 = 0, CRUCIBLE_F16 = 1 };
enum crucible_pool_kind { CRUCIBLE_POOL_K = 0, CRUCIBLE_POOL_V = 1 };

/* Index of the prefill position offset in the device params buffer
 * (gpu.rs:78 PARAM_PREFILL_POS, kernels.cu:43). */
#define CRUCIBLE_PARAM_PREFILL_POS 5
/* Index of the visible length in the params buffer (gpu.rs:70 PARAM_SEQ). */
#define CRUCIBLE_PARAM_SEQ 3
#define CRUCIBLE_PAGE_TOKENS 16

/* ------------------------------------------------------------------ library */

/* Version string of this library (static storage). */
const char* crucible_attn_version(void);

/* Launch-shape overrides, for tests and tuning sweeps. Every entry point picks its
 * kernel shape on its own; a key set to a value other than -1 forces that choice for
 * every later launch in the process. Each key starts at the value of its environment
 * variable (crucible_attn_tuning_name), read once per process; unset or unparsable
 * means -1. Values that a key does not accept are rejected with CRUCIBLE_ERR_INVALID.
 * The setting is process-wide: change it only while no other thread launches. */
enum crucible_tuning_key {
    CRUCIBLE_TUNE_DECODE_PAGES = 0,        /* decode pages per wave: 1, 2, 4 */
    CRUCIBLE_TUNE_DECODE_WAVES = 1,        /* decode waves per workgroup: 4, 8 */
    CRUCIBLE_TUNE_DECODE_ORDER = 2,        /* decode grid order: 0 split, 1 request, 2 compact */
    CRUCIBLE_TUNE_PREFILL_DIRECT = 3,      /* prefill register-direct form: 0, 1 */
    CRUCIBLE_TUNE_PREFILL_HEAVY_FIRST = 4, /* prefill longest-first grid: 0, 1 */
    CRUCIBLE_TUNE_PREFILL_QB = 5,          /* prefill 16-row blocks per wave: 1, 2 */
    CRUCIBLE_TUNE_PREFILL_BUFS = 6,        /* prefill LDS ring depth in key tiles: 4, 6 */
    CRUCIBLE_TUNE_LINEAR_TILE = 7,         /* projection tiles: 4 or 16 columns (decode), 32 (prompt rows) */
    CRUCIBLE_TUNE_DECODE_COMBINE_WIDTH = 8, /* decode splits merged per round trip: 8, 16 */
    CRUCIBLE_TUNE_PREFILL_P16 = 9,         /* prefill P operand: 0 fp16 hi + lo (default), 1 one fp16 */
    CRUCIBLE_TUNE_PREFILL_M32 = 10,        /* prefill 32-row waves on 32x32 MFMAs: 1 (default), 0 */
    CRUCIBLE_TUNE_PREFILL_PERSIST = 11,    /* prefill persistent 16-row LDS form for segment rows
                                              (a static longest-first list of the row tiles that
                                              hold rows): 0 off (default), 1 one workgroup per
                                              resident slot, n >= 2 a grid of n workgroups */
    CRUCIBLE_TUNE_LINEAR_PREFETCH = 12,    /* the _prefetch projections' next-kernel prefetch:
                                              1 on (default), 0 off */
    CRUCIBLE_TUNE_COUNT = 13
};
int crucible_attn_set_tuning(int key, int value);
/* Current value of a key (-1: automatic, or an unknown key). */
int crucible_attn_get_tuning(int key);
/* Name of a key's environment variable (static storage), NULL for an unknown key. */
const char* crucible_attn_tuning_name(int key);

/* Copy the calling thread's last error message into buf (NUL-terminated,
 * truncated to n). Returns the status of that error (CRUCIBLE_OK if none). */
int crucible_attn_last_error(char* buf, size_t n);

/* ------------------------------------------------------------------ KV append
 * src is [rows][kv_dim] in src_dtype; f32 values are rounded to fp16 (RNE).
 * `kind` says which pool layout `pool` has (K or V).
 */

/* Replaces Gpu::cache_store (gpu.rs:1259-1279; kernel kernels.cu:1079-1092):
 * contiguous cache, position pos_offset + row, layer region at layer_base. */
int crucible_cache_store(const void* src, int src_dtype, void* cache, int kind,
                         int64_t rows, int64_t kv_dim, int64_t layer_base,
                         int64_t pos_offset, crucible_stream_t stream);

/* Replaces Gpu::cache_store_paged (gpu.rs:1281-1307; kernels.cu:1646-1669):
 * one sequence's table, position params[5] + row. */
int crucible_cache_store_paged(const void* src, int src_dtype, void* pool, int kind,
                               const int32_t* page_table, int64_t rows, int64_t kv_dim,
                               int64_t n_layer, int64_t layer, const int32_t* params,
                               crucible_stream_t stream);

/* Replaces Gpu::cache_store_rows_paged (gpu.rs:1405-1439; kernels.cu:1713-1731):
 * row r at positions[r] through page_tables[r * table_stride + ...]. */
int crucible_cache_store_rows_paged(const void* src, int src_dtype, void* pool, int kind,
                                    const int32_t* page_tables, const int32_t* positions,
                                    int64_t rows, int64_t kv_dim, int64_t table_stride,
                                    int64_t n_layer, int64_t layer, crucible_stream_t stream);

/* Replaces Gpu::cache_store_packed_paged (gpu.rs:1800-1835; kernels.cu:2280-2292):
 * row r at positions[r] through tables[owners[r] * table_stride + ...]. */
int crucible_cache_store_packed_paged(const void* src, int src_dtype, void* pool, int kind,
                                      const int32_t* tables, const int32_t* owners,
                                      const int32_t* positions, int64_t rows, int64_t kv_dim,
                                      int64_t table_stride, int64_t n_layer, int64_t layer,
                                      crucible_stream_t stream);

/* ------------------------------------------------------------------ decode
 * q is [batch][n_head * head_dim] (q_dtype), out is [batch][n_head * head_dim]
 * (out_dtype). n_head is a multiple of n_kv_head; query head h reads KV head
 * h / (n_head / n_kv_head). head_dim 64 (every preset) runs the MFMA kernels, with
 * n_head / n_kv_head <= 16. Any other head_dim that is a multiple of 8 up to 256 runs a
 * generic kernel (one workgroup per request and query head, f32 arithmetic, same pool
 * layout and the same results to the tolerance of f32 accumulation); it uses no
 * workspace, the fused entries run their appends as two cache_store_rows_paged launches
 * (RoPE rows: one append launch) before it, and attention_split leaves its partial
 * buffers untouched. The same holds for the prefill entries below.
 * The split-K partials live in a caller-provided workspace of at least
 * crucible_attention_decode_workspace_bytes(...) bytes (no allocation here; 0 for an
 * empty batch, SIZE_MAX for a shape past the entry points' limits), 16-byte aligned.
 * It starts with a fixed region of 65536 u32 counters, one per (request, kv head) (so
 * batch * n_kv_head <= 65536; one per 64-byte line while batch * n_kv_head <= 4096,
 * so that the splits' atomics on different counters do not queue on one line), that
 * order the in-kernel combine of the splits: zero the workspace once when it is
 * allocated; every launch leaves the counters zeroed again. A unit plan follows, also
 * at a fixed place (1.5 MiB): launches of batch <= 64 in the compact grid order record there
 * which (request, kv head, split) each workgroup served and its page ids, with
 * the lengths, positions and launch shape they came from; a later launch on the
 * same workspace whose lengths, positions and shape are equal loads its unit in
 * the round trip that loads the lengths instead of searching for it. Page ids
 * are still read from the table on every launch (beside the page loads, which
 * are reissued if an id changed), so a rewritten table is always honoured; the
 * plan only saves the search. An entry is used only for the same table address and
 * the same k_pool and v_pool addresses. Its page ids are loaded from before they are
 * checked, so one case is left to the caller: a pool freed and allocated again, smaller,
 * at the same address, served by a table at its old address. Zero the workspace again
 * (or use another) when a pool is reallocated; pools allocated once, as the reference
 * engine allocates them, never meet this. Calls of any batch size may share one
 * workspace, one launch at a time (launches that share it must be ordered, e.g.
 * on one stream). Two launches that run at once on one workspace (two streams
 * without an event between them) race on the counters and partials: a split can
 * count toward the other launch's combine, which then merges partials that are
 * not yet written or belong to the other call. The result is wrong output, and a
 * counter left nonzero that corrupts later launches too; nothing detects it. Give
 * each stream its own workspace.
 *
 * Ordering of the in-kernel combine: each split writes its partial with
 * agent-coherent (sc1) stores, which bypass the non-coherent per-XCD L2 state, and
 * waits for their acknowledgement (s_waitcnt vmcnt(0)) before one lane increments
 * the counter; the workgroup that completes the count reads the partials with sc1
 * loads, which miss any stale line. The wait is a hardware ordering point, not a
 * C++ fence; the cross-order and repeated-launch bit-identity tests guard it.
 * Verified with the ROCm 7.2 hipcc (AMD clang 22) of this build.
 */

size_t crucible_attention_decode_workspace_bytes(int64_t batch, int64_t n_head,
                                                 int64_t max_seq);

/* Replaces Gpu::attention_decode_paged (gpu.rs:1441-1500; kernels.cu:1741-1839).
 * seq_lens[b] <= 0 marks an inactive request: its output is left untouched. */
int crucible_attention_decode_paged(const void* q, int q_dtype, const void* k_pool,
                                    const void* v_pool, void* out, int out_dtype,
                                    const int32_t* page_tables, const int32_t* seq_lens,
                                    int64_t batch, int64_t n_head, int64_t n_kv_head,
                                    int64_t head_dim, int64_t table_stride, int64_t n_layer,
                                    int64_t layer, int64_t kv_dim, int64_t max_seq,
                                    void* workspace, size_t workspace_bytes,
                                    crucible_stream_t stream);

/* Fused form of the reference's per-layer decode sequence (gpu_model.rs:1434-1507):
 *   Gpu::cache_store_rows_paged(k_new -> k_pool, positions)   (gpu.rs:1405-1439)
 *   Gpu::cache_store_rows_paged(v_new -> v_pool, positions)
 *   Gpu::attention_decode_paged(q, ..., seq_lens)             (gpu.rs:1441-1500)
 * in one launch. Row b < batch is appended at positions[b] (k_new/v_new are
 * [batch][kv_dim] in kv_dtype, rounded to fp16); the pools receive exactly the
 * bytes the two appends write, and `out` is what attention_decode_paged computes
 * after them (seq_lens[b] <= 0: no output for b, the row is still appended).
 * Same workspace as attention_decode_paged. */
int crucible_attention_decode_paged_append(
    const void* q, int q_dtype, const void* k_new, const void* v_new, int kv_dtype,
    void* k_pool, void* v_pool, void* out, int out_dtype, const int32_t* page_tables,
    const int32_t* positions, const int32_t* seq_lens, int64_t batch, int64_t n_head,
    int64_t n_kv_head, int64_t head_dim, int64_t table_stride, int64_t n_layer, int64_t layer,
    int64_t kv_dim, int64_t max_seq, void* workspace, size_t workspace_bytes,
    crucible_stream_t stream);

/* The decode kernel a call would launch for this shape, as profilers name it:
 * "decode_kernel<PAGES, WAVES, QF32, APPEND, PAGED, ORDER, ROPE, CW>" (NUL-terminated,
 * truncated to n). entry: 0 attention_decode_paged, 1 attention_decode_paged_append,
 * 2 attention_decode_qkv_paged_append. Launches nothing. */
int crucible_attention_decode_kernel_name(int64_t batch, int64_t n_head, int64_t n_kv_head,
                                          int64_t max_seq, int q_dtype, int entry, char* buf,
                                          size_t n);

/* No counterpart in the reference. For callers that cannot allocate device memory
 * (code under hipGraph capture, tight serving loops, harnesses that forbid hipMalloc):
 * crucible_attention_decode_paged_append with the split-K scratch taken from a
 * file-scope device array of this library (4 MiB per GPU, held until the process ends)
 * instead of a workspace argument. Same kernels, same results bit for bit. Limits:
 * batch * n_kv_head <= 8192, and batch * n_head * n_splits * 66 * 4 bytes of partials
 * <= 4 MiB - 32 KiB (4,161,536 bytes), where n_splits = ceil(ceil(max_seq / 16) /
 * split pages) and a split is the 8, 16 or 32 pages the decode shape picks from
 * batch * n_kv_head * ceil(max_seq / 16). Batch 16 x 12 query heads (3 or 12 kv heads)
 * fits up to max_seq 20,992 tokens (82 splits of 16 pages); larger calls return
 * CRUCIBLE_ERR_WORKSPACE before any launch. It calls no
 * hipMalloc or hipFree; the first call on a device looks up the array's address and
 * clears its counters with a small kernel on `stream` (under stream capture that clear
 * is recorded into the graph, which is harmless: the counters are zero at load and every
 * launch leaves them zero; a failed lookup is tried again on the next call). Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (several streams, or
 * threads) race and must be ordered by the caller. */
int crucible_attention_decode_paged_append_noalloc(
    const void* q, int q_dtype, const void* k_new, const void* v_new, int kv_dtype,
    void* k_pool, void* v_pool, void* out, int out_dtype, const int32_t* page_tables,
    const int32_t* positions, const int32_t* seq_lens, int64_t batch, int64_t n_head,
    int64_t n_kv_head, int64_t head_dim, int64_t table_stride, int64_t n_layer, int64_t layer,
    int64_t kv_dim, int64_t max_seq, crucible_stream_t stream);

/* The same fused step fed straight from the fused q/k/v projection, with the RoPE of
 * the reference's decode step (rope_rows before the K append and on q, gpu_model.rs:1424-1444;
 * RopeTable::apply, ops.rs:124-135) applied in the same launch. Row b of qkv
 * (f32, row stride qkv_row_stride, a multiple of 4) holds q (n_head*head_dim), k (kv_dim),
 * v (kv_dim). q and k are rotated at positions[b] with rope_cos/rope_sin
 * ([rope_max_pos][head_dim/2] f32, 16-byte aligned, rope_max_pos >= max_seq; both NULL: no
 * rotation), each product
 * and difference rounded on its own. k and v are appended at positions[b] and attention
 * runs over seq_lens[b] keys. Bit-identical to crucible_rope_split_qkv followed by
 * crucible_attention_decode_paged_append. */
int crucible_attention_decode_qkv_paged_append(
    const float* qkv, int64_t qkv_row_stride, const float* rope_cos, const float* rope_sin,
    int64_t rope_max_pos, void* k_pool, void* v_pool, void* out, int out_dtype,
    const int32_t* page_tables, const int32_t* positions, const int32_t* seq_lens, int64_t batch,
    int64_t n_head, int64_t n_kv_head, int64_t head_dim, int64_t table_stride, int64_t n_layer,
    int64_t layer, int64_t kv_dim, int64_t max_seq, void* workspace, size_t workspace_bytes,
    crucible_stream_t stream);

/* Replaces Gpu::attention_decode (gpu.rs:762-817; kernels.cu:288-389): one
 * sequence in a contiguous cache, visible length params[CRUCIBLE_PARAM_SEQ]. */
int crucible_attention_decode(const void* q, int q_dtype, const void* k_cache,
                              const void* v_cache, void* out, int out_dtype, int64_t n_head,
                              int64_t n_kv_head, int64_t head_dim, const int32_t* params,
                              int64_t max_seq, int64_t cache_stride, int64_t layer_base,
                              void* workspace, size_t workspace_bytes,
                              crucible_stream_t stream);

/* Replaces Gpu::attention_split (gpu.rs:1936-2014; kernels.cu:692-850): the
 * flash-decoding form of attention_decode with caller-owned partials, laid out
 * as in the reference: partial_o [n_head][n_chunks][head_dim], partial_m and
 * partial_l [n_head][n_chunks], n_chunks = ceil(capacity / 128). The partial
 * values are internal to the combine; only `out` is part of the contract. */
int crucible_attention_split(const void* q, int q_dtype, const void* k_cache,
                             const void* v_cache, float* partial_o, float* partial_m,
                             float* partial_l, void* out, int out_dtype, int64_t n_head,
                             int64_t n_kv_head, int64_t head_dim, const int32_t* params,
                             int64_t capacity, int64_t cache_stride, int64_t layer_base,
                             crucible_stream_t stream);

/* ------------------------------------------------------------------ prefill
 * Causal attention for query rows whose keys are already in the pool. q is
 * [rows][n_head * head_dim], out likewise. Row r sees keys [0, pos_r].
 * Arithmetic (head_dim 64): QK^T and PV on fp16 MFMAs with f32 accumulation, softmax in
 * f32. P enters the PV product as fp16 hi + lo (about 22 bits; within the reference
 * validator's element gate, 2e-5 + 2e-5|ref|, unwidened). CRUCIBLE_TUNE_PREFILL_P16 = 1
 * carries P as one fp16 operand rounded to nearest even instead: one PV product per block
 * instead of two (about 1.3x faster tile loops on long prompts), and an output then moves
 * by at most 2^-11 sum_i w_i |v_i| from exact softmax weights (max-abs 4.4e-4 over the
 * reference's corpus).
 */

/* Replaces Gpu::attention_prefill_paged (gpu.rs:1502-1549; kernels.cu:1927-1936):
 * one sequence, row r at position params[5] + r. */
int crucible_attention_prefill_paged(const void* q, int q_dtype, const void* k_pool,
                                     const void* v_pool, void* out, int out_dtype,
                                     const int32_t* page_table, int64_t rows, int64_t n_head,
                                     int64_t n_kv_head, int64_t head_dim, int64_t n_layer,
                                     int64_t layer, int64_t kv_dim, int64_t max_seq,
                                     const int32_t* params, crucible_stream_t stream);

/* Replaces Gpu::attention_prefill_packed (gpu.rs:1551-1604; kernels.cu:1938-1948):
 * row r belongs to request owners[r] at position positions[r]. Rows of one
 * request need not be adjacent; adjacent rows of one request share K/V tiles. */
int crucible_attention_prefill_packed(const void* q, int q_dtype, const void* k_pool,
                                      const void* v_pool, void* out, int out_dtype,
                                      const int32_t* tables, const int32_t* owners,
                                      const int32_t* positions, int64_t rows,
                                      int64_t table_stride, int64_t n_head, int64_t n_kv_head,
                                      int64_t head_dim, int64_t n_layer, int64_t layer,
                                      int64_t kv_dim, int64_t max_seq, crucible_stream_t stream);

/* Replaces Gpu::attention_prefill_tiled (gpu.rs:1606-1751; kernels.cu:1950-2276):
 * segments[4*i .. 4*i+3] = {packed_start, chunk_len, absolute_start, table_index}.
 * Query row packed_start + j is at position absolute_start + j. With hybrid = 0 every key
 * comes from the pools (append the chunk first; current_k/current_v are not read). With
 * hybrid = 1 (gpu.rs:1691-1697, kernels.cu:2012-2016) keys at or past a segment's
 * absolute_start come from the chunk's own rows instead: current_k / current_v are f32
 * [packed row][kv_dim], key position p of segment i at packed row packed_start + p -
 * absolute_start, rounded to fp16 as the append stores them (so the result equals the
 * hybrid = 0 result over a pool holding the appended chunk); hybrid launches take the
 * register-direct kernel. score_capacity is validated as in the reference but not needed
 * here. */
int crucible_attention_prefill_tiled(const void* q, int q_dtype, const void* k_pool,
                                     const void* v_pool, const void* current_k,
                                     const void* current_v, void* out, int out_dtype,
                                     const int32_t* tables, const int32_t* segments,
                                     int64_t requests, int64_t max_chunk, int64_t table_stride,
                                     int64_t n_head, int64_t n_kv_head, int64_t head_dim,
                                     int64_t n_layer, int64_t layer, int64_t kv_dim,
                                     int hybrid, int64_t score_capacity,
                                     crucible_stream_t stream);

/* Replaces Gpu::attention_prefill (gpu.rs:1886-1934; kernels.cu:1099-1172):
 * contiguous cache, row r at position pos_offset + r. */
int crucible_attention_prefill(const void* q, int q_dtype, const void* k_cache,
                               const void* v_cache, void* out, int out_dtype, int64_t rows,
                               int64_t n_head, int64_t n_kv_head, int64_t head_dim,
                               int64_t max_seq, int64_t cache_stride, int64_t layer_base,
                               int64_t pos_offset, crucible_stream_t stream);

/* ------------------------------------------------------------------ greedy selection */

/* Replaces Gpu::argmax_rows (gpu.rs:562-580; kernels.cu:1215-1260): out[r] = index of
 * the largest x[r * cols + i], with the host rule of sampling.rs:141-150 (ties to the
 * lowest index, -0.0 == +0.0, NaN never displaces an element, a NaN at index 0 yields
 * 0). x is [rows][cols] f32, out is [rows] int32. */
int crucible_argmax_rows(const float* x, int32_t* out, int64_t rows, int64_t cols,
                         crucible_stream_t stream);

/* The tail of a greedy batched decode step, kept on the device so the step replays as one
 * graph. Replaces argmax_rows at the end of queue_decode_batch (gpu_model.rs:1586), the
 * host's per-step upload of positions and lengths (upload_batch, gpu_model.rs:1088-1147)
 * and the next step's embed_batch (gpu_model.rs:1401). For each row r < rows:
 *   token = argmax(logits[r][0..cols)) by the argmax_rows rule; tokens[r] = token;
 *   history[step * rows + r] = token when 0 <= step < max_steps;
 *   positions[r] += 1; lens[r] += 1; x[r * ldx + k] = emb[token * n_embd + k], k < n_embd;
 * then *step += 1. `done` is a caller-owned u32 that must read 0 before the first call;
 * the call leaves it 0. Calls that overlap on the same buffers race. */
int crucible_greedy_advance(const float* logits, int64_t rows, int64_t cols, const float* emb,
                            int64_t n_embd, float* x, int64_t ldx, int32_t* tokens,
                            int32_t* history, int64_t* step, int64_t max_steps,
                            int32_t* positions, int32_t* lens, uint32_t* done,
                            crucible_stream_t stream);

/* ------------------------------------------------------------------ decode-step glue
 * The projections and row operations that surround attention in the reference's batched
 * decode step (gpu_model.rs:1393-1605 queue_decode_batch), with the reference CPU
 * arithmetic of engine/src/ops.rs so greedy tokens match the CPU model exactly:
 * projections accumulate every product in f64 and round once to f32 (ops.rs:17-32,
 * matvec), where the reference GPU kernels accumulate in f32. Weights are fp16
 * [n_out][k_in] row-major (the reference's [out][in] order); activations are f32.
 */

/* y[m][n] = f32(sum_k f64(w[n][k]) * f64(h[m][k])) for m < rows, n < n_out; replaces the
 * batched GEMV (kernels.cu:1539-1607, gpu.rs gemv_batch) for the q/k/v, o, down and
 * vocabulary projections. h = x, or rmsnorm(x, norm_w, eps) when norm_w is not NULL
 * (ops.rs:39-52: f64 mean of squares, h = f32(f64(x) * scale) * norm_w). out = y, or
 * resid + y when resid is not NULL (the residual add of model.rs:237-241,270-274; resid
 * may equal out, element-wise in place). x [rows][ldx], out and resid [rows][ldo].
 * k_in must be a multiple of 32; x, w and norm_w 16-byte aligned, ldx a multiple of 4. */
int crucible_linear_f64acc(const float* x, int64_t ldx, const float* norm_w, float eps,
                           const void* w, int64_t n_out, int64_t k_in, const float* resid,
                           float* out, int64_t ldo, int64_t rows, crucible_stream_t stream);

/* SwiGLU input of the MLP (model.rs:252-262): out[m][j] = silu(g) * u with
 * g = f64-accumulated rmsnorm(x) . w_gate[j], u = the same with w_up[j], each rounded to
 * f32, and silu(g) = g / (1 + exp(-g)) (ops.rs:83-85). Replaces the gate/up GEMVs and
 * swiglu_batch_f32 (kernels.cu:1038-1047). w_gate, w_up: [hidden][k_in] fp16. */
int crucible_linear_swiglu_f64acc(const float* x, int64_t ldx, const float* norm_w, float eps,
                                  const void* w_gate, const void* w_up, int64_t hidden,
                                  int64_t k_in, float* out, int64_t ldo, int64_t rows,
                                  crucible_stream_t stream);

/* The two products above, with a prefetch of the next kernel's read-only operands: the
 * prefetch_bytes bytes at prefetch (typically the next projection's weights) are read, one
 * word per 64-byte line, by the product's workgroups right after they have issued their own
 * loads, so that the next kernel finds them in the last-level cache instead of waiting a
 * cold HBM round trip. The outputs are those of the plain entry points, bit for bit; only
 * the decode-sized tilings (rows below the prompt-sized GEMM's threshold) issue it, and at
 * most 128 KB a workgroup. prefetch may be NULL with prefetch_bytes 0; otherwise it must be
 * 4-byte aligned and prefetch_bytes a non-negative multiple of 64; its memory must stay
 * allocated until the launch completes. CRUCIBLE_TUNE_LINEAR_PREFETCH = 0 turns the
 * prefetch off. No counterpart in the reference: its decode step launches the same kernels
 * back to back, each waiting for its weights (gpu_model.rs:1393-1605). */
int crucible_linear_f64acc_prefetch(const float* x, int64_t ldx, const float* norm_w, float eps,
                                    const void* w, int64_t n_out, int64_t k_in,
                                    const float* resid, float* out, int64_t ldo, int64_t rows,
                                    const void* prefetch, int64_t prefetch_bytes,
                                    crucible_stream_t stream);
int crucible_linear_swiglu_f64acc_prefetch(const float* x, int64_t ldx, const float* norm_w,
                                           float eps, const void* w_gate, const void* w_up,
                                           int64_t hidden, int64_t k_in, float* out,
                                           int64_t ldo, int64_t rows, const void* prefetch,
                                           int64_t prefetch_bytes, crucible_stream_t stream);

/* RMSNorm of each row (ops.rs:39-52; replaces rmsnorm_batch_f32, kernels.cu:968-996). */
int crucible_rmsnorm_rows(const float* x, int64_t ldx, const float* w, float eps, float* out,
                          int64_t ldo, int64_t rows, int64_t n, crucible_stream_t stream);

/* Split fused [q | k | v] rows (n_head, n_kv_head, n_kv_head heads of head_dim, any even
 * head_dim) into contiguous q [rows][n_head*head_dim], k and v [rows][n_kv_head*head_dim],
 * rotating q and k at
 * positions[row] (RopeTable::apply, ops.rs:124-135; rope_rows_f32, kernels.cu:1677-1706).
 * cos/sin tables are [max_pos][head_dim/2] f32. A position outside [0, max_pos) writes
 * NaN rows. */
int crucible_rope_split_qkv(const float* qkv, int64_t ld, float* q, float* k, float* v,
                            const float* cos_table, const float* sin_table,
                            const int32_t* positions, int64_t rows, int64_t n_head,
                            int64_t n_kv_head, int64_t head_dim, int64_t max_pos,
                            crucible_stream_t stream);

/* ------------------------------------------------------------------ host helpers */

/* Build prefill segments from cumulative sequence offsets (host memory):
 * cu_seqlens[0..n] with cu_seqlens[0] = 0; absolute_starts[i] (NULL = all 0);
 * table i for sequence i. Writes 4*n int32 to segments_out and returns the
 * largest chunk length, or -1 if the offsets are not non-decreasing. */
int64_t crucible_segments_from_cu_seqlens(const int32_t* cu_seqlens, int64_t n,
                                          const int32_t* absolute_starts,
                                          int32_t* segments_out);

/* ------------------------------------------------------------------ paging (host)
 * The reference allocator (engine/src/paged.rs:64-242) restated in C++ for a
 * C/C++ caller: a stack free list (first alloc is page 0), per-sequence tables
 * with all-or-nothing growth, zero-padded device tables. Handles are opaque.
 */
typedef struct crucible_page_pool crucible_page_pool;
typedef struct crucible_seq_pages crucible_seq_pages;

crucible_page_pool* crucible_page_pool_new(int64_t n_pages, int64_t n_layer, int64_t kv_dim);
void crucible_page_pool_free(crucible_page_pool* pool);
int64_t crucible_page_pool_free_pages(const crucible_page_pool* pool);
int64_t crucible_page_pool_used_pages(const crucible_page_pool* pool);
/* Returns the page id, or -1 when exhausted (error message set). */
int64_t crucible_page_pool_alloc(crucible_page_pool* pool);
int crucible_page_pool_release(crucible_page_pool* pool, int64_t page);

crucible_seq_pages* crucible_seq_pages_new(void);
void crucible_seq_pages_free(crucible_seq_pages* seq);
int64_t crucible_seq_pages_len(const crucible_seq_pages* seq);
int64_t crucible_seq_pages_n_pages(const crucible_seq_pages* seq);
int crucible_seq_pages_grow(crucible_seq_pages* seq, crucible_page_pool* pool, int64_t extra);
int crucible_seq_pages_release(crucible_seq_pages* seq, crucible_page_pool* pool);
/* (page, slot) of position pos; returns CRUCIBLE_ERR_INVALID past the end. */
int crucible_seq_pages_translate(const crucible_seq_pages* seq, int64_t pos, int64_t* page,
                                 int64_t* slot);
/* Write the table padded with zeros to `stride` entries (host memory). */
int crucible_seq_pages_table_padded(const crucible_seq_pages* seq, int64_t stride,
                                    int32_t* out);
/* prefill.rs:160-172: ceil((prompt + generated - 1) / 16), or -1 if invalid. */
int64_t crucible_request_page_reservation(int64_t prompt, int64_t generated, int64_t context);

#ifdef __cplusplus
}
#endif

#endif /* CRUCIBLE_ATTN_H */
