// A native (non-Python) caller of the C ABI that runs a small engine step sequence the way
// the reference's GPU model orders it (engine/src/gpu_model.rs: prefill through
// queue_prefill_transformer_impl, :3254-3580, then batched decode steps through
// queue_decode_batch, :1393-1605), for every layer of a 3-layer model:
//   prefill:  crucible_cache_store_packed_paged (K, V) + crucible_attention_prefill_tiled
//   decode:   crucible_attention_decode_paged_append, 4 steps, each one token per request
// Every buffer is hipMalloc'ed by this program; the library allocates nothing. Each launch's
// output is checked against the CPU oracle (oracle/oracle.c, linked as test infrastructure)
// under the reference validator's element gate (|d| <= 2e-5 + 2e-5 |ref|,
// gpu_attention_validation.rs:20-22), and the pools are compared bit for bit with the
// oracle's appends. Prints one line per check; exits 0 when all pass.
//
// Built by __graft_entry__.build() (tests/_build/native_step) and run by
// tests/test_gpu_native_caller.py.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../include/crucible_attn.h"

extern "C" {
// CPU oracle (oracle/oracle.c): reference arithmetic restated, test infrastructure only.
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
void orc_cache_store(int mode, int v_kind, const float* src, const uint16_t* src_f16,
                     uint16_t* pool, const int32_t* tables, const int32_t* positions,
                     const int32_t* owners, const int32_t* params, int64_t rows, int64_t kv_dim,
                     int64_t table_stride, int64_t n_layer, int64_t layer, int64_t layer_base,
                     int64_t pos_offset);
int orc_attention_paged_rows(const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                             const int32_t* tables, const int32_t* table_index,
                             const int32_t* lens, int64_t rows, int64_t n_head,
                             int64_t n_kv_head, int64_t head_dim, int64_t table_stride,
                             int64_t n_layer, int64_t layer, double scale, int precise,
                             float* out);
}

namespace {

constexpr int kStoreRows = 0, kStorePacked = 2;  // orc_cache_store modes

int g_failures = 0;

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        std::fprintf(stderr, "HIP error at %s: %s\n", what, hipGetErrorString(e));
        std::exit(2);
    }
}

void abi_ok(int rc, const char* what) {
    if (rc != CRUCIBLE_OK) {
        char msg[512];
        crucible_attn_last_error(msg, sizeof(msg));
        std::fprintf(stderr, "%s failed (%d): %s\n", what, rc, msg);
        std::exit(3);
    }
}

// splitmix64 -> uniform -> Box-Muller: deterministic inputs without a library
struct Rng {
    uint64_t s;
    uint64_t next() {
        uint64_t z = (s += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    }
    double uniform() { return ((next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
    float normal() {
        const double u = uniform(), v = uniform();
        return (float)(std::sqrt(-2.0 * std::log(u)) * std::cos(6.283185307179586 * v));
    }
};

template <class T>
T* dev_alloc(size_t n) {
    void* p = nullptr;
    hip_ok(hipMalloc(&p, n * sizeof(T) + 16), "hipMalloc");
    return static_cast<T*>(p);
}

template <class T>
void upload(T* d, const std::vector<T>& h) {
    hip_ok(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice), "upload");
}

template <class T>
std::vector<T> download(const T* d, size_t n) {
    std::vector<T> h(n);
    hip_ok(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost), "download");
    return h;
}

void check_gate(const char* what, const std::vector<float>& got, const std::vector<float>& want) {
    double worst = 0.0;
    size_t bad = 0;
    for (size_t i = 0; i < got.size(); ++i) {
        const double d = std::fabs((double)got[i] - (double)want[i]);
        if (!(d <= 2e-5 + 2e-5 * std::fabs((double)want[i]))) ++bad;
        if (d > worst || std::isnan(d)) worst = std::isnan(d) ? INFINITY : d;
    }
    std::printf("%-34s max-abs %.3e, %zu of %zu elements outside the gate\n", what, worst, bad,
                got.size());
    if (bad) ++g_failures;
}

void check_pool(const char* what, const uint16_t* d_pool, const std::vector<uint16_t>& want) {
    const std::vector<uint16_t> got = download(d_pool, want.size());
    const bool same = std::memcmp(got.data(), want.data(), want.size() * 2) == 0;
    std::printf("%-34s %s\n", what, same ? "bit-identical to the oracle's appends" : "DIFFERS");
    if (!same) ++g_failures;
}

}  // namespace

int main() {
    std::printf("native caller: %s\n", crucible_attn_version());
    // 120m-preset attention geometry, 3 layers, 4 requests
    const int n_head = 12, n_kv = 3, hd = 64, kv_dim = n_kv * hd, n_layer = 3;
    const int batch = 4, max_seq = 512, stride = max_seq / 16, decode_steps = 4;
    const int prompt[batch] = {37, 129, 300, 16};
    const int n_pages = batch * stride + 1;
    const int64_t pool_elems = (int64_t)n_pages * n_layer * 16 * kv_dim;
    Rng rng{20260908};

    // page tables: a shuffled pool, each request's pages disjoint (paged.rs allocation)
    std::vector<int32_t> perm(n_pages);
    for (int i = 0; i < n_pages; ++i) perm[i] = i;
    for (int i = n_pages - 1; i > 0; --i) std::swap(perm[i], perm[rng.next() % (uint64_t)(i + 1)]);
    std::vector<int32_t> tables(batch * stride);
    for (int b = 0; b < batch; ++b)
        for (int p = 0; p < stride; ++p) tables[b * stride + p] = perm[b * stride + p];

    // pools start as fp16 noise (never-written slots hold finite garbage)
    std::vector<uint16_t> k_pool(pool_elems), v_pool(pool_elems);
    for (auto& x : k_pool) x = orc_f32_to_f16(rng.normal());
    for (auto& x : v_pool) x = orc_f32_to_f16(rng.normal());

    hipStream_t stream;
    hip_ok(hipStreamCreate(&stream), "hipStreamCreate");
    crucible_stream_t cs = reinterpret_cast<crucible_stream_t>(stream);
    uint16_t* d_k = dev_alloc<uint16_t>(pool_elems);
    uint16_t* d_v = dev_alloc<uint16_t>(pool_elems);
    int32_t* d_tables = dev_alloc<int32_t>(tables.size());
    upload(d_k, k_pool);
    upload(d_v, v_pool);
    upload(d_tables, tables);

    // ---- prefill: packed rows of every prompt, K/V through the packed append, then the
    // segment-form causal attention, layer by layer
    int rows = 0;
    for (int b = 0; b < batch; ++b) rows += prompt[b];
    std::vector<int32_t> owners, positions, segments;
    for (int b = 0, start = 0; b < batch; start += prompt[b], ++b) {
        segments.insert(segments.end(), {start, prompt[b], 0, b});
        for (int i = 0; i < prompt[b]; ++i) {
            owners.push_back(b);
            positions.push_back(i);
        }
    }
    int32_t* d_owners = dev_alloc<int32_t>(rows);
    int32_t* d_positions = dev_alloc<int32_t>(rows);
    int32_t* d_segments = dev_alloc<int32_t>(segments.size());
    upload(d_owners, owners);
    upload(d_positions, positions);
    upload(d_segments, segments);
    float* d_src = dev_alloc<float>((size_t)rows * n_head * hd);
    float* d_out = dev_alloc<float>((size_t)rows * n_head * hd);
    std::vector<int32_t> plens(rows);
    for (int r = 0; r < rows; ++r) plens[r] = positions[r] + 1;
    for (int layer = 0; layer < n_layer; ++layer) {
        std::vector<float> kr((size_t)rows * kv_dim), vr((size_t)rows * kv_dim),
            q((size_t)rows * n_head * hd);
        for (auto& x : kr) x = rng.normal();
        for (auto& x : vr) x = rng.normal();
        for (auto& x : q) x = rng.normal();
        for (int kind = 0; kind < 2; ++kind) {
            const std::vector<float>& src = kind ? vr : kr;
            upload(d_src, src);
            abi_ok(crucible_cache_store_packed_paged(d_src, CRUCIBLE_F32, kind ? d_v : d_k,
                                                     kind ? CRUCIBLE_POOL_V : CRUCIBLE_POOL_K,
                                                     d_tables, d_owners, d_positions, rows,
                                                     kv_dim, stride, n_layer, layer, cs),
                   "cache_store_packed_paged");
            hip_ok(hipStreamSynchronize(stream), "sync");
            orc_cache_store(kStorePacked, kind, src.data(), nullptr, kind ? v_pool.data() : k_pool.data(),
                            tables.data(), positions.data(), owners.data(), nullptr, rows, kv_dim,
                            stride, n_layer, layer, 0, 0);
        }
        upload(d_src, q);
        abi_ok(crucible_attention_prefill_tiled(d_src, CRUCIBLE_F32, d_k, d_v, nullptr, nullptr,
                                                d_out, CRUCIBLE_F32, d_tables, d_segments, batch,
                                                300, stride, n_head, n_kv, hd, n_layer, layer,
                                                kv_dim, 0, max_seq, cs),
               "attention_prefill_tiled");
        hip_ok(hipStreamSynchronize(stream), "sync");
        std::vector<float> want((size_t)rows * n_head * hd);
        orc_attention_paged_rows(q.data(), k_pool.data(), v_pool.data(), tables.data(),
                                 owners.data(), plens.data(), rows, n_head, n_kv, hd, stride,
                                 n_layer, layer, 0.125, 1, want.data());
        char what[64];
        std::snprintf(what, sizeof(what), "prefill layer %d", layer);
        check_gate(what, download(d_out, want.size()), want);
    }
    check_pool("prefill K pool", d_k, k_pool);
    check_pool("prefill V pool", d_v, v_pool);

    // ---- decode: each step appends one token per request at its next position and
    // attends over len + 1 keys, per layer, on one workspace (ordered on one stream)
    const size_t ws_bytes = crucible_attention_decode_workspace_bytes(batch, n_head, max_seq);
    void* d_ws = nullptr;
    hip_ok(hipMalloc(&d_ws, ws_bytes), "hipMalloc workspace");
    hip_ok(hipMemset(d_ws, 0, ws_bytes), "hipMemset workspace");
    int32_t* d_pos = dev_alloc<int32_t>(batch);
    int32_t* d_lens = dev_alloc<int32_t>(batch);
    float* d_q = dev_alloc<float>((size_t)batch * n_head * hd);
    float* d_kn = dev_alloc<float>((size_t)batch * kv_dim);
    float* d_vn = dev_alloc<float>((size_t)batch * kv_dim);
    std::vector<int32_t> table_index(batch);
    for (int b = 0; b < batch; ++b) table_index[b] = b;
    for (int step = 0; step < decode_steps; ++step) {
        std::vector<int32_t> pos(batch), lens(batch);
        for (int b = 0; b < batch; ++b) {
            pos[b] = prompt[b] + step;
            lens[b] = pos[b] + 1;
        }
        upload(d_pos, pos);
        upload(d_lens, lens);
        for (int layer = 0; layer < n_layer; ++layer) {
            std::vector<float> q((size_t)batch * n_head * hd), kn((size_t)batch * kv_dim),
                vn((size_t)batch * kv_dim);
            for (auto& x : q) x = rng.normal();
            for (auto& x : kn) x = rng.normal();
            for (auto& x : vn) x = rng.normal();
            upload(d_q, q);
            upload(d_kn, kn);
            upload(d_vn, vn);
            abi_ok(crucible_attention_decode_paged_append(
                       d_q, CRUCIBLE_F32, d_kn, d_vn, CRUCIBLE_F32, d_k, d_v, d_out,
                       CRUCIBLE_F32, d_tables, d_pos, d_lens, batch, n_head, n_kv, hd, stride,
                       n_layer, layer, kv_dim, max_seq, d_ws, ws_bytes, cs),
                   "attention_decode_paged_append");
            hip_ok(hipStreamSynchronize(stream), "sync");
            orc_cache_store(kStoreRows, 0, kn.data(), nullptr, k_pool.data(), tables.data(),
                            pos.data(), nullptr, nullptr, batch, kv_dim, stride, n_layer, layer,
                            0, 0);
            orc_cache_store(kStoreRows, 1, vn.data(), nullptr, v_pool.data(), tables.data(),
                            pos.data(), nullptr, nullptr, batch, kv_dim, stride, n_layer, layer,
                            0, 0);
            std::vector<float> want((size_t)batch * n_head * hd);
            orc_attention_paged_rows(q.data(), k_pool.data(), v_pool.data(), tables.data(),
                                     table_index.data(), lens.data(), batch, n_head, n_kv, hd,
                                     stride, n_layer, layer, 0.125, 1, want.data());
            char what[64];
            std::snprintf(what, sizeof(what), "decode step %d layer %d", step, layer);
            check_gate(what, download(d_out, want.size()), want);
        }
    }
    check_pool("decode K pool", d_k, k_pool);
    check_pool("decode V pool", d_v, v_pool);
    std::printf("native caller: %d failed checks\n", g_failures);
    return g_failures ? 1 : 0;
}
