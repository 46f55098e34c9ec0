// Library-wide C-ABI pieces: thread-local error reporting, version, and the
// cu_seqlens -> segment helper used by packed prefill callers.
#include "common.hpp"

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace crucible {

namespace {
thread_local char g_last_message[512] = "";
thread_local int g_last_status = CRUCIBLE_OK;
}  // namespace

void set_error(int status, const char* fmt, ...) {
    g_last_status = status;
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_message, sizeof(g_last_message), fmt, ap);
    va_end(ap);
}

int device_cu_count() {
    constexpr int kMaxDevices = 64;
    constexpr int kFallback = 256;  // MI355X
    static std::atomic<int> cache[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();  // a failed query must not read as a later launch failure
        return kFallback;
    }
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        n = kFallback;
    }
    cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

// Launch-shape overrides. Each key starts at its environment variable, read once per process
// (the first time any key is asked for), and after that changes only through
// crucible_attn_set_tuning. -1 means the launcher's own choice.
namespace {
struct TuneKey {
    const char* env;
    int lo, hi;  // accepted values
};
constexpr TuneKey kTuneKeys[CRUCIBLE_TUNE_COUNT] = {
    {"CRUCIBLE_DECODE_PAGES", 1, 4},          // pages per wave: 1, 2 or 4
    {"CRUCIBLE_DECODE_WAVES", 4, 8},          // waves per workgroup: 4 or 8
    {"CRUCIBLE_DECODE_ORDER", 0, 2},          // 0 split, 1 request, 2 compact
    {"CRUCIBLE_PREFILL_DIRECT", 0, 1},        // register-direct form off / on
    {"CRUCIBLE_PREFILL_HEAVY_FIRST", 0, 1},   // longest-first grid off / on
    {"CRUCIBLE_PREFILL_QB", 1, 2},            // 16-row blocks per wave
    {"CRUCIBLE_PREFILL_BUFS", 4, 6},          // key tiles in the LDS ring: 4 or 6
    {"CRUCIBLE_LINEAR_TILE", 4, 32},          // projection tiles: 4, 16 or 32 (see below)
    {"CRUCIBLE_DECODE_COMBINE_WIDTH", 8, 16}, // splits merged per round trip: 8 or 16
    {"CRUCIBLE_PREFILL_P16", 0, 1},           // prefill P operand: fp16 hi + lo / one fp16
    {"CRUCIBLE_PREFILL_M32", 0, 1},           // prefill 32-row waves on 32x32 MFMAs off / on
    {"CRUCIBLE_PREFILL_PERSIST", 0, 65536},   // prefill persistent LDS form off / on / n workgroups
    {"CRUCIBLE_LINEAR_PREFETCH", 0, 1},       // projections' next-kernel prefetch off / on
};

bool tune_value_ok(int key, int v) {
    switch (key) {
        case CRUCIBLE_TUNE_DECODE_PAGES: return v == 1 || v == 2 || v == 4;
        case CRUCIBLE_TUNE_DECODE_WAVES: return v == 4 || v == 8;
        case CRUCIBLE_TUNE_PREFILL_BUFS: return v == 4 || v == 6;
        case CRUCIBLE_TUNE_LINEAR_TILE: return v == 4 || v == 16 || v == 32;
        case CRUCIBLE_TUNE_DECODE_COMBINE_WIDTH: return v == 8 || v == 16;
        default: return v >= kTuneKeys[key].lo && v <= kTuneKeys[key].hi;
    }
}

int parse_env(int key, const char* s) {
    if (key == CRUCIBLE_TUNE_DECODE_ORDER) {
        if (!std::strcmp(s, "split")) return 0;
        if (!std::strcmp(s, "request")) return 1;
        if (!std::strcmp(s, "compact")) return 2;
        return -1;
    }
    char* end = nullptr;
    const long v = std::strtol(s, &end, 10);
    if (end == s || *end != '\0') return -1;
    if (key == CRUCIBLE_TUNE_PREFILL_DIRECT || key == CRUCIBLE_TUNE_PREFILL_HEAVY_FIRST ||
        key == CRUCIBLE_TUNE_PREFILL_P16 || key == CRUCIBLE_TUNE_PREFILL_M32 ||
        key == CRUCIBLE_TUNE_LINEAR_PREFETCH)
        return v != 0;
    return tune_value_ok(key, (int)v) ? (int)v : -1;
}

std::atomic<int> g_tune[CRUCIBLE_TUNE_COUNT];
std::once_flag g_tune_once;

void tune_init() {
    std::call_once(g_tune_once, [] {
        for (int k = 0; k < CRUCIBLE_TUNE_COUNT; ++k) {
            const char* env = std::getenv(kTuneKeys[k].env);
            g_tune[k].store(env ? parse_env(k, env) : -1, std::memory_order_relaxed);
        }
    });
}
}  // namespace

int tuning(int key) {
    tune_init();
    return g_tune[key].load(std::memory_order_relaxed);
}

int fail_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e == hipSuccess) return CRUCIBLE_OK;
    set_error(CRUCIBLE_ERR_LAUNCH, "%s: HIP launch failed: %s", what, hipGetErrorString(e));
    return CRUCIBLE_ERR_LAUNCH;
}

}  // namespace crucible

extern "C" const char* crucible_attn_version(void) {
    return "crucible_attn 0.1.0 gfx950";
}

extern "C" int crucible_attn_set_tuning(int key, int value) {
    if (key < 0 || key >= CRUCIBLE_TUNE_COUNT) {
        crucible::set_error(CRUCIBLE_ERR_INVALID, "set_tuning: unknown key %d", key);
        return CRUCIBLE_ERR_INVALID;
    }
    if (value != -1 && !crucible::tune_value_ok(key, value)) {
        crucible::set_error(CRUCIBLE_ERR_INVALID, "set_tuning: %s does not take %d",
                            crucible::kTuneKeys[key].env, value);
        return CRUCIBLE_ERR_INVALID;
    }
    crucible::tune_init();
    crucible::g_tune[key].store(value, std::memory_order_relaxed);
    return CRUCIBLE_OK;
}

extern "C" int crucible_attn_get_tuning(int key) {
    if (key < 0 || key >= CRUCIBLE_TUNE_COUNT) return -1;
    return crucible::tuning(key);
}

extern "C" const char* crucible_attn_tuning_name(int key) {
    if (key < 0 || key >= CRUCIBLE_TUNE_COUNT) return nullptr;
    return crucible::kTuneKeys[key].env;
}

extern "C" int crucible_attn_last_error(char* buf, size_t n) {
    if (buf && n) {
        std::strncpy(buf, crucible::g_last_message, n - 1);
        buf[n - 1] = '\0';
    }
    return crucible::g_last_status;
}

// Segments are {packed_start, chunk_len, absolute_start, table_index}, the
// descriptor of gpu_model.rs:2885-2890 (prepare_packed_prefill).
extern "C" int64_t crucible_segments_from_cu_seqlens(const int32_t* cu_seqlens, int64_t n,
                                                     const int32_t* absolute_starts,
                                                     int32_t* segments_out) {
    if (!cu_seqlens || !segments_out || n < 0 || cu_seqlens[0] != 0) {
        crucible::set_error(CRUCIBLE_ERR_INVALID, "cu_seqlens must start at 0");
        return -1;
    }
    int64_t max_chunk = 0;
    for (int64_t i = 0; i < n; ++i) {
        const int64_t len = (int64_t)cu_seqlens[i + 1] - cu_seqlens[i];
        if (len < 0) {
            crucible::set_error(CRUCIBLE_ERR_INVALID, "cu_seqlens decreases at %lld",
                                (long long)i);
            return -1;
        }
        segments_out[4 * i + 0] = cu_seqlens[i];
        segments_out[4 * i + 1] = (int32_t)len;
        segments_out[4 * i + 2] = absolute_starts ? absolute_starts[i] : 0;
        segments_out[4 * i + 3] = (int32_t)i;
        if (len > max_chunk) max_chunk = len;
    }
    return max_chunk;
}
