// Library-wide C-ABI pieces: thread-local error reporting, version, and the
// cu_seqlens -> segment helper used by packed prefill callers.
#include "common.hpp"

#include <atomic>
#include <cstring>

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
