// A HIP runtime with no device, for the host-code sanitizer run of the library's argument
// validation (tests/test_abi_sanitized.py). The library's objects, built with the
// sanitizers on their host code, are linked against these definitions instead of
// libamdhip64: kernel registration does nothing, and every runtime call fails with
// hipErrorNoDevice, as the real runtime does on a host without a GPU (hipGetLastError
// returns and clears the last failure, which is how the library's launch checks read it).
// The real runtime works there too, but under AddressSanitizer its start-up maps large
// address ranges and each call takes seconds; no call here reaches a device either way.
#include <hip/hip_runtime_api.h>

#include <cstddef>

namespace {
hipError_t g_last = hipSuccess;

hipError_t no_device() {
    g_last = hipErrorNoDevice;
    return hipErrorNoDevice;
}

void* g_module = nullptr;
}  // namespace

extern "C" {

void** __hipRegisterFatBinary(const void*) { return &g_module; }
void __hipRegisterFunction(void**, const void*, char*, const char*, unsigned int, void*, void*,
                           void*, void*, int*) {}
void __hipRegisterVar(void**, void*, char*, char*, int, size_t, int, int) {}
void __hipUnregisterFatBinary(void**) {}

}  // extern "C"

hipError_t __hipPushCallConfiguration(dim3, dim3, size_t, hipStream_t) { return hipSuccess; }
hipError_t __hipPopCallConfiguration(dim3* grid, dim3* block, size_t* shared,
                                     hipStream_t* stream) {
    *grid = dim3(1, 1, 1);
    *block = dim3(1, 1, 1);
    *shared = 0;
    *stream = nullptr;
    return hipSuccess;
}

hipError_t hipGetDevice(int*) { return no_device(); }
hipError_t hipDeviceGetAttribute(int*, hipDeviceAttribute_t, int) { return no_device(); }
hipError_t hipGetLastError() {
    const hipError_t e = g_last;
    g_last = hipSuccess;
    return e;
}
const char* hipGetErrorString(hipError_t) { return "no device (stub runtime)"; }
hipError_t hipGetSymbolAddress(void**, const void*) { return no_device(); }
hipError_t hipLaunchKernel(const void*, dim3, dim3, void**, size_t, hipStream_t) {
    return no_device();
}
hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int*, const void*, int, size_t) {
    return no_device();
}
