// Library-wide host state: the per-thread error string behind hs_last_error,
// the argument / HIP error helpers every entry point returns through, and the
// cached CU count per device.  Host-only translation unit.
#include <array>
#include <atomic>
#include <string>

#include "hs_gpu.h"
#include "hs_internal.hpp"

namespace hs {

namespace {
thread_local std::string g_last_error;
std::array<std::atomic<int>, 64> g_cu_count{};
}  // namespace

void set_error(const std::string& message) { g_last_error = message; }
void clear_error() { g_last_error.clear(); }

int reject(const char* message) {
    g_last_error = message;
    return HS_ERR_ARGUMENT;
}

int hip_fail(hipError_t status, const char* what) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(status);
    return HS_ERR_HIP;
}

int device_cu_count() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return 256;
    int cached = g_cu_count[device].load(std::memory_order_relaxed);
    if (cached > 0) return cached;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        cus <= 0)
        cus = 256;
    g_cu_count[device].store(cus, std::memory_order_relaxed);
    return cus;
}

bool stream_capturing(hipStream_t stream) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &capture) != hipSuccess) {
        (void)hipGetLastError();  // not the caller's launch error
        return true;
    }
    return capture != hipStreamCaptureStatusNone;
}

void clear_status_if_captured(hs_status_t* status, uint32_t count, hipStream_t stream) {
    if (status && count && stream_capturing(stream))
        launch_fill_u32(reinterpret_cast<uint32_t*>(status),
                        count * static_cast<uint32_t>(sizeof(hs_status_t) / sizeof(uint32_t)), 0u, stream);
}

uint32_t next_stamp() {
    static std::atomic<uint32_t> calls{0};
    return (calls.fetch_add(1, std::memory_order_relaxed) & 0x7fffffffu) | 0x80000000u;
}

}  // namespace hs

extern "C" {

const char* hs_version(void) { return "hillserve_amd 0.1 gfx950"; }
const char* hs_last_error(void) { return hs::g_last_error.c_str(); }

}  // extern "C"
