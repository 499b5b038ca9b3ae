#include "common/common.h"

#include <array>
#include <atomic>
#include <cstdarg>
#include <cstdio>

namespace {

// This thread's last message; 512 bytes hold every message the library writes.
thread_local std::array<char, 512> g_message{};

// Compute units per device ordinal (0 = not read yet). A race between two
// first readers stores the same value twice.
constexpr int kDevices = 64;
std::array<std::atomic<int>, kDevices> g_cus{};

}  // namespace

namespace flint {

flint_status fail(flint_status status, const char* format, ...) {
    va_list args;
    va_start(args, format);
    std::vsnprintf(g_message.data(), g_message.size(), format, args);
    va_end(args);
    return status;
}

flint_status hip_failure(hipError_t error, const char* file, int line) {
    (void)hipGetLastError();
    return fail(FLINT_ERROR_CUDA, "%s: %s (%s:%d)", hipGetErrorName(error),
                hipGetErrorString(error), file, line);
}

hipError_t device_cus(int* cus) {
    int device = 0;
    if (const hipError_t e = hipGetDevice(&device); e != hipSuccess) return e;
    const bool cached = device >= 0 && device < kDevices;
    if (cached) {
        if (const int known = g_cus[device].load(std::memory_order_relaxed); known > 0) {
            *cus = known;
            return hipSuccess;
        }
    }
    int n = 0;
    if (const hipError_t e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device);
        e != hipSuccess)
        return e;
    if (cached) g_cus[device].store(n, std::memory_order_relaxed);
    *cus = n;
    return hipSuccess;
}

}  // namespace flint

extern "C" {

FLINT_API const char* flint_last_error(void) { return g_message.data(); }

FLINT_API const char* flint_version(void) { return "0.1.0"; }

FLINT_API const char* flint_status_string(flint_status status) {
    static const char* const kNames[] = {"ok", "invalid argument", "CUDA error"};
    const int i = static_cast<int>(status);
    return i >= 0 && i < 3 ? kNames[i] : "unknown status";
}

}  // extern "C"
