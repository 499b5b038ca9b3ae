#include "common/common.h"

#include <cstdarg>
#include <cstdio>
#include <mutex>

namespace {

// Long enough for every message this library writes; longer ones truncate.
thread_local char last_error[512] = "";

}  // namespace

namespace flint {

flint_status fail(flint_status status, const char* format, ...) {
    va_list args;
    va_start(args, format);
    std::vsnprintf(last_error, sizeof last_error, format, args);
    va_end(args);
    return status;
}

flint_status check_buffers(const char* function, const Buffer* buffers, size_t count,
                           size_t outputs) {
    for (size_t i = 0; i < count; ++i) {
        const Buffer& b = buffers[i];
        if (b.pointer == nullptr) {
            return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: %s is null", function, b.name);
        }
        if (!aligned16(b.pointer)) {
            return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: %s is not 16-byte aligned", function,
                        b.name);
        }
        if (!fits(b.pointer, b.bytes)) {
            return fail(FLINT_ERROR_INVALID_ARGUMENT,
                        "%s: %s runs past the end of the address space", function, b.name);
        }
    }
    for (size_t i = 0; i < outputs; ++i) {
        for (size_t j = i + 1; j < count; ++j) {
            if (overlap(buffers[i].pointer, buffers[i].bytes, buffers[j].pointer,
                        buffers[j].bytes)) {
                return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: %s and %s overlap", function,
                            buffers[i].name, buffers[j].name);
            }
        }
    }
    return FLINT_OK;
}

hipError_t device_cus(int* cus) {
    static std::mutex lock;
    static int cached[64] = {};
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    if (device >= 0 && device < 64) {
        std::lock_guard<std::mutex> guard(lock);
        if (cached[device] == 0) {
            int n = 0;
            e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device);
            if (e != hipSuccess) return e;
            cached[device] = n;
        }
        *cus = cached[device];
        return hipSuccess;
    }
    return hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, device);
}

}  // namespace flint

extern "C" {

FLINT_API const char* flint_last_error(void) { return last_error; }

FLINT_API const char* flint_version(void) { return "0.1.0"; }

FLINT_API const char* flint_status_string(flint_status status) {
    switch (status) {
    case FLINT_OK:
        return "ok";
    case FLINT_ERROR_INVALID_ARGUMENT:
        return "invalid argument";
    case FLINT_ERROR_CUDA:
        return "CUDA error";
    default:
        return "unknown status";
    }
}

}  // extern "C"
