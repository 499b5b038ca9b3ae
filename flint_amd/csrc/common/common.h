// Error recording and pointer checks shared by every C-ABI entry point.
//
// Behaviour follows the reference's src/common/error.{h,cpp} and
// src/common/checks.{h,cpp}: a thread-local last-error message, a macro that
// turns a failed runtime call into FLINT_ERROR_CUDA (clearing the runtime's
// sticky error), and a buffer check that tests, in order, null, 16-byte
// alignment, address-space wrap and output/other overlap.
#pragma once

#include <cstddef>
#include <cstdint>

#include <hip/hip_runtime.h>

#include "flint/flint.h"

namespace flint {

// Records a printf-style message for flint_last_error and returns status.
flint_status fail(flint_status status, const char* format, ...)
    __attribute__((__format__(__printf__, 2, 3)));

inline bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// [p, p + bytes) stays inside the address space.
inline bool fits(const void* p, size_t bytes) {
    return bytes <= UINTPTR_MAX - reinterpret_cast<uintptr_t>(p);
}

inline bool overlap(const void* a, size_t a_bytes, const void* b, size_t b_bytes) {
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(a);
    const uintptr_t b0 = reinterpret_cast<uintptr_t>(b);
    return a0 < b0 + b_bytes && b0 < a0 + a_bytes;
}

struct Buffer {
    const char* name;
    const void* pointer;
    size_t bytes;
};

// Checks each buffer for null, alignment and wrap, then that none of the first
// `outputs` buffers overlaps any buffer listed after it (ref
// src/common/checks.cpp:7-34). Returns FLINT_OK or the first failure.
flint_status check_buffers(const char* function, const Buffer* buffers, size_t count,
                           size_t outputs);

inline hipStream_t to_hip(flint_stream s) { return reinterpret_cast<hipStream_t>(s); }

// Compute units of the current device (cached per device).
hipError_t device_cus(int* cus);

}  // namespace flint

// A failed HIP call returns FLINT_ERROR_CUDA with "name: description (file:line)"
// and clears the runtime's last error (ref src/common/error.h:28-38).
#define FLINT_HIP_CHECK(call)                                                           \
    do {                                                                                \
        const hipError_t flint_hip_error_ = (call);                                     \
        if (flint_hip_error_ != hipSuccess) {                                           \
            (void)hipGetLastError();                                                    \
            return ::flint::fail(FLINT_ERROR_CUDA, "%s: %s (%s:%d)",                    \
                                 hipGetErrorName(flint_hip_error_),                     \
                                 hipGetErrorString(flint_hip_error_), __FILE__, __LINE__); \
        }                                                                               \
    } while (0)
