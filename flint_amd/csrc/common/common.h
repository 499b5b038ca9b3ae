// Status plumbing shared by every C-ABI entry point: the per-thread message
// behind flint_last_error, the conversion of a failed HIP call into
// FLINT_ERROR_CUDA, and the device's compute-unit count.
//
// Argument checking lives in common/args.h.
#pragma once

#include <cstddef>

#include <hip/hip_runtime.h>

#include "flint/flint.h"

namespace flint {

// Stores a printf-style message as this thread's last error and returns
// `status` (so a check can `return fail(...)`). A message longer than the
// buffer is cut short.
flint_status fail(flint_status status, const char* format, ...)
    __attribute__((__format__(__printf__, 2, 3)));

// The FLINT_ERROR_CUDA status of a HIP call that returned `error` at
// file:line. The message reads "hipErrorName: description (file:line)", the
// shape the reference's callers parse (ref src/common/error.h:28-38), and the
// runtime's sticky last error is consumed so that the next call starts clean.
flint_status hip_failure(hipError_t error, const char* file, int line);

inline hipStream_t to_hip(flint_stream s) { return reinterpret_cast<hipStream_t>(s); }

// Compute units of the current device, read once per device.
hipError_t device_cus(int* cus);

}  // namespace flint

// Evaluates a HIP call once; on failure the enclosing entry point returns
// hip_failure's status.
#define FLINT_HIP_CHECK(call)                                                          \
    do {                                                                               \
        if (const hipError_t flint_err_ = (call); flint_err_ != hipSuccess)            \
            return ::flint::hip_failure(flint_err_, __FILE__, __LINE__);               \
    } while (0)
