/* libflint: an entry point for callers that cannot allocate device memory.
 *
 * No counterpart in the reference's ABI. It is for code that may not call
 * hipMalloc or take a caller-sized workspace: work under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation.
 */
#ifndef FLINT_FLINT_NOALLOC_H
#define FLINT_FLINT_NOALLOC_H

#include "flint/flint.h"

#ifdef __cplusplus
extern "C" {
#endif

/* flint_bias_gradient without a workspace argument: the same kernels, the same
 * checks on rows and cols, and bit-identical results, with the per-chunk
 * partials kept in a device array of 4 MiB that the library holds on every
 * device it runs on until the process ends. It allocates nothing; the array's
 * device address is looked up once per device, on that device's first call.
 * Sizes whose partials need more (ceil(rows / 256) * cols * 8 bytes above
 * 4 MiB, e.g. 8,192 rows of more than 16,384 columns) are refused with
 * FLINT_ERROR_INVALID_ARGUMENT. Every call on one device shares its array and
 * leaves its partials there: calls in one stream's order are safe, calls that
 * overlap on one device (several streams or threads) race. */
FLINT_API flint_status flint_bias_gradient_noalloc(void* dbias, const void* dy, size_t rows,
                                                   size_t cols, int accumulate,
                                                   flint_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* FLINT_FLINT_NOALLOC_H */
