// The sum of a split TN's k-slice partials: tn_reduce (gemm.hip) and the
// GPT-2 model's merged gradient finish (reductions.hip) run this same loop.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

namespace flint {

// y = p0 + p1 + ... (+ the old y first when accumulating), in split order,
// over the float4 quads first, first + stride, ... < quads; split s's partials
// start s * quads quads into `partials` (ref src/kernels/gemm.cu:678-703 for
// the order).
__device__ inline void add_split_partials(float* __restrict__ y,
                                          const float* __restrict__ partials, size_t quads,
                                          int splits, int accumulate, size_t first,
                                          size_t stride) {
    typedef float quad4 __attribute__((ext_vector_type(4)));
    const quad4* p = reinterpret_cast<const quad4*>(partials);
    quad4* out = reinterpret_cast<quad4*>(y);
    for (size_t i = first; i < quads; i += stride) {
        quad4 sum = p[i];
        for (int s = 1; s < splits; ++s) sum += p[size_t(s) * quads + i];
        if (accumulate) sum = out[i] + sum;
        out[i] = sum;
    }
}

}  // namespace flint
