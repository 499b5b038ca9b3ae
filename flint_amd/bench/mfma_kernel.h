// The MFMA ceiling loop (the MI355X counterpart of the reference's tensor-core
// peak loop, ref bench/mma_kernels.cu:16-30): every wave issues back-to-back
// v_mfma_f32_32x32x16_f16 on CHAINS independent accumulators, so the loop is
// bound by the matrix cores alone. Shared by flint_bench_mfma and flint_bench.
//
// Every operand element is a (A operand) or b (B operand), so each MFMA adds
// 16ab to each accumulator element. With a = 1 and b = 2^-10 the sums stay
// exact in FP32, and every lane checks its accumulators against iters * 16ab
// at the end, setting *bad on a mismatch: the timed loop proves its own result.
#pragma once

#include <hip/hip_runtime.h>

typedef _Float16 mfma_f16x8 __attribute__((ext_vector_type(8)));
typedef float mfma_f32x16 __attribute__((ext_vector_type(16)));

template <int CHAINS>
__global__ void __launch_bounds__(256) mfma_loop(int* bad, int iters, float a_val, float b_val) {
    mfma_f16x8 a, b;
    for (int i = 0; i < 8; ++i) {
        a[i] = _Float16(a_val);
        b[i] = _Float16(b_val);
    }
    mfma_f32x16 c[CHAINS];
    for (int j = 0; j < CHAINS; ++j) c[j] = mfma_f32x16{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < CHAINS; ++j) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c[j], 0, 0, 0);
    }
    const float want = float(iters) * 16.0f * float(_Float16(a_val)) * float(_Float16(b_val));
    bool ok = true;
    for (int j = 0; j < CHAINS; ++j)
        for (int i = 0; i < 16; ++i) ok = ok && c[j][i] == want;
    if (!ok) bad[0] = 1;
}

// MFMAs one wave issues per launch, spread over the chains.
constexpr int kMfmaPerWave = 32768;
// FLOPs of one v_mfma_f32_32x32x16_f16: 32 x 32 x 16 multiply-adds.
constexpr double kMfmaFlops = 32.0 * 32.0 * 16.0 * 2.0;

// FLOPs of one mfma_loop launch: blocks x 4 waves x iters x chains MFMAs.
inline double mfma_loop_flops(int blocks, int iters, int chains) {
    return double(blocks) * 4.0 * double(iters) * chains * kMfmaFlops;
}

// Launches mfma_loop<chains> (4, 8 or 16) on blocks workgroups of 4 waves.
inline hipError_t launch_mfma_loop(int chains, int blocks, int* bad, int iters, hipStream_t stream) {
    const float a = 1.0f, b = 1.0f / 1024.0f;
    switch (chains) {
    case 4: hipLaunchKernelGGL(mfma_loop<4>, dim3(blocks), dim3(256), 0, stream, bad, iters, a, b); break;
    case 8: hipLaunchKernelGGL(mfma_loop<8>, dim3(blocks), dim3(256), 0, stream, bad, iters, a, b); break;
    case 16: hipLaunchKernelGGL(mfma_loop<16>, dim3(blocks), dim3(256), 0, stream, bad, iters, a, b); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
