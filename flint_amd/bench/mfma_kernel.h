// The MFMA ceiling loop (the MI355X counterpart of the reference's tensor-core
// peak loop, ref bench/mma_kernels.cu:16-30): every wave issues back-to-back
// v_mfma_f32_32x32x16_f16 on CHAINS independent accumulators, so the loop is
// bound by the matrix cores alone (flint_bench's mma benchmark).
//
// Operands vary across lanes and elements, as a GEMM's do (the matrix cores'
// power, and so the clock, depend on the bits they switch): A elements are
// +-1 or +-2 and B elements +-2^-10 or +-2^-9, signs and magnitudes hashed from
// (lane, element, seed). Every product is a multiple of 2^-10 and the running
// sums stay below 2^11, so every accumulator is exact in FP32 and its value
// does not depend on summation order. The check uses an invariant of the
// product that holds for any placement of rows and columns on lanes: the sum
// of all of C equals iters x sum_k (sum over rows of A[., k]) (sum over columns
// of B[k, .]). Lane l holds A row l % 32 and B column l % 32 at k-block l / 32
// (the same k-block for both operands), so the column and row sums are sums
// over the 32 lanes of a half. Both sides are summed in FP64, exactly; lane 0
// sets *bad on a mismatch.
#pragma once

#include <hip/hip_runtime.h>

typedef _Float16 mfma_f16x8 __attribute__((ext_vector_type(8)));
typedef float mfma_f32x16 __attribute__((ext_vector_type(16)));

__device__ inline float mfma_operand(unsigned lane, unsigned i, unsigned seed, float scale) {
    unsigned h = (lane * 8u + i) * 0x9E3779B1u ^ seed * 0x85EBCA77u;
    h ^= h >> 15;
    h *= 0x2C1B3C6Du;
    h ^= h >> 13;
    return (h & 1u ? -scale : scale) * (h & 2u ? 2.0f : 1.0f);
}

__device__ inline double mfma_wave_sum(double v, int width) {
    for (int o = 1; o < width; o <<= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int CHAINS>
__global__ void __launch_bounds__(256) mfma_loop(int* bad, int iters, unsigned seed) {
    const unsigned lane = threadIdx.x % 64;
    mfma_f16x8 a, b;
    for (int i = 0; i < 8; ++i) {
        a[i] = _Float16(mfma_operand(lane, i, seed, 1.0f));
        b[i] = _Float16(mfma_operand(lane, i, seed + 1, 1.0f / 1024.0f));
    }
    mfma_f32x16 c[CHAINS];
    for (int j = 0; j < CHAINS; ++j) c[j] = mfma_f32x16{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < CHAINS; ++j) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c[j], 0, 0, 0);
    }
    double got = 0;
    for (int j = 0; j < CHAINS; ++j)
        for (int r = 0; r < 16; ++r) got += double(c[j][r]);
    got = mfma_wave_sum(got, 64);
    double dot = 0;   // this half's sum over its 8 k of colsum(A) * rowsum(B)
    for (int i = 0; i < 8; ++i)
        dot += mfma_wave_sum(double(a[i]), 32) * mfma_wave_sum(double(b[i]), 32);
    const double want = double(iters) * CHAINS * (dot + __shfl_xor(dot, 32, 64));
    if (lane == 0 && got != want) bad[0] = 1;
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
    const unsigned seed = 20251;
    switch (chains) {
    case 4: hipLaunchKernelGGL(mfma_loop<4>, dim3(blocks), dim3(256), 0, stream, bad, iters, seed); break;
    case 8: hipLaunchKernelGGL(mfma_loop<8>, dim3(blocks), dim3(256), 0, stream, bad, iters, seed); break;
    case 16: hipLaunchKernelGGL(mfma_loop<16>, dim3(blocks), dim3(256), 0, stream, bad, iters, seed); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
