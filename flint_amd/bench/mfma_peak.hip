// MFMA ceiling microbenchmark (the MI355X counterpart of the reference's
// tensor-core peak loop, ref bench/mma_kernels.cu:16-30): every wave of a full
// grid issues back-to-back v_mfma_f32_32x32x16_f16 on 4 independent
// accumulators, so the loop is bound by the matrix cores alone. Prints one JSON
// line: achieved TFLOP/s, the dense FP16 peak at the device's clock, the ratio.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__global__ void __launch_bounds__(256) mfma_loop(float* out, int iters, float seed) {
    f16x8 a, b;
    for (int i = 0; i < 8; ++i) {
        a[i] = _Float16(seed * (threadIdx.x + i));
        b[i] = _Float16(seed * (i - threadIdx.x));
    }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < iters; ++it) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c3, 0, 0, 0);
    }
    float s = 0.0f;
    for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i];
    if (s == 12345.678f) out[threadIdx.x] = s;   // keeps the loop alive
}

#define CHECK(x)                                                              \
    do {                                                                      \
        hipError_t e_ = (x);                                                  \
        if (e_ != hipSuccess) {                                               \
            std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));      \
            return 1;                                                         \
        }                                                                     \
    } while (0)

int main(int argc, char** argv) {
    const int iters = argc > 1 ? std::atoi(argv[1]) : 20000;
    int cus = 0, khz = 0;
    CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    CHECK(hipDeviceGetAttribute(&khz, hipDeviceAttributeClockRate, 0));
    float* out = nullptr;
    CHECK(hipMalloc(&out, 1024 * sizeof(float)));
    const int blocks = cus * 2;   // 2 workgroups of 4 waves per CU
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    hipLaunchKernelGGL(mfma_loop, dim3(blocks), dim3(256), 0, 0, out, iters / 10, 1e-3f);
    CHECK(hipDeviceSynchronize());
    CHECK(hipEventRecord(a, 0));
    hipLaunchKernelGGL(mfma_loop, dim3(blocks), dim3(256), 0, 0, out, iters, 1e-3f);
    CHECK(hipEventRecord(b, 0));
    CHECK(hipEventSynchronize(b));
    float ms = 0.0f;
    CHECK(hipEventElapsedTime(&ms, a, b));
    const double flops = double(blocks) * 4 /*waves*/ * iters * 4 /*mfma*/ * 32.0 * 32 * 16 * 2;
    const double tf = flops / (ms * 1e-3) / 1e12;
    const double peak_clock = double(cus) * 4096.0 * (khz * 1e3) / 1e12;
    std::printf("{\"kernel\": \"mfma_f32_32x32x16_f16 loop\", \"tflops\": %.1f, \"cus\": %d, "
                "\"max_sclk_mhz\": %.0f, \"peak_at_max_sclk\": %.1f, \"frac_of_2516.6\": %.4f, "
                "\"ms\": %.3f}\n",
                tf, cus, khz / 1e3, peak_clock, tf / 2516.6, ms);
    CHECK(hipFree(out));
    return 0;
}
