// MFMA ceiling microbenchmark (the MI355X counterpart of the reference's
// tensor-core peak loop, ref bench/mma_kernels.cu:16-30): every wave of a full
// grid issues back-to-back v_mfma_f32_32x32x16_f16 on 4 independent
// accumulators, so the loop is bound by the matrix cores alone. Prints one JSON
// line: achieved TFLOP/s, the dense FP16 peak at the device's clock, the ratio.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#include "mfma_kernel.h"

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
    int* bad = nullptr;
    CHECK(hipMalloc(&bad, sizeof(int)));
    CHECK(hipMemset(bad, 0, sizeof(int)));
    const int blocks = cus * 2;   // 2 workgroups of 4 waves per CU
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    CHECK(launch_mfma_loop(4, blocks, bad, iters / 10, 0));
    CHECK(hipDeviceSynchronize());
    CHECK(hipEventRecord(a, 0));
    CHECK(launch_mfma_loop(4, blocks, bad, iters, 0));
    CHECK(hipEventRecord(b, 0));
    CHECK(hipEventSynchronize(b));
    float ms = 0.0f;
    CHECK(hipEventElapsedTime(&ms, a, b));
    const double flops = mfma_loop_flops(blocks, iters, 4);
    int wrong = 0;
    CHECK(hipMemcpy(&wrong, bad, sizeof(int), hipMemcpyDeviceToHost));
    const double tf = flops / (ms * 1e-3) / 1e12;
    const double peak_clock = double(cus) * 4096.0 * (khz * 1e3) / 1e12;
    std::printf("{\"kernel\": \"mfma_f32_32x32x16_f16 loop\", \"tflops\": %.1f, \"cus\": %d, "
                "\"max_sclk_mhz\": %.0f, \"peak_at_max_sclk\": %.1f, \"frac_of_2516.6\": %.4f, "
                "\"ms\": %.3f, \"result_exact\": %s}\n",
                tf, cus, khz / 1e3, peak_clock, tf / 2516.6, ms, wrong ? "false" : "true");
    CHECK(hipFree(bad));
    return wrong ? 1 : 0;
}
