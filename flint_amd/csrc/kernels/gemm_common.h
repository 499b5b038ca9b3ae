// Definitions shared by the GEMM kernels (gemm.hip: the register-staged and
// two-workgroup-per-CU family; gemm_pipe.hip: the one-wave-per-SIMD NT
// pipeline): vector types, the epilogue kinds, the LDS swizzle, GELU and its
// derivative, the tile map, wait and barrier helpers, and the kernel operands.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels/kernels.h"

namespace flint {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) _Float16 lds_half;


enum class Layout { kNT, kNN, kTN };
// What the kernel's store stage does. kTn writes FP32 (plain, accumulate or a
// split's partial); kTnHalf is the batched TN's FP16 output.
enum class Store { kNone, kBias, kBiasGelu, kBiasResidual, kDGelu, kScale, kTn, kTnHalf };

// Position of 16-byte chunk `chunk` of LDS row `row` (BK / 8 chunks a row).
// BK 64: 128-byte rows, key (row ^ row >> 3) & 7; BK 32: 64-byte rows, key
// (row >> 1 ^ row >> 2) & 3. Either keeps the 8 / 16 rows that one LDS cycle
// serves (32 / 64 banks) on distinct banks for a fragment read.
template <int BK>
__device__ __forceinline__ int swizzle(int row, int chunk) {
    if constexpr (BK == 64) return chunk ^ ((row ^ (row >> 3)) & 7);
    else return chunk ^ (((row >> 1) ^ (row >> 2)) & 3);
}

// GPT-2's tanh GELU. 0.5 s (1 + tanh u) equals s / (1 + exp(-2u)), which has
// no cancellation for negative s; u = sqrt(2/pi) (s + 0.044715 s^3). The
// exponential is 2^(s (c0 + c1 s^2)) on v_exp_f32 and the quotient one
// v_rcp_f32 multiply: about 1e-6 relative error, far inside FP16's rounding.
// +inf gives +inf, -inf gives NaN (as the tanh form does), large negative s -0.
__device__ __forceinline__ float gelu(float s) {
    constexpr float c0 = -2.3022082f;          // -2 sqrt(2/pi) log2(e)
    constexpr float c1 = -0.10294324f;         // c0 * 0.044715
    const float e = __builtin_amdgcn_exp2f(s * __builtin_fmaf(c1, s * s, c0));
    return s * __builtin_amdgcn_rcpf(1.0f + e);
}

// d/ds [s sigma(2u)] = sigma + s sigma (1 - sigma) 2u', 2u' = 2 sqrt(2/pi)
// (1 + 3 * 0.044715 s^2). 1 - sigma is taken as e sigma for s >= 0 (keeps
// precision as sigma -> 1) and directly for s < 0 (e may overflow there).
// Infinite s returns GELU's limits; NaN propagates. Every lane computes g and
// then selects: the empty asm keeps the compiler from moving g's arithmetic
// into a branch around the rare infinite case (per element, that branch cost
// more than the arithmetic it skipped).
__device__ __forceinline__ float gelu_grad(float s) {
    constexpr float c0 = -2.3022082f;
    constexpr float c1 = -0.10294324f;
    const float e = __builtin_amdgcn_exp2f(s * __builtin_fmaf(c1, s * s, c0));
    const float sigma = __builtin_amdgcn_rcpf(1.0f + e);
    const float one_minus = s < 0.0f ? 1.0f - sigma : e * sigma;
    const float q = s * one_minus * __builtin_fmaf(0.21406444860866706f, s * s, 1.5957691216057308f);
    float g = __builtin_fmaf(sigma, q, sigma);
    asm volatile("" : "+v"(g));
    return __builtin_isinf(s) ? (s > 0.0f ? 1.0f : 0.0f) : g;
}

struct TileArgs {
    int tiles_m, tiles_n;     // macro-tiles per batch / split
    int tiles_per_slice;      // tiles_m * tiles_n
    int slices;               // batches, or k splits for TN
    int group_m;              // grouped ordering width (in m tiles)
    int split_len;            // TN: k per split (multiple of 64)
};

// Maps logical tile id `id` (< tiles_per_slice * slices) to (slice, tile_m,
// tile_n). Workgroups run persistently: workgroup b takes ids b, b + G, b + 2G,
// ... (G = grid size, a multiple of 8 when there are at least 8 ids), so id % 8
// is the XCD the workgroup runs on (XCDs take workgroups round-robin). The
// remap gives XCD x the contiguous range [x * total/8, (x+1) * total/8) of
// tiles when total is a multiple of 8; within a slice, tiles go in groups of
// group_m rows of tiles, column by column, for L2 reuse.
__device__ __forceinline__ void map_tile(const TileArgs& t, unsigned id, int* slice, int* tm,
                                         int* tn) {
    const unsigned total = unsigned(t.tiles_per_slice) * unsigned(t.slices);
    if ((total & 7u) == 0) id = (id & 7u) * (total >> 3) + (id >> 3);
    *slice = int(id / unsigned(t.tiles_per_slice));
    const int in_slice = int(id % unsigned(t.tiles_per_slice));
    const int per_group = t.group_m * t.tiles_n;
    const int group = in_slice / per_group;
    const int first_m = group * t.group_m;
    const int rows = min(t.tiles_m - first_m, t.group_m);
    const int in_group = in_slice - group * per_group;
    *tm = first_m + in_group % rows;
    *tn = in_group / rows;
}

// A wave-uniform pointer held in scalar registers (buffer resources need one).
__device__ __forceinline__ _Float16* uniform_ptr(const _Float16* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(v >> 32));
    return reinterpret_cast<_Float16*>((uint64_t(hi) << 32) | lo);
}

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt left at their maxima), gfx9
// encoding: vmcnt[3:0] in bits 3:0 and vmcnt[5:4] in bits 15:14.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier without a memory fence. __syncthreads() carries a release
// fence, for which the compiler drains vmcnt to 0 before the s_barrier: every
// global->LDS prefetch of later k-steps would then retire at every k-step and
// the pipeline would be one step deep whatever STAGES says. Here LDS traffic
// (ds_write and ds_read) is waited with lgkmcnt(0), and the global->LDS loads
// a step needs are waited by the caller with an explicit vmcnt; loads into
// registers are tracked by the compiler as usual. The empty asm statements keep
// memory accesses from moving across the barrier.
__device__ __forceinline__ void block_sync() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0); vmcnt and expcnt at their maxima
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

struct Operands {
    void* y;
    const _Float16* x;
    const _Float16* w;
    const float* bias;     // bias (n FP32)
    void* aux;             // pre (GELU out / dGELU in) or residual
    float* partials;       // TN split partials, or null
    float scale;
    int accumulate;        // TN: y += instead of y =
    int m, n, k;
    int causal;            // attention (pipeline only): the per-slice m x m
                           // operand (NT's y, NN's and TN's x) is zero, or
                           // not wanted, above its diagonal
    HeadView wv, yv;       // batched NN / TN (pipeline only): w (k-major) and
                           // y as heads views
};

}  // namespace
}  // namespace flint
