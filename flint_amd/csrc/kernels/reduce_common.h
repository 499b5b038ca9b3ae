// Device helpers shared by the row-reduction kernels: compensated sums, wave64
// reductions, 16-byte chunk (un)packing and an accurate exp built on
// v_exp_f32.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

// No implicit fused multiply-adds anywhere after this point: HIP's __fmul_rn /
// __fadd_rn are plain operators, and a contracted a.sum + u*v would make the
// TwoSum error terms inexact and change the shape-only summation orders.
#pragma clang fp contract(off)

namespace flint {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));

// A rounded sum and the running sum of the rounding errors left in it
// (Knuth's TwoSum per addition; Ogita-Rump-Oishi Sum2).
struct Comp {
    float sum = 0.0f;
    float error = 0.0f;
};

// Single IEEE operations, written here (under contract(off)) rather than via
// HIP's __f*_rn, whose bodies carry the header's contraction setting.
__device__ __forceinline__ float add_rn(float a, float b) { return a + b; }
__device__ __forceinline__ float sub_rn(float a, float b) { return a - b; }
__device__ __forceinline__ float mul_rn(float a, float b) { return a * b; }

__device__ __forceinline__ void comp_add(Comp& a, float v) {
    const float t = add_rn(a.sum, v);
    const float v_part = sub_rn(t, a.sum);
    a.error = add_rn(a.error, add_rn(sub_rn(a.sum, sub_rn(t, v_part)), sub_rn(v, v_part)));
    a.sum = t;
}

// Merges (b_sum, b_error) into a: both errors first, then b's sum by TwoSum.
// Symmetric in a and b bit for bit, since TwoSum's error is exact.
__device__ __forceinline__ void comp_merge(Comp& a, float b_sum, float b_error) {
    const float errors = add_rn(a.error, b_error);
    a.error = 0.0f;
    comp_add(a, b_sum);
    a.error = add_rn(a.error, errors);
}

// Adds d*d with the product's own rounding error (exact via fma).
__device__ __forceinline__ void comp_add_square(Comp& a, float d) {
    const float p = mul_rn(d, d);
    a.error = add_rn(a.error, __builtin_fmaf(d, d, -p));
    comp_add(a, p);
}

// Adds u*v with the product's rounding error.
__device__ __forceinline__ void comp_add_product(Comp& a, float u, float v) {
    const float p = mul_rn(u, v);
    a.error = add_rn(a.error, __builtin_fmaf(u, v, -p));
    comp_add(a, p);
}

// Butterfly over `width` lanes (a power of two up to 64) starting at xor
// offset width/2. Every lane of the group ends with the same bits.
template <int WIDTH>
__device__ __forceinline__ Comp comp_reduce(Comp a) {
#pragma unroll
    for (int off = WIDTH / 2; off > 0; off /= 2) {
        const float s = __shfl_xor(a.sum, off, 64);
        const float e = __shfl_xor(a.error, off, 64);
        comp_merge(a, s, e);
    }
    return a;
}

// DPP lane exchanges for wave-wide all-reductions (no LDS round trip):
// quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror (lane i <-> 7 - i within
// 8) and row_mirror (i <-> 15 - i within 16); then ds_swizzle xor 16 and one
// bpermute for xor 32. After step k every lane holds the total of its group
// of 2^k lanes.
__device__ __forceinline__ float dpp_f(float v, int ctrl_sel) {
    const int x = __builtin_bit_cast(int, v);
    int r;
    switch (ctrl_sel) {
    case 0: r = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false); break;
    case 1: r = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false); break;
    case 2: r = __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false); break;
    case 3: r = __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false); break;
    case 4: r = __builtin_amdgcn_ds_swizzle(x, 0x401F); break;
    default: r = __shfl_xor(x, 32, 64); break;
    }
    return __builtin_bit_cast(float, r);
}

// The value of lane (this lane ^ OFF), OFF a power of two below 64: DPP for
// 1, 2 (quad permutes) and 8 (row_ror:8 within 16 lanes), ds_swizzle for 4
// and 16, ds_bpermute for 32. The same values as __shfl_xor(v, OFF, 64),
// with only the cross-row exchanges through the LDS unit.
template <int OFF>
__device__ __forceinline__ float xor_lane(float v) {
    static_assert(OFF > 0 && OFF < 64 && (OFF & (OFF - 1)) == 0, "a lane bit");
    const int x = __builtin_bit_cast(int, v);
    int r;
    if constexpr (OFF == 1) r = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);
    else if constexpr (OFF == 2) r = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);
    else if constexpr (OFF == 8) r = __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false);
    else if constexpr (OFF == 4) r = __builtin_amdgcn_ds_swizzle(x, 0x101F);
    else if constexpr (OFF == 16) r = __builtin_amdgcn_ds_swizzle(x, 0x401F);
    else r = __shfl_xor(x, 32, 64);
    return __builtin_bit_cast(float, r);
}

// Compensated all-reduce over the 64 lanes; every lane ends with the same
// bits (comp_merge is symmetric). The order differs from comp_reduce<64>.
__device__ __forceinline__ Comp comp_allreduce64(Comp a) {
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        const float s = dpp_f(a.sum, k);
        const float e = dpp_f(a.error, k);
        comp_merge(a, s, e);
    }
    return a;
}

template <int WIDTH>
__device__ __forceinline__ float sum_reduce(float v) {
#pragma unroll
    for (int off = WIDTH / 2; off > 0; off /= 2) v = add_rn(v, __shfl_xor(v, off, 64));
    return v;
}

// IEEE maximum (NaN-propagating) over `width` lanes.
template <int WIDTH>
__device__ __forceinline__ float maximum_reduce(float v) {
#pragma unroll
    for (int off = WIDTH / 2; off > 0; off /= 2)
        v = __builtin_elementwise_maximum(v, __shfl_xor(v, off, 64));
    return v;
}

template <int WIDTH>
__device__ __forceinline__ float max_reduce(float v) {
#pragma unroll
    for (int off = WIDTH / 2; off > 0; off /= 2) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// exp(x) for x <= 0 or NaN (a softmax's score minus its row max), to about 2
// FP32 ulps, by Cody and Waite's argument reduction: hi = RN(x log2e) with
// log2(e) rounded to a float, e = 2^hi from v_exp_f32, and the rest of the
// exponent r = x - hi ln 2 (in natural-log units, exactly what x log2(e) - hi
// is worth once multiplied by ln 2) formed by two fmas with ln 2 split in two
// floats, so r's error is far below 2^-24. exp(x) = e exp(r) = e + e r + ...,
// and |r| < 2^-16 on the clamped range leaves the second order below 2^-33.
// Below -150 the result is +0 (2^hi is below the smallest denormal), so x is
// clamped there first by a NaN-propagating maximum, which keeps r finite
// (x = -inf included) and NaN a NaN.
__device__ __forceinline__ float exp_accurate_nonpos(float x) {
    constexpr float kLog2e = 1.44269502162933349609375f;   // float(log2 e)
    constexpr double kLn2 = 0.6931471805599453094172321;
    constexpr float kLn2Hi = float(kLn2);
    constexpr float kLn2Lo = float(kLn2 - double(kLn2Hi));
    x = __builtin_elementwise_maximum(x, -150.0f);
    const float hi = x * kLog2e;
    const float r = __builtin_fmaf(-hi, kLn2Lo, __builtin_fmaf(-hi, kLn2Hi, x));
    const float e = __builtin_amdgcn_exp2f(hi);
    return __builtin_fmaf(e, r, e);
}

__device__ __forceinline__ void unpack8(const h8& h, float (&v)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = float(h[i]);
}

// RN16 of a value already rounded to FP32, as the reference's
// __float2half_rn of a float. The empty asm hides how x was formed, so that
// the compiler cannot fold the multiply or fma that produced it into a
// v_fma_mix with one rounding straight to FP16 (different in the last bit now
// and then, and chosen per value by the instruction selector).
__device__ __forceinline__ _Float16 to_half(float x) {
    asm("" : "+v"(x));
    return _Float16(x);
}

__device__ __forceinline__ h8 pack8(const float (&v)[8]) {
    h8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = to_half(v[i]);
    return h;
}

// Streaming access for the row passes, which read each input byte and write
// each output byte once per launch: the nt bit marks the lines as the first
// to leave the caches.
__device__ __forceinline__ h8 load_stream(const h8* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void store_stream(h8* p, const h8& v) { __builtin_nontemporal_store(v, p); }

}  // namespace flint
