// The GPT-2 model's stored-probability attention (the reference's call
// sequence, ref src/model/gpt2.cpp: scores by the batched NT product, the
// causal softmax, and their backward), with two pairs of its launches fused
// and their intermediate kept out of memory, bit for bit:
//  * scores_softmax: P = causal_softmax_forward(RN16(scale * Q Kᵀ)), the
//    product of flint_gemm_nt_batched followed by
//    flint_causal_softmax_forward;
//  * scores_softmax_backward: dS = causal_softmax_backward(P, RN16(dO Vᵀ)),
//    the product of flint_gemm_nt_batched (scale 1) followed by
//    flint_causal_softmax_backward.
// Each workgroup takes 32 query rows of one head: its eight waves compute the
// row block's scores (or dP) against the keys up to the block's last row with
// the same MFMA chain as the pipeline's NT tile (gemm_pipe.hip: A = 32 key
// rows, B = 32 query rows, k in four 16-wide steps from a zero accumulator,
// then RN16(sum * scale)), stage them as FP16 rows in LDS, and then run the
// row passes of softmax_rows.h on them, one row per wave at a time. The
// scores never reach HBM: the row passes write P (dS) exactly as the public
// entry points do, zeros up to the same zero span included.
// Two workgroups share a CU (66 KB of staged rows each), so 16 waves hide the
// row passes' latency; the row passes' VALU work (exp_accurate per score)
// bounds the forward. Measured in the GPT-2 124M step (8 x 1024 tokens, one
// MI355X, same process): forward 79 us against 40 + 59 us for the product
// and the softmax pass, backward 90 against 40 + 61; the step 14.06 ->
// 13.64 ms. Sixteen waves a workgroup gave 13.61 ms with a register spill in
// the backward; four, 14.60 (slower than the two launches).
// Head width 64, lengths a multiple of 32 up to 1,024 (the staged rows fit in
// LDS); operands are [batches][length][64] FP16 rows, or heads views of token
// rows (HeadView: the model reads q, k, v and dO where the projections left
// them), P and dS [batches][length][length].
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common/common.h"
#include "kernels/kernels.h"
#include "kernels/softmax_rows.h"

namespace flint {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

constexpr int kBlockRows = 32;     // query rows per workgroup: one MFMA B block
constexpr int kHeadWidth = 64;     // k of the products: four MFMA steps
constexpr int kMaxLength = 1024;
constexpr int kPad = 8;            // halves after each staged row (bank spread)
constexpr int kWaves = 8;           // waves per workgroup
constexpr int kGroupsPerWave = kMaxLength / 32 / kWaves;
constexpr int kRowsPerWave = kBlockRows / kWaves;   // row passes per wave
static_assert(kBlockRows % kWaves == 0, "whole rows per wave");

// The staged row stride (halves) for a sequence length, and the block's LDS
// (sized for the longest rows: 66 KB, two workgroups per CU).
__host__ __device__ constexpr int staged_stride(int length) { return length + kPad; }
constexpr int kStagedHalves = kBlockRows * staged_stride(kMaxLength);

// Scores of rows r0 .. r0 + 31 of one head against keys 0 .. r0 + 31 into the
// staged rows `st` (row i of the block at st + i * stride): wave w takes the
// 32-key groups w, w + kWaves, ... Lane l holds query row r0 + l % 32 and, per
// 16-wide k-step, k columns 8 (l / 32) .. + 8 of it (the pipeline's B
// fragment) and likewise key rows (its A fragment); accumulator element r is
// key 8 (r / 4) + 4 (l / 32) + r % 4 of the group for that query.
__device__ __forceinline__ void stage_scores(_Float16* st, int stride, const _Float16* q, int q_ld,
                                             const _Float16* k, int k_ld, int r0, float scale,
                                             int wave, int lane) {
    const int fr = lane & 31, fc = lane >> 5;
    h8 qf[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
        qf[kk] = *reinterpret_cast<const h8*>(q + size_t(r0 + fr) * q_ld + kk * 16 + fc * 8);
    const int groups = r0 / 32 + 1;
    // Every group's key fragments first, so that their loads overlap.
    h8 kf[kGroupsPerWave][4];
#pragma unroll
    for (int gi = 0; gi < kGroupsPerWave; ++gi) {
        const int g = wave + kWaves * gi;
        if (g < groups) {
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                kf[gi][kk] = *reinterpret_cast<const h8*>(k + size_t(g * 32 + fr) * k_ld +
                                                          kk * 16 + fc * 8);
        }
    }
#pragma unroll
    for (int gi = 0; gi < kGroupsPerWave; ++gi) {
        const int g = wave + kWaves * gi;
        if (g < groups) {
            f32x16 acc = {};
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[gi][kk], qf[kk], acc, 0, 0, 0);
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const h4 v = {to_half(acc[r4 * 4 + 0] * scale), to_half(acc[r4 * 4 + 1] * scale),
                              to_half(acc[r4 * 4 + 2] * scale), to_half(acc[r4 * 4 + 3] * scale)};
                *reinterpret_cast<h4*>(st + fr * stride + g * 32 + r4 * 8 + fc * 4) = v;
            }
        }
    }
}

// Workgroup -> (head, 32-row block): the blocks with the most keys first.
__device__ __forceinline__ void block_of(int batches, int blocks_per_head, int* b, int* r0) {
    const int id = int(blockIdx.x);
    *b = id % batches;
    *r0 = (blocks_per_head - 1 - id / batches) * kBlockRows;
}

__global__ void __launch_bounds__(kWaves * 64)
__attribute__((amdgpu_waves_per_eu(kWaves / 2, kWaves / 2)))
scores_softmax(h8* __restrict__ p, const _Float16* __restrict__ q, const _Float16* __restrict__ k,
               HeadView qv, HeadView kv, int batches, int length, float scale, int zero_span) {
    __shared__ __attribute__((aligned(16))) _Float16 staged[kStagedHalves];
    const int wave = int(threadIdx.x >> 6), lane = int(threadIdx.x & 63);
    int b, r0;
    block_of(batches, length / kBlockRows, &b, &r0);
    const size_t head = size_t(b) * length;
    const int stride = staged_stride(length);
    stage_scores(staged, stride, q + head_view_offset(qv, b), qv.ld, k + head_view_offset(kv, b),
                 kv.ld, r0, scale, wave, lane);
    __syncthreads();
    // The wave's rows wave, wave + kWaves, ... side by side.
    const int chunks = length >> 3;
    h8 raw[kRowsPerWave][2];
    int tt[kRowsPerWave];
    h8* prs[kRowsPerWave];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
        const int i = wave + r * kWaves;
        const int t = r0 + i;
        tt[r] = t;
        prs[r] = p + (head + t) * chunks;
        const int visible_chunks = (t >> 3) + 1;
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
            const int c = lane + c2 * 64;
            if (c < visible_chunks)
                raw[r][c2] = *reinterpret_cast<const h8*>(staged + i * stride + c * 8);
        }
    }
    softmax_forward_rows<kRowsPerWave>(prs, raw, tt, chunks, lane, zero_span);
}

// dp staged as above (dO for q, V for k, scale 1); then per row the
// backward's row pass with p from memory. ds may not alias p.
__global__ void __launch_bounds__(kWaves * 64)
__attribute__((amdgpu_waves_per_eu(kWaves / 2, kWaves / 2)))
scores_softmax_backward(h8* __restrict__ ds, const h8* __restrict__ p,
                        const _Float16* __restrict__ dout, const _Float16* __restrict__ v,
                        HeadView dv_, HeadView vv, int batches, int length, float scale,
                        int zero_span) {
    __shared__ __attribute__((aligned(16))) _Float16 staged[kStagedHalves];
    const int wave = int(threadIdx.x >> 6), lane = int(threadIdx.x & 63);
    int b, r0;
    block_of(batches, length / kBlockRows, &b, &r0);
    const size_t head = size_t(b) * length;
    const int stride = staged_stride(length);
    stage_scores(staged, stride, dout + head_view_offset(dv_, b), dv_.ld,
                 v + head_view_offset(vv, b), vv.ld, r0, 1.0f, wave, lane);
    __syncthreads();
    // The wave's rows side by side, their p loads in flight together.
    const int chunks = length >> 3;
    h8 ph[kRowsPerWave][2], dh[kRowsPerWave][2];
    int tt[kRowsPerWave];
    h8* dsr[kRowsPerWave];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
        const int i = wave + r * kWaves;
        const int t = r0 + i;
        const size_t row = head + t;
        tt[r] = t;
        dsr[r] = ds + row * chunks;
        const int visible_chunks = (t >> 3) + 1;
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
            const int c = lane + c2 * 64;
            if (c < visible_chunks) {
                ph[r][c2] = load_stream(p + row * chunks + c);
                dh[r][c2] = *reinterpret_cast<const h8*>(staged + i * stride + c * 8);
            }
        }
    }
    softmax_backward_rows<kRowsPerWave>(dsr, ph, dh, tt, chunks, lane, scale, zero_span);
}

}  // namespace

bool attn_scores_fusable(size_t length, size_t head_width) {
    return head_width == size_t(kHeadWidth) && length >= size_t(kBlockRows) &&
           length % kBlockRows == 0 && length <= size_t(kMaxLength);
}

namespace {

// The operand rows of each slice: a heads view, or [batches][length][64].
HeadView rows_of(const HeadView* v, size_t length) {
    if (v != nullptr) return *v;
    HeadView c;
    c.heads = 1;
    c.ld = kHeadWidth;
    c.seq = (long long)(length) * kHeadWidth;
    c.head = 0;
    return c;
}

bool launchable(size_t batches, size_t length, size_t head_width, int zero_span,
                const HeadView& a, const HeadView& b) {
    auto ok = [&](const HeadView& v) {
        return v.heads > 0 && batches % size_t(v.heads) == 0 && v.ld >= kHeadWidth &&
               v.seq >= 0 && v.head >= 0;
    };
    return attn_scores_fusable(length, head_width) && batches > 0 && batches <= 65535 &&
           zero_span >= 0 && zero_span % 8 == 0 && ok(a) && ok(b);
}

}  // namespace

hipError_t launch_attn_scores_softmax(void* p, const void* q, const void* k, size_t batches,
                                      size_t length, size_t head_width, float scale,
                                      hipStream_t stream, int zero_span, const HeadView* qv,
                                      const HeadView* kv) {
    const HeadView qr = rows_of(qv, length), kr = rows_of(kv, length);
    if (!launchable(batches, length, head_width, zero_span, qr, kr)) return hipErrorInvalidValue;
    const unsigned blocks = unsigned(batches * (length / kBlockRows));
    hipLaunchKernelGGL(scores_softmax, dim3(blocks), dim3(kWaves * 64), 0, stream,
                       static_cast<h8*>(p), static_cast<const _Float16*>(q),
                       static_cast<const _Float16*>(k), qr, kr, int(batches), int(length), scale,
                       zero_span);
    return hipGetLastError();
}

hipError_t launch_attn_scores_softmax_backward(void* ds, const void* p, const void* dout,
                                               const void* v, size_t batches, size_t length,
                                               size_t head_width, float scale,
                                               hipStream_t stream, int zero_span,
                                               const HeadView* dov, const HeadView* vv) {
    const HeadView dr = rows_of(dov, length), vr = rows_of(vv, length);
    if (!launchable(batches, length, head_width, zero_span, dr, vr)) return hipErrorInvalidValue;
    const unsigned blocks = unsigned(batches * (length / kBlockRows));
    hipLaunchKernelGGL(scores_softmax_backward, dim3(blocks), dim3(kWaves * 64), 0, stream,
                       static_cast<h8*>(ds), static_cast<const h8*>(p),
                       static_cast<const _Float16*>(dout), static_cast<const _Float16*>(v), dr,
                       vr, int(batches), int(length), scale, zero_span);
    return hipGetLastError();
}

}  // namespace flint
