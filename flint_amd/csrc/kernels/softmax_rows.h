// The row arithmetic of the causal softmax passes, shared by the row kernels
// (reductions.hip: flint_causal_softmax_forward / _backward) and the fused
// attention passes of the GPT-2 model (attention_stored.hip), so that both
// produce the same bits. One wave per row of length <= 1024; lane l holds the
// row's 16-byte chunks l and l + 64 (8 FP16 each). Row t sees columns 0..t;
// chunks past the diagonal are written as zeros (up to written_chunks) and
// never read. Reference formulas: ref src/kernels/softmax.cu (forward),
// ref src/kernels/softmax_backward.cu (backward).
#pragma once

#include "kernels/reduce_common.h"

namespace flint {

// Chunks of row t written by the causal passes: all of them, or with a zero
// span Z, those below the end of the Z-column block holding the diagonal (the
// model's causal GEMMs read no further; the chunks past it keep old values).
__device__ __forceinline__ int written_chunks(int t, int chunks, int zero_span) {
    if (zero_span == 0) return chunks;
    const int end = (t / zero_span + 1) * (zero_span >> 3);
    return end < chunks ? end : chunks;
}

// p's row t from its scores: raw holds this lane's visible chunks (lane and
// lane + 64, those below (t >> 3) + 1). max, then sum of exp(s - max) in the
// lane's order (chunk lane, then lane + 64; columns 0..7) and the wave's
// butterfly, then p = RN16(RN(e * RN(1 / sum))).
__device__ __forceinline__ void softmax_forward_row(h8* pr, const h8 (&raw)[2], int t, int chunks,
                                                    int lane, int zero_span) {
    const int visible_chunks = (t >> 3) + 1;
    float v[2][8];
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = lane + i * 64;
        if (c < visible_chunks) {
            unpack8(raw[i], v[i]);
            const int vis = min(t + 1 - c * 8, 8);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (j < vis) mx = fmaxf(mx, v[i][j]);
        }
    }
    mx = max_reduce<64>(mx);
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = lane + i * 64;
        if (c < visible_chunks) {
            const int vis = min(t + 1 - c * 8, 8);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                v[i][j] = j < vis ? exp_accurate(v[i][j] - mx) : 0.0f;
                sum = add_rn(sum, v[i][j]);
            }
        }
    }
    sum = sum_reduce<64>(sum);
    const float inv = __fdiv_rn(1.0f, sum);
    const int written = written_chunks(t, chunks, zero_span);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = lane + i * 64;
        if (c < written) {
            if (c < visible_chunks) {
                // Masked columns of the diagonal chunk are selected as +0, not
                // formed as 0 / sum: a row whose sum is NaN keeps them +0.
                const int vis = min(t + 1 - c * 8, 8);
                float o[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = j < vis ? mul_rn(v[i][j], inv) : 0.0f;
                pr[c] = pack8(o);
            } else {
                pr[c] = h8{};
            }
        }
    }
}

// ds's row t: pv and dv hold this lane's visible chunks of p and dp. D is the
// compensated sum (TwoSum) of the rounded products p * dp in the lane's order
// and the wave's butterfly; ds = RN16(RN(RN(p * RN(RN(dp - D.sum) - D.error))
// * scale)), with D.error dropped when D.sum is not finite.
__device__ __forceinline__ void softmax_backward_row(h8* dsr, const float (&pv)[2][8],
                                                     const float (&dv)[2][8], int t, int chunks,
                                                     int lane, float scale, int zero_span) {
    const int visible_chunks = (t >> 3) + 1;
    Comp d;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = lane + i * 64;
        if (c < visible_chunks) {
            const int vis = min(t + 1 - c * 8, 8);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (j < vis) comp_add(d, mul_rn(pv[i][j], dv[i][j]));
        }
    }
    d = comp_reduce<64>(d);
    if (!__builtin_isfinite(d.sum)) d.error = 0.0f;
    const int written = written_chunks(t, chunks, zero_span);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = lane + i * 64;
        if (c < written) {
            if (c < visible_chunks) {
                const int vis = min(t + 1 - c * 8, 8);
                float o[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float diff = sub_rn(sub_rn(dv[i][j], d.sum), d.error);
                    o[j] = j < vis ? mul_rn(mul_rn(pv[i][j], diff), scale) : 0.0f;
                }
                store_stream(dsr + c, pack8(o));
            } else {
                store_stream(dsr + c, h8{});
            }
        }
    }
}

}  // namespace flint
