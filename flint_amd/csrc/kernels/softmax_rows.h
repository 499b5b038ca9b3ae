// The row arithmetic of the causal softmax passes, shared by the row kernels
// (reductions.hip: flint_causal_softmax_forward / _backward) and the fused
// attention passes of the GPT-2 model (attention_stored.hip), so that both
// produce the same bits. One wave per row of length <= 1024 (a wave may take
// several rows side by side); lane l holds the
// row's 16-byte chunks l and l + 64 (8 FP16 each). Row t sees columns 0..t;
// chunks past the diagonal are written as zeros (up to written_chunks) and
// never read. Reference formulas: ref src/kernels/softmax.cu (forward),
// ref src/kernels/softmax_backward.cu (backward).
#pragma once

#include <type_traits>

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

// p's rows t[0..R) from their scores, one wave each, the R rows side by side
// (their reductions' lane exchanges interleaved, so that one row's latency
// hides the others'): raw[r] holds this lane's visible chunks of row r (lane
// and lane + 64, those below (t >> 3) + 1). Per row: max, then the sum of
// exp(s - max) in the lane's order (chunk lane, then lane + 64; columns
// 0..7) and the wave's butterfly, then p = RN16(RN(e * RN(1 / sum))). Each
// row's arithmetic is the same whatever R is.
template <int R>
__device__ __forceinline__ void softmax_forward_rows(h8* const (&pr)[R], const h8 (&raw)[R][2],
                                                     const int (&t)[R], int chunks, int lane,
                                                     int zero_span) {
    // The masked columns of the diagonal chunk (the one lane whose chunk
    // holds column t) read as -inf: they leave the max alone and their exp is
    // +0, the 0 the sum adds for them, so no other element needs a select.
    // (The max is never NaN, fmaxf dropping NaN operands, so every masked
    // difference is -inf or, in a row whose max is -inf, NaN; such a row's
    // sum is NaN from its visible columns already. No difference is +inf.)
    float v[R][2][8];
    float mx[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int visible_chunks = (t[r] >> 3) + 1;
        mx[r] = -__builtin_huge_valf();
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = lane + i * 64;
            if (c < visible_chunks) {
                unpack8(raw[r][i], v[r][i]);
                const int vis = t[r] + 1 - c * 8;
                if (vis < 8) {
#pragma unroll
                    for (int j = 1; j < 8; ++j)
                        if (j >= vis) v[r][i][j] = -__builtin_huge_valf();
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) mx[r] = fmaxf(mx[r], v[r][i][j]);
            }
        }
    }
    // max_reduce<64> of each row (the lane exchanges of xor_lane: the max of
    // the same values in the same order).
    auto max_step = [&](auto off) {
#pragma unroll
        for (int r = 0; r < R; ++r) mx[r] = fmaxf(mx[r], xor_lane<decltype(off)::value>(mx[r]));
    };
    max_step(std::integral_constant<int, 32>{});
    max_step(std::integral_constant<int, 16>{});
    max_step(std::integral_constant<int, 8>{});
    max_step(std::integral_constant<int, 4>{});
    max_step(std::integral_constant<int, 2>{});
    max_step(std::integral_constant<int, 1>{});
    float sum[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int visible_chunks = (t[r] >> 3) + 1;
        // -0 + e is e for every e (+0 included), so the first add folds away;
        // lane 0 always adds at least one e >= +0, so the row's sum is never
        // -0 and equals the one started from +0.
        sum[r] = -0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = lane + i * 64;
            if (c < visible_chunks) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    v[r][i][j] = exp_accurate_nonpos(v[r][i][j] - mx[r]);
                    sum[r] = add_rn(sum[r], v[r][i][j]);
                }
            }
        }
    }
    // sum_reduce<64> of each row: the butterfly's adds in its order.
    auto sum_step = [&](auto off) {
#pragma unroll
        for (int r = 0; r < R; ++r) sum[r] = add_rn(sum[r], xor_lane<decltype(off)::value>(sum[r]));
    };
    sum_step(std::integral_constant<int, 32>{});
    sum_step(std::integral_constant<int, 16>{});
    sum_step(std::integral_constant<int, 8>{});
    sum_step(std::integral_constant<int, 4>{});
    sum_step(std::integral_constant<int, 2>{});
    sum_step(std::integral_constant<int, 1>{});
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int visible_chunks = (t[r] >> 3) + 1;
        const float inv = __fdiv_rn(1.0f, sum[r]);
        const int written = written_chunks(t[r], chunks, zero_span);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = lane + i * 64;
            if (c < written) {
                if (c < visible_chunks) {
                    // Masked columns of the diagonal chunk are set to +0, not
                    // formed as 0 * (1 / sum): a row whose sum is NaN keeps
                    // them +0.
                    const int vis = t[r] + 1 - c * 8;
                    float o[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) o[j] = mul_rn(v[r][i][j], inv);
                    if (vis < 8) {
#pragma unroll
                        for (int j = 1; j < 8; ++j)
                            if (j >= vis) o[j] = 0.0f;
                    }
                    pr[r][c] = pack8(o);
                } else {
                    pr[r][c] = h8{};
                }
            }
        }
    }
}

// One row: softmax_forward_rows<1>.
__device__ __forceinline__ void softmax_forward_row(h8* pr, const h8 (&raw)[2], int t, int chunks,
                                                    int lane, int zero_span) {
    h8* const prs[1] = {pr};
    const h8 (&raws)[1][2] = *reinterpret_cast<const h8 (*)[1][2]>(&raw);
    const int ts[1] = {t};
    softmax_forward_rows<1>(prs, raws, ts, chunks, lane, zero_span);
}

// ds's rows t[0..R), one wave each, the R rows side by side: ph[r] and dh[r]
// hold this lane's visible chunks of p and dp. D is the compensated sum
// (TwoSum) of the rounded products p * dp in the lane's order and the wave's
// butterfly; ds = RN16(RN(RN(p * RN(RN(dp - D.sum) - D.error)) * scale)),
// with D.error dropped when D.sum is not finite.
template <int R>
__device__ __forceinline__ void softmax_backward_rows(h8* const (&dsr)[R], const h8 (&ph)[R][2],
                                                      const h8 (&dh)[R][2], const int (&t)[R],
                                                      int chunks, int lane, float scale,
                                                      int zero_span) {
    // The masked columns of the diagonal chunk add a product of -0, which
    // leaves a finite D exactly as it was (its error is never -0), and a
    // D.sum that is not finite drops D.error anyway.
    Comp d[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int visible_chunks = (t[r] >> 3) + 1;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = lane + i * 64;
            if (c < visible_chunks) {
                float pv[8], dv[8];
                unpack8(ph[r][i], pv);
                unpack8(dh[r][i], dv);
                float prod[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) prod[j] = mul_rn(pv[j], dv[j]);
                const int vis = t[r] + 1 - c * 8;
                if (vis < 8) {
#pragma unroll
                    for (int j = 1; j < 8; ++j)
                        if (j >= vis) prod[j] = -0.0f;
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) comp_add(d[r], prod[j]);
            }
        }
    }
    // comp_reduce<64> of each row: the butterfly's merges in its order.
    auto comp_step = [&](auto off) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float s = xor_lane<decltype(off)::value>(d[r].sum);
            const float e = xor_lane<decltype(off)::value>(d[r].error);
            comp_merge(d[r], s, e);
        }
    };
    comp_step(std::integral_constant<int, 32>{});
    comp_step(std::integral_constant<int, 16>{});
    comp_step(std::integral_constant<int, 8>{});
    comp_step(std::integral_constant<int, 4>{});
    comp_step(std::integral_constant<int, 2>{});
    comp_step(std::integral_constant<int, 1>{});
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (!__builtin_isfinite(d[r].sum)) d[r].error = 0.0f;
        const int visible_chunks = (t[r] >> 3) + 1;
        const int written = written_chunks(t[r], chunks, zero_span);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = lane + i * 64;
            if (c < written) {
                if (c < visible_chunks) {
                    float pv[8], dv[8];
                    unpack8(ph[r][i], pv);
                    unpack8(dh[r][i], dv);
                    const int vis = t[r] + 1 - c * 8;
                    float o[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const float diff = sub_rn(sub_rn(dv[j], d[r].sum), d[r].error);
                        o[j] = mul_rn(mul_rn(pv[j], diff), scale);
                    }
                    if (vis < 8) {
#pragma unroll
                        for (int j = 1; j < 8; ++j)
                            if (j >= vis) o[j] = 0.0f;
                    }
                    store_stream(dsr[r] + c, pack8(o));
                } else {
                    store_stream(dsr[r] + c, h8{});
                }
            }
        }
    }
}

// One row: softmax_backward_rows<1>.
__device__ __forceinline__ void softmax_backward_row(h8* dsr, const h8 (&ph)[2], const h8 (&dh)[2],
                                                     int t, int chunks, int lane, float scale,
                                                     int zero_span) {
    h8* const dsrs[1] = {dsr};
    const h8 (&phs)[1][2] = *reinterpret_cast<const h8 (*)[1][2]>(&ph);
    const h8 (&dhs)[1][2] = *reinterpret_cast<const h8 (*)[1][2]>(&dh);
    const int ts[1] = {t};
    softmax_backward_rows<1>(dsrs, phs, dhs, ts, chunks, lane, scale, zero_span);
}

}  // namespace flint
