// Row and column reductions on wave64: LayerNorm forward/backward, the bias
// gradient, causal softmax forward/backward and the fused softmax +
// cross-entropy. All arithmetic is FP32 and each output rounds once.
//
// Design:
//  * Rows that fit are held in registers, so each input byte crosses HBM once
//    (the reference re-reads rows per pass: ref src/kernels/layernorm.cu:123-150,
//    softmax.cu:86-121, cross_entropy.cu:123-171). All loads and stores are
//    16-byte vectors.
//  * LayerNorm forward and causal softmax take one wave per row; softmax +
//    cross-entropy takes a 512-thread workgroup per 100 KB row.
//  * Where the reference promises a bit-reproducible order that depends only
//    on the shape (bias gradient, LayerNorm's dgamma / dbeta / dx: ref
//    flint.h:144-146, :224-227), the same per-column and per-row orders are
//    kept: 256-row chunks, 8 row-phases per chunk, chunk merges strided over
//    32 lanes and a 32-lane butterfly, run here on half-waves.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "common/common.h"
#include "kernels/kernels.h"
#include "kernels/reduce_common.h"

#pragma clang fp contract(off)

namespace flint {
namespace {

// Row kernels loop over rows with a grid stride; their grids stay below this
// many 256-thread workgroups (2^32 work-items per grid dimension).
constexpr size_t kMaxBlocks = size_t{1} << 22;

// ---------------------------------------------------------------- LayerNorm fwd

constexpr int kLnRowsPerBlock = 4;

// One wave per row; lane l holds float4 groups l, l + 64, ... (up to CPL of
// them) for the whole kernel.
template <int CPL>
__global__ void __launch_bounds__(256)
layernorm_forward_regs(_Float16* __restrict__ y, float* __restrict__ mean,
                       float* __restrict__ rstd, const float* __restrict__ x,
                       const float* __restrict__ gamma, const float* __restrict__ beta,
                       size_t rows, int cols, float eps) {
    for (size_t row = size_t(blockIdx.x) * kLnRowsPerBlock + (threadIdx.x >> 6); row < rows;
         row += size_t(gridDim.x) * kLnRowsPerBlock) {
    const int lane = threadIdx.x & 63;
    const int groups = cols >> 2;
    const f4* xr = reinterpret_cast<const f4*>(x + row * cols);
    f4 v[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int g = lane + i * 64;
        v[i] = g < groups ? xr[g] : f4{};
    }
    Comp s;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        if (lane + i * 64 < groups) {
#pragma unroll
            for (int j = 0; j < 4; ++j) comp_add(s, v[i][j]);
        }
    }
    s = comp_reduce<64>(s);
    const float n = float(cols);
    const float mu = __fdiv_rn(add_rn(s.sum, s.error), n);
    Comp q;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        if (lane + i * 64 < groups) {
#pragma unroll
            for (int j = 0; j < 4; ++j) comp_add_square(q, sub_rn(v[i][j], mu));
        }
    }
    q = comp_reduce<64>(q);
    const float var = __fdiv_rn(add_rn(q.sum, q.error), n);
    const float rs = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(var, eps)));
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    h4* yr = reinterpret_cast<h4*>(y + row * cols);
    const f4* g4 = reinterpret_cast<const f4*>(gamma);
    const f4* b4 = reinterpret_cast<const f4*>(beta);
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int g = lane + i * 64;
        if (g < groups) {
            const f4 ga = g4[g];
            const f4 be = b4[g];
            h4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                o[j] = _Float16(__builtin_fmaf(mul_rn(sub_rn(v[i][j], mu), rs), ga[j], be[j]));
            yr[g] = o;
        }
    }
    if (lane == 0) {
        mean[row] = mu;
        rstd[row] = rs;
    }
    }
}

// Any cols: three passes over the row from memory, scalar values.
__global__ void __launch_bounds__(256)
layernorm_forward_any(_Float16* __restrict__ y, float* __restrict__ mean,
                      float* __restrict__ rstd, const float* __restrict__ x,
                      const float* __restrict__ gamma, const float* __restrict__ beta,
                      size_t rows, int cols, float eps) {
    for (size_t row = size_t(blockIdx.x) * kLnRowsPerBlock + (threadIdx.x >> 6); row < rows;
         row += size_t(gridDim.x) * kLnRowsPerBlock) {
    const int lane = threadIdx.x & 63;
    const float* xr = x + row * cols;
    Comp s;
    for (int c = lane; c < cols; c += 64) comp_add(s, xr[c]);
    s = comp_reduce<64>(s);
    const float n = float(cols);
    const float mu = __fdiv_rn(add_rn(s.sum, s.error), n);
    Comp q;
    for (int c = lane; c < cols; c += 64) comp_add_square(q, sub_rn(xr[c], mu));
    q = comp_reduce<64>(q);
    const float var = __fdiv_rn(add_rn(q.sum, q.error), n);
    const float rs = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(var, eps)));
    _Float16* yr = y + row * cols;
    for (int c = lane; c < cols; c += 64)
        yr[c] = _Float16(__builtin_fmaf(mul_rn(sub_rn(xr[c], mu), rs), gamma[c], beta[c]));
    if (lane == 0) {
        mean[row] = mu;
        rstd[row] = rs;
    }
    }
}

// ------------------------------------------------------- bias gradient passes

constexpr int kChunkRows = int(kBiasGradientChunkRows);
constexpr int kPhases = 8;   // row phases per chunk: thread y adds rows y, y+8, ...
constexpr int kPieceCols = 8;  // 16 bytes of FP16

// Partial (sum, error) pairs per 256-row chunk and column. One wave per block:
// 8 pieces of 8 columns across, 8 row phases down. Thread (px, y) adds rows
// y, y + 8, ... of the chunk in order; then phase 0 merges phases 1..7 in
// order. With DGAMMA the values are dy * xhat, xhat = (x - mean) * rstd;
// otherwise dy. The chunk's sums go to workspace row 2c, its errors to 2c + 1.
template <bool DGAMMA>
__global__ void __launch_bounds__(64)
column_partials(float* __restrict__ partial, const _Float16* __restrict__ dy,
                const float* __restrict__ x, const float* __restrict__ mean,
                const float* __restrict__ rstd, size_t rows, int cols) {
    __shared__ float sums[kPhases][8][kPieceCols];
    __shared__ float errs[kPhases][8][kPieceCols];
    const int px = threadIdx.x & 7;
    const int ph = threadIdx.x >> 3;
    const int pieces = cols / kPieceCols;
    const int piece = blockIdx.x * 8 + px;
    const size_t first = size_t(blockIdx.y) * kChunkRows;
    const size_t end = rows - first < size_t(kChunkRows) ? rows : first + kChunkRows;
    Comp acc[kPieceCols];
    if (piece < pieces) {
        for (size_t r = first + ph; r < end; r += kPhases) {
            const h8 d = *reinterpret_cast<const h8*>(dy + r * cols + piece * kPieceCols);
            if (DGAMMA) {
                const float mu = mean[r];
                const float rs = rstd[r];
                const f4* xp = reinterpret_cast<const f4*>(x + r * cols + piece * kPieceCols);
                const f4 x0 = xp[0];
                const f4 x1 = xp[1];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float xv = j < 4 ? x0[j] : x1[j - 4];
                    comp_add_product(acc[j], float(d[j]), mul_rn(sub_rn(xv, mu), rs));
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) comp_add(acc[j], float(d[j]));
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        sums[ph][px][j] = acc[j].sum;
        errs[ph][px][j] = acc[j].error;
    }
    __syncthreads();
    if (ph != 0 || piece >= pieces) return;
    for (int o = 1; o < kPhases; ++o) {
#pragma unroll
        for (int j = 0; j < 8; ++j) comp_merge(acc[j], sums[o][px][j], errs[o][px][j]);
    }
    float* srow = partial + size_t(blockIdx.y) * 2 * cols + piece * kPieceCols;
    float* erow = srow + cols;
    f4* s4 = reinterpret_cast<f4*>(srow);
    f4* e4 = reinterpret_cast<f4*>(erow);
    s4[0] = f4{acc[0].sum, acc[1].sum, acc[2].sum, acc[3].sum};
    s4[1] = f4{acc[4].sum, acc[5].sum, acc[6].sum, acc[7].sum};
    e4[0] = f4{acc[0].error, acc[1].error, acc[2].error, acc[3].error};
    e4[1] = f4{acc[4].error, acc[5].error, acc[6].error, acc[7].error};
}

// The merged value of a compensated sum. A non-finite sum is returned alone:
// its error is then inf - inf = NaN and would turn an inf column into NaN.
__device__ __forceinline__ float comp_value(const Comp& a) {
    return __builtin_isfinite(a.sum) ? add_rn(a.sum, a.error) : a.sum;
}

// Merges chunk partials per column: each 32-lane half-wave owns 4 columns.
// Lane l merges chunks l, l + 32, ... in order, then a butterfly over the 32
// lanes (xor 16, 8, 4, 2, 1) merges those.
__global__ void __launch_bounds__(256)
column_finish(float* __restrict__ out, const float* __restrict__ partial, size_t chunks,
              int cols, int accumulate) {
    const int quad = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int quads = cols / 4;
    if (quad >= quads) return;   // whole half-waves leave together
    const int lane = threadIdx.x & 31;
    Comp t[4];
    for (size_t c = lane; c < chunks; c += 32) {
        const f4 s = reinterpret_cast<const f4*>(partial + c * 2 * cols)[quad];
        const f4 e = reinterpret_cast<const f4*>(partial + c * 2 * cols + cols)[quad];
#pragma unroll
        for (int j = 0; j < 4; ++j) comp_merge(t[j], s[j], e[j]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) t[j] = comp_reduce<32>(t[j]);
    if (lane != 0) return;
    f4 r = {comp_value(t[0]), comp_value(t[1]), comp_value(t[2]), comp_value(t[3])};
    f4* o = reinterpret_cast<f4*>(out) + quad;
    if (accumulate) {
        const f4 old = *o;
        r = f4{add_rn(old[0], r[0]), add_rn(old[1], r[1]), add_rn(old[2], r[2]),
               add_rn(old[3], r[3])};
    }
    *o = r;
}

hipError_t launch_partials(bool dgamma, float* partial, const void* dy, const void* x,
                           const void* mean, const void* rstd, size_t rows, size_t cols,
                           hipStream_t stream) {
    const unsigned chunks = unsigned((rows + kChunkRows - 1) / kChunkRows);
    const unsigned tiles = unsigned((cols / kPieceCols + 7) / 8);
    const dim3 grid(tiles, chunks);
    if (dgamma) {
        hipLaunchKernelGGL(column_partials<true>, grid, dim3(64), 0, stream, partial,
                           static_cast<const _Float16*>(dy), static_cast<const float*>(x),
                           static_cast<const float*>(mean), static_cast<const float*>(rstd),
                           rows, int(cols));
    } else {
        hipLaunchKernelGGL(column_partials<false>, grid, dim3(64), 0, stream, partial,
                           static_cast<const _Float16*>(dy), nullptr, nullptr, nullptr, rows,
                           int(cols));
    }
    return hipGetLastError();
}

// ------------------------------------------------------------ LayerNorm dx

// One 32-lane half-wave per row: lane l takes pieces l, l + 32, ... (up to PPL
// of them, 8 columns each), adds g = dy gamma and g xhat over them in order
// with plain FP32 adds, and a 32-lane butterfly totals them. The second pass
// reuses the registers.
template <int PPL>
__global__ void __launch_bounds__(256)
layernorm_backward_dx(float* __restrict__ dx, const _Float16* __restrict__ dy,
                      const float* __restrict__ x, const float* __restrict__ mean,
                      const float* __restrict__ rstd, const float* __restrict__ gamma,
                      size_t rows, int cols, int accumulate) {
    for (size_t row = size_t(blockIdx.x) * 8 + (threadIdx.x >> 5); row < rows;
         row += size_t(gridDim.x) * 8) {
    const int lane = threadIdx.x & 31;
    const int pieces = cols / 8;
    const float mu = mean[row];
    const float rs = rstd[row];
    float g[PPL][8];
    float xh[PPL][8];
    float g_sum = 0.0f, gx_sum = 0.0f;
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
        const int p = lane + i * 32;
        if (p < pieces) {
            const h8 d = *reinterpret_cast<const h8*>(dy + row * cols + p * 8);
            const f4* xp = reinterpret_cast<const f4*>(x + row * cols + p * 8);
            const f4* gp = reinterpret_cast<const f4*>(gamma + p * 8);
            const f4 x0 = xp[0], x1 = xp[1], g0 = gp[0], g1 = gp[1];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float xv = j < 4 ? x0[j] : x1[j - 4];
                const float gv = j < 4 ? g0[j] : g1[j - 4];
                g[i][j] = mul_rn(float(d[j]), gv);
                xh[i][j] = mul_rn(sub_rn(xv, mu), rs);
                g_sum = add_rn(g_sum, g[i][j]);
                gx_sum = add_rn(gx_sum, mul_rn(g[i][j], xh[i][j]));
            }
        }
    }
    const float n = float(cols);
    const float g_mean = __fdiv_rn(sum_reduce<32>(g_sum), n);
    const float gx_mean = __fdiv_rn(sum_reduce<32>(gx_sum), n);
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
        const int p = lane + i * 32;
        if (p < pieces) {
            float o[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                o[j] = mul_rn(rs, sub_rn(sub_rn(g[i][j], g_mean), mul_rn(xh[i][j], gx_mean)));
            f4* dp = reinterpret_cast<f4*>(dx + row * cols + p * 8);
            if (accumulate) {
                const f4 a = dp[0], b = dp[1];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    o[j] = add_rn(a[j], o[j]);
                    o[j + 4] = add_rn(b[j], o[j + 4]);
                }
            }
            dp[0] = f4{o[0], o[1], o[2], o[3]};
            dp[1] = f4{o[4], o[5], o[6], o[7]};
        }
    }
    }
}

// Any cols (multiple of 8): the same order, two passes over memory.
__global__ void __launch_bounds__(256)
layernorm_backward_dx_any(float* __restrict__ dx, const _Float16* __restrict__ dy,
                          const float* __restrict__ x, const float* __restrict__ mean,
                          const float* __restrict__ rstd, const float* __restrict__ gamma,
                          size_t rows, int cols, int accumulate) {
    for (size_t row = size_t(blockIdx.x) * 8 + (threadIdx.x >> 5); row < rows;
         row += size_t(gridDim.x) * 8) {
    const int lane = threadIdx.x & 31;
    const int pieces = cols / 8;
    const float mu = mean[row];
    const float rs = rstd[row];
    const _Float16* dr = dy + row * cols;
    const float* xr = x + row * cols;
    float g_sum = 0.0f, gx_sum = 0.0f;
    for (int p = lane; p < pieces; p += 32) {
        for (int j = 0; j < 8; ++j) {
            const int c = p * 8 + j;
            const float gv = mul_rn(float(dr[c]), gamma[c]);
            g_sum = add_rn(g_sum, gv);
            gx_sum = add_rn(gx_sum, mul_rn(gv, mul_rn(sub_rn(xr[c], mu), rs)));
        }
    }
    const float n = float(cols);
    const float g_mean = __fdiv_rn(sum_reduce<32>(g_sum), n);
    const float gx_mean = __fdiv_rn(sum_reduce<32>(gx_sum), n);
    float* o = dx + row * cols;
    for (int p = lane; p < pieces; p += 32) {
        for (int j = 0; j < 8; ++j) {
            const int c = p * 8 + j;
            const float gv = mul_rn(float(dr[c]), gamma[c]);
            const float xh = mul_rn(sub_rn(xr[c], mu), rs);
            float v = mul_rn(rs, sub_rn(sub_rn(gv, g_mean), mul_rn(xh, gx_mean)));
            if (accumulate) v = add_rn(o[c], v);
            o[c] = v;
        }
    }
    }
}

// ------------------------------------------------------------ causal softmax

constexpr int kSmRowsPerBlock = 4;

// One wave per row of length L <= 1024: lane l holds chunks l and l + 64.
// Row t sees columns 0..t; masked chunks are written as zeros and never read.
__global__ void __launch_bounds__(256)
causal_softmax_forward(h8* __restrict__ p, const h8* __restrict__ s, size_t rows, int length) {
    for (size_t row = size_t(blockIdx.x) * kSmRowsPerBlock + (threadIdx.x >> 6); row < rows;
         row += size_t(gridDim.x) * kSmRowsPerBlock) {
    const int lane = threadIdx.x & 63;
    const int chunks = length >> 3;
    const int t = int(row % size_t(length));
    const int visible_chunks = (t >> 3) + 1;
    const h8* sr = s + row * chunks;
    h8* pr = p + row * chunks;
    float v[2][8];
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = lane + i * 64;
        if (c < visible_chunks) {
            unpack8(sr[c], v[i]);
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
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = lane + i * 64;
        if (c < chunks) {
            if (c < visible_chunks) {
                float o[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = mul_rn(v[i][j], inv);
                pr[c] = pack8(o);
            } else {
                pr[c] = h8{};
            }
        }
    }
    }
}

// ds = scale * p * ((dp - D.sum) - D.error) over the visible columns, with D
// the compensated sum of the exact products p * dp. Each lane reads all of
// its dp before the butterfly and writes only its own chunks afterwards, so
// ds may alias dp.
__global__ void __launch_bounds__(256)
causal_softmax_backward(h8* ds, const h8* __restrict__ p, const h8* dp, size_t rows, int length,
                        float scale) {
    for (size_t row = size_t(blockIdx.x) * kSmRowsPerBlock + (threadIdx.x >> 6); row < rows;
         row += size_t(gridDim.x) * kSmRowsPerBlock) {
    const int lane = threadIdx.x & 63;
    const int chunks = length >> 3;
    const int t = int(row % size_t(length));
    const int visible_chunks = (t >> 3) + 1;
    float pv[2][8], dv[2][8];
    Comp d;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = lane + i * 64;
        if (c < visible_chunks) {
            unpack8(p[row * chunks + c], pv[i]);
            unpack8(dp[row * chunks + c], dv[i]);
            const int vis = min(t + 1 - c * 8, 8);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (j < vis) comp_add(d, mul_rn(pv[i][j], dv[i][j]));
        }
    }
    d = comp_reduce<64>(d);
    if (!__builtin_isfinite(d.sum)) d.error = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = lane + i * 64;
        if (c < chunks) {
            if (c < visible_chunks) {
                const int vis = min(t + 1 - c * 8, 8);
                float o[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float diff = sub_rn(sub_rn(dv[i][j], d.sum), d.error);
                    o[j] = j < vis ? mul_rn(mul_rn(pv[i][j], diff), scale) : 0.0f;
                }
                ds[row * chunks + c] = pack8(o);
            } else {
                ds[row * chunks + c] = h8{};
            }
        }
    }
    }
}

// --------------------------------------------------- softmax + cross-entropy

constexpr int kCeThreads = 512;
constexpr int kCeWaves = kCeThreads / 64;

// One workgroup per row. Thread t holds vocab chunks t, t + 512, ... (up to
// CPT of them) from a single HBM read: max, then e = exp(l - max) kept in
// registers with a compensated sum (merged lane -> wave -> workgroup in a fixed
// order), then dlogits = RN16(scale (e / sum - [c == target])) and
// row_loss = log(sum) - (l_target - max).
template <int CPT>
__global__ void __launch_bounds__(kCeThreads)
softmax_cross_entropy(h8* __restrict__ dlogits, float* __restrict__ row_loss,
                      const h8* __restrict__ logits, const uint16_t* __restrict__ targets,
                      float scale, int vocab, int cols) {
    __shared__ float red_a[kCeWaves];
    __shared__ float red_b[kCeWaves];
    const size_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int chunks = cols >> 3;
    const int vocab_chunks = (vocab + 7) >> 3;
    const h8* lr = logits + row * chunks;
    h8* dr = dlogits + row * chunks;

    float v[CPT][8];
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = tid + i * kCeThreads;
        if (c < vocab_chunks) {
            unpack8(lr[c], v[i]);
            const int cnt = min(vocab - c * 8, 8);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (j < cnt) mx = fmaxf(mx, v[i][j]);
        }
    }
    mx = max_reduce<64>(mx);
    if (lane == 0) red_a[wave] = mx;
    __syncthreads();
    mx = red_a[0];
#pragma unroll
    for (int w = 1; w < kCeWaves; ++w) mx = fmaxf(mx, red_a[w]);
    __syncthreads();

    const int target = targets[row];
    float gap_t = 0.0f;
    bool own_target = false;
    Comp s;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = tid + i * kCeThreads;
        if (c < vocab_chunks) {
            const int cnt = min(vocab - c * 8, 8);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float gap = v[i][j] - mx;
                if (j < cnt && c * 8 + j == target) {
                    gap_t = gap;
                    own_target = true;
                }
                v[i][j] = j < cnt ? exp_accurate(gap) : 0.0f;
                if (j < cnt) comp_add(s, v[i][j]);
            }
        }
    }
    s = comp_reduce<64>(s);
    if (lane == 0) {
        red_a[wave] = s.sum;
        red_b[wave] = s.error;
    }
    __syncthreads();
    Comp tot;
    tot.sum = red_a[0];
    tot.error = red_b[0];
#pragma unroll
    for (int w = 1; w < kCeWaves; ++w) comp_merge(tot, red_a[w], red_b[w]);
    const float sum = add_rn(tot.sum, tot.error);
    const float inv = __fdiv_rn(1.0f, sum);
    if (own_target) row_loss[row] = sub_rn(logf(sum), gap_t);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = tid + i * kCeThreads;
        if (c < vocab_chunks) {
            float o[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float pj = mul_rn(v[i][j], inv);
                if (c * 8 + j == target) pj = sub_rn(pj, 1.0f);
                o[j] = mul_rn(pj, scale);
            }
            const int cnt = min(vocab - c * 8, 8);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (j >= cnt) o[j] = 0.0f;
            dr[c] = pack8(o);
        }
    }
    for (int c = vocab_chunks + tid; c < chunks; c += kCeThreads) dr[c] = h8{};
}

}  // namespace

// ---------------------------------------------------------------- launchers

hipError_t launch_layernorm_forward(void* y, void* mean, void* rstd, const void* x,
                                    const void* gamma, const void* beta, size_t rows, size_t cols,
                                    float eps, hipStream_t stream) {
    const unsigned blocks = unsigned(std::min<size_t>((rows + kLnRowsPerBlock - 1) / kLnRowsPerBlock, kMaxBlocks));
    auto* yh = static_cast<_Float16*>(y);
    auto* mf = static_cast<float*>(mean);
    auto* rf = static_cast<float*>(rstd);
    const auto* xf = static_cast<const float*>(x);
    const auto* gf = static_cast<const float*>(gamma);
    const auto* bf = static_cast<const float*>(beta);
    const int c = int(cols);
#define FLINT_LN(CPL)                                                                       \
    hipLaunchKernelGGL(layernorm_forward_regs<CPL>, dim3(blocks), dim3(256), 0, stream, yh, mf, \
                       rf, xf, gf, bf, rows, c, eps)
    const size_t groups = cols / 4;
    if (cols % 4 == 0 && groups <= 64) FLINT_LN(1);
    else if (cols % 4 == 0 && groups <= 128) FLINT_LN(2);
    else if (cols % 4 == 0 && groups <= 192) FLINT_LN(3);
    else if (cols % 4 == 0 && groups <= 256) FLINT_LN(4);
    else if (cols % 4 == 0 && groups <= 512) FLINT_LN(8);
    else if (cols % 4 == 0 && groups <= 1024) FLINT_LN(16);
    else
        hipLaunchKernelGGL(layernorm_forward_any, dim3(blocks), dim3(256), 0, stream, yh, mf, rf,
                           xf, gf, bf, rows, c, eps);
#undef FLINT_LN
    return hipGetLastError();
}

hipError_t launch_bias_gradient_finish(void* out, const void* workspace, size_t rows,
                                       size_t cols, bool accumulate, hipStream_t stream) {
    const size_t chunks = (rows + kChunkRows - 1) / kChunkRows;
    const unsigned blocks = unsigned((cols / 4 + 7) / 8);
    hipLaunchKernelGGL(column_finish, dim3(blocks), dim3(256), 0, stream,
                       static_cast<float*>(out), static_cast<const float*>(workspace), chunks,
                       int(cols), accumulate ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_bias_gradient(void* dbias, const void* dy, size_t rows, size_t cols,
                                bool accumulate, void* workspace, hipStream_t stream) {
    if (hipError_t e = launch_partials(false, static_cast<float*>(workspace), dy, nullptr, nullptr,
                                       nullptr, rows, cols, stream);
        e != hipSuccess) {
        return e;
    }
    return launch_bias_gradient_finish(dbias, workspace, rows, cols, accumulate, stream);
}

hipError_t launch_layernorm_backward(void* dx, void* dgamma, void* dbeta, const void* dy,
                                     const void* x, const void* mean, const void* rstd,
                                     const void* gamma, size_t rows, size_t cols,
                                     bool accumulate_dx, bool accumulate_params, void* workspace,
                                     hipStream_t stream) {
    // dbeta is the bias gradient of dy; dgamma reuses the workspace after it.
    if (hipError_t e = launch_bias_gradient(dbeta, dy, rows, cols, accumulate_params, workspace,
                                            stream);
        e != hipSuccess) {
        return e;
    }
    if (hipError_t e = launch_partials(true, static_cast<float*>(workspace), dy, x, mean, rstd,
                                       rows, cols, stream);
        e != hipSuccess) {
        return e;
    }
    if (hipError_t e = launch_bias_gradient_finish(dgamma, workspace, rows, cols,
                                                   accumulate_params, stream);
        e != hipSuccess) {
        return e;
    }
    const unsigned blocks = unsigned(std::min<size_t>((rows + 7) / 8, kMaxBlocks));
    auto* dxf = static_cast<float*>(dx);
    const auto* dyh = static_cast<const _Float16*>(dy);
    const auto* xf = static_cast<const float*>(x);
    const auto* mf = static_cast<const float*>(mean);
    const auto* rf = static_cast<const float*>(rstd);
    const auto* gf = static_cast<const float*>(gamma);
    const int c = int(cols);
    const int acc = accumulate_dx ? 1 : 0;
    const size_t pieces = cols / 8;
#define FLINT_DX(PPL)                                                                        \
    hipLaunchKernelGGL(layernorm_backward_dx<PPL>, dim3(blocks), dim3(256), 0, stream, dxf, dyh, \
                       xf, mf, rf, gf, rows, c, acc)
    if (pieces <= 32) FLINT_DX(1);
    else if (pieces <= 64) FLINT_DX(2);
    else if (pieces <= 96) FLINT_DX(3);
    else if (pieces <= 128) FLINT_DX(4);
    else if (pieces <= 256) FLINT_DX(8);
    else
        hipLaunchKernelGGL(layernorm_backward_dx_any, dim3(blocks), dim3(256), 0, stream, dxf,
                           dyh, xf, mf, rf, gf, rows, c, acc);
#undef FLINT_DX
    return hipGetLastError();
}

hipError_t launch_causal_softmax_forward(void* p, const void* s, size_t rows, size_t length,
                                         hipStream_t stream) {
    const unsigned blocks = unsigned(std::min<size_t>((rows + kSmRowsPerBlock - 1) / kSmRowsPerBlock, kMaxBlocks));
    hipLaunchKernelGGL(causal_softmax_forward, dim3(blocks), dim3(256), 0, stream,
                       static_cast<h8*>(p), static_cast<const h8*>(s), rows, int(length));
    return hipGetLastError();
}

hipError_t launch_causal_softmax_backward(void* ds, const void* p, const void* dp, size_t rows,
                                          size_t length, float scale, hipStream_t stream) {
    const unsigned blocks = unsigned(std::min<size_t>((rows + kSmRowsPerBlock - 1) / kSmRowsPerBlock, kMaxBlocks));
    hipLaunchKernelGGL(causal_softmax_backward, dim3(blocks), dim3(256), 0, stream,
                       static_cast<h8*>(ds), static_cast<const h8*>(p),
                       static_cast<const h8*>(dp), rows, int(length), scale);
    return hipGetLastError();
}

hipError_t launch_softmax_cross_entropy(void* dlogits, void* row_loss, const void* logits,
                                        const void* targets, float scale, size_t rows,
                                        size_t vocab, size_t cols, hipStream_t stream) {
    const size_t vocab_chunks = (vocab + 7) / 8;
    const size_t per = (vocab_chunks + kCeThreads - 1) / kCeThreads;
    auto* d = static_cast<h8*>(dlogits);
    auto* l = static_cast<float*>(row_loss);
    const auto* lg = static_cast<const h8*>(logits);
    const auto* tg = static_cast<const uint16_t*>(targets);
    // Grid x holds up to 2^31 - 1 rows per launch; larger row counts go in slices.
    for (size_t done = 0; done < rows;) {
        const size_t n = std::min<size_t>(rows - done, size_t{1} << 22);
#define FLINT_CE(CPT)                                                                        \
    hipLaunchKernelGGL(softmax_cross_entropy<CPT>, dim3(unsigned(n)), dim3(kCeThreads), 0,     \
                       stream, d + done * (cols / 8), l + done, lg + done * (cols / 8),      \
                       tg + done, scale, int(vocab), int(cols))
        if (per <= 1) FLINT_CE(1);
        else if (per <= 2) FLINT_CE(2);
        else if (per <= 4) FLINT_CE(4);
        else if (per <= 8) FLINT_CE(8);
        else if (per <= 13) FLINT_CE(13);
        else FLINT_CE(16);
#undef FLINT_CE
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
        done += n;
    }
    return hipSuccess;
}

}  // namespace flint
