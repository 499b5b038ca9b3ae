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
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstdint>
#include <mutex>

#include "common/common.h"
#include "common/tuning.h"
#include "kernels/kernels.h"
#include "kernels/reduce_common.h"
#include "kernels/softmax_rows.h"
#include "kernels/split_sum.h"

#pragma clang fp contract(off)

namespace flint {
namespace {

// Row kernels loop over rows with a grid stride; their grids stay below this
// many 256-thread workgroups (2^32 work-items per grid dimension).
constexpr size_t kMaxBlocks = size_t{1} << 22;

// ---------------------------------------------------------------- LayerNorm fwd

constexpr int kLnRowsPerBlock = 4;

// One wave per row; lane l holds float4 groups l, l + 64, ... (up to CPL of
// them). Waves stride over rows (the grid is sized to the GPU), load the next
// row before reducing the current one, and keep gamma and beta in registers
// for all their rows. The two compensated wave reductions use DPP exchanges.
template <int CPL>
__global__ void __launch_bounds__(256)
layernorm_forward_regs(_Float16* __restrict__ y, float* __restrict__ mean,
                       float* __restrict__ rstd, const float* __restrict__ x,
                       const float* __restrict__ gamma, const float* __restrict__ beta,
                       size_t rows, int cols, float eps) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63;
    const int groups = cols >> 2;
    const size_t stride = size_t(gridDim.x) * kLnRowsPerBlock;
    const f4* g4 = reinterpret_cast<const f4*>(gamma);
    const f4* b4 = reinterpret_cast<const f4*>(beta);
    f4 ga[CPL], be[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int g = lane + i * 64;
        ga[i] = g < groups ? g4[g] : f4{};
        be[i] = g < groups ? b4[g] : f4{};
    }
    size_t row = size_t(blockIdx.x) * kLnRowsPerBlock + (threadIdx.x >> 6);
    f4 v[CPL];
    auto load_row = [&](size_t r, f4 (&dst)[CPL]) {
        const f4* xr = reinterpret_cast<const f4*>(x + r * cols);
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int g = lane + i * 64;
            dst[i] = g < groups ? xr[g] : f4{};
        }
    };
    if (row < rows) load_row(row, v);
    for (; row < rows; row += stride) {
        f4 nxt[CPL];
        if (row + stride < rows) load_row(row + stride, nxt);
        Comp s;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            if (lane + i * 64 < groups) {
#pragma unroll
                for (int j = 0; j < 4; ++j) comp_add(s, v[i][j]);
            }
        }
        s = comp_allreduce64(s);
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
        q = comp_allreduce64(q);
        const float var = __fdiv_rn(add_rn(q.sum, q.error), n);
        const float rs = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(var, eps)));
        h4* yr = reinterpret_cast<h4*>(y + row * cols);
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int g = lane + i * 64;
            if (g < groups) {
                h4 o;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    o[j] = to_half(__builtin_fmaf(mul_rn(sub_rn(v[i][j], mu), rs), ga[i][j],
                                                  be[i][j]));
                yr[g] = o;
            }
        }
        if (lane == 0) {
            mean[row] = mu;
            rstd[row] = rs;
        }
#pragma unroll
        for (int i = 0; i < CPL; ++i) v[i] = nxt[i];
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
        yr[c] = to_half(__builtin_fmaf(mul_rn(sub_rn(xr[c], mu), rs), gamma[c], beta[c]));
    if (lane == 0) {
        mean[row] = mu;
        rstd[row] = rs;
    }
    }
}

// ------------------------------------------------------- bias gradient passes

constexpr int kChunkRows = int(kBiasGradientChunkRows);
constexpr int kPhases = 8;   // row phases per chunk: thread y adds rows y, y+8, ...

// Partial (sum, error) pairs per 256-row chunk and column, in the reference's
// order (ref bias_gradient.cu:1-25, layernorm_backward.cu:120-200): for each
// column, row phase y (0..7) adds rows y, y + 8, ... of the chunk in order,
// then phase 0 merges phases 1..7 in order, over the values of dy. The
// chunk's sums go to workspace row 2c, its errors to 2c + 1.
//
// Workgroup = one chunk x 64 * CPL columns: wave y is phase y, lane l holds
// CPL adjacent columns, so a wave reads 128 * CPL B of dy per row. A lane issues all of its (up to 32) row loads before the first add:
// every workgroup keeps its whole chunk slice in flight, which makes the pass
// bandwidth- rather than latency-bound. Workgroup ids run over chunks first
// (measured faster than tiles first on 8192 x 768 and 8192 x 3072).
template <int CPL>
__global__ void __launch_bounds__(kPhases * 64)
column_partials(float* __restrict__ partial, const _Float16* __restrict__ dy, size_t rows,
                int cols, size_t chunks, size_t blocks) {
    constexpr int kPer = kChunkRows / kPhases;   // 32 rows per phase
    constexpr int kTile = 64 * CPL;
    typedef _Float16 hv __attribute__((ext_vector_type(CPL)));
    typedef float fv __attribute__((ext_vector_type(CPL)));
    __shared__ float sums[kPhases - 1][kTile];
    __shared__ float errs[kPhases - 1][kTile];
    const int lane = threadIdx.x & 63;
    const int ph = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    for (size_t b = blockIdx.x; b < blocks; b += gridDim.x) {
        const int tile = int(b / chunks);
        const size_t chunk = b - size_t(tile) * chunks;
        const size_t first = chunk * kChunkRows;
        const int count = rows - first < size_t(kChunkRows) ? int(rows - first) : kChunkRows;
        const int n = count > ph ? (count - ph + kPhases - 1) / kPhases : 0;
        const int col = tile * kTile + lane * CPL;
        const bool live = col < cols;   // cols is a multiple of 8, so of CPL
        // Rows past the chunk's end and columns past cols load element 0
        // instead (always valid) and are never added: no branch around the
        // loads, so all of them issue before the first wait.
        const size_t step = size_t(kPhases) * size_t(cols);
        size_t at = (first + ph) * size_t(cols) + col;
        hv d[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const size_t use = k < n && live ? at : 0;
            d[k] = *reinterpret_cast<const hv*>(dy + use);
            at += step;
        }
        Comp acc[CPL];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            if (k < n) {
#pragma unroll
                for (int j = 0; j < CPL; ++j) comp_add(acc[j], float(d[k][j]));
            }
        }
        if (ph > 0) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                sums[ph - 1][lane * CPL + j] = acc[j].sum;
                errs[ph - 1][lane * CPL + j] = acc[j].error;
            }
        }
        __syncthreads();
        if (ph == 0 && live) {
#pragma unroll
            for (int o = 0; o < kPhases - 1; ++o) {
#pragma unroll
                for (int j = 0; j < CPL; ++j)
                    comp_merge(acc[j], sums[o][lane * CPL + j], errs[o][lane * CPL + j]);
            }
            fv sv, ev;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                sv[j] = acc[j].sum;
                ev[j] = acc[j].error;
            }
            *reinterpret_cast<fv*>(partial + chunk * 2 * cols + col) = sv;
            *reinterpret_cast<fv*>(partial + (chunk * 2 + 1) * cols + col) = ev;
        }
        __syncthreads();
    }
}

// The merged value of a compensated sum. A non-finite sum is returned alone:
// its error is then inf - inf = NaN and would turn an inf column into NaN.
__device__ __forceinline__ float comp_value(const Comp& a) {
    return __builtin_isfinite(a.sum) ? add_rn(a.sum, a.error) : a.sum;
}

// Merges chunk partials per column: each 32-lane half-wave owns 4 columns.
// Lane l merges chunks l, l + 32, ... in order, then a butterfly over the 32
// lanes (xor 16, 8, 4, 2, 1) merges those.
__device__ __forceinline__ void finish_quad(float* out, const float* partial, size_t chunks,
                                            int cols, int accumulate, int quad, int lane) {
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

__global__ void __launch_bounds__(256)
column_finish(float* __restrict__ out, const float* __restrict__ partial, size_t chunks,
              int cols, int accumulate) {
    const int quad = blockIdx.x * 8 + (threadIdx.x >> 5);
    if (quad >= cols / 4) return;   // whole half-waves leave together
    finish_quad(out, partial, chunks, cols, accumulate, quad, threadIdx.x & 31);
}

// A merge of two column-partial sets (a LayerNorm's dbeta into out0, dgamma
// into out1).
struct ColumnFinish {
    float* out0;
    float* out1;
    const float* part0;
    const float* part1;
    size_t chunks;
    int accumulate;
};

// One linear layer's gradients in one launch: workgroups [0, reduce_blocks)
// sum the weight gradient's k-split partials (tn_reduce's loop), the rest
// merge the bias gradient's chunk partials (column_finish's).
__global__ void __launch_bounds__(256)
linear_grads_finish(float* __restrict__ dw, const float* __restrict__ dw_partials, size_t quads,
                    int splits, int accumulate_w, unsigned reduce_blocks, float* __restrict__ db,
                    const float* __restrict__ db_partial, size_t chunks, int cols,
                    int accumulate_b, unsigned finish_blocks, ColumnFinish ln, int ln_cols) {
    if (blockIdx.x < reduce_blocks) {
        add_split_partials(dw, dw_partials, quads, splits, accumulate_w,
                           size_t(blockIdx.x) * 256 + threadIdx.x, size_t(reduce_blocks) * 256);
        return;
    }
    if (blockIdx.x >= reduce_blocks + finish_blocks) {
        // A LayerNorm backward's deferred dbeta / dgamma merge.
        const int ln_quads = ln_cols / 4;
        const int job = int(blockIdx.x - reduce_blocks - finish_blocks) * 8 + (threadIdx.x >> 5);
        if (job >= 2 * ln_quads) return;   // whole half-waves leave together
        const bool second = job >= ln_quads;
        finish_quad(second ? ln.out1 : ln.out0, second ? ln.part1 : ln.part0, ln.chunks, ln_cols,
                    ln.accumulate, second ? job - ln_quads : job, threadIdx.x & 31);
        return;
    }
    const int quad = int(blockIdx.x - reduce_blocks) * 8 + (threadIdx.x >> 5);
    if (quad >= cols / 4) return;   // whole half-waves leave together
    finish_quad(db, db_partial, chunks, cols, accumulate_b, quad, threadIdx.x & 31);
}

// LayerNorm's dbeta and dgamma partials in one pass over dy and x: per
// 256-row chunk and column, exactly the sums of column_partials<false, 1> and
// column_partials<true, 1>, in their order, into part0 and part1. The dx
// kernel launched after it merges them (ColumnFinish).
// Units b = first, first + stride, ... < blocks (chunk x 64 columns each) of a
// kPhases * 64-thread workgroup.
__device__ __forceinline__ void partials2_units(float* part0, float* part1,
                                                const _Float16* __restrict__ dy,
                                                const float* __restrict__ x,
                                                const float* __restrict__ mean,
                                                const float* __restrict__ rstd, size_t rows,
                                                int cols, size_t chunks, size_t blocks,
                                                size_t first, size_t stride_b) {
    constexpr int kPer = kChunkRows / kPhases;
    __shared__ float sums[2][kPhases - 1][64];
    __shared__ float errs[2][kPhases - 1][64];
    const int lane = threadIdx.x & 63;
    const int ph = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    for (size_t b = first; b < blocks; b += stride_b) {
        const int tile = int(b / chunks);
        const size_t chunk = b - size_t(tile) * chunks;
        const size_t first = chunk * kChunkRows;
        const int count = rows - first < size_t(kChunkRows) ? int(rows - first) : kChunkRows;
        const int n = count > ph ? (count - ph + kPhases - 1) / kPhases : 0;
        const int col = tile * 64 + lane;
        const bool live = col < cols;
        const size_t step = size_t(kPhases) * size_t(cols);
        size_t at = (first + ph) * size_t(cols) + col;
        _Float16 d[kPer];
        float xv[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const size_t use = k < n && live ? at : 0;
            d[k] = dy[use];
            xv[k] = x[use];
            at += step;
        }
        // The phase's rows' mean and rstd, lane k holding row k's, loaded with
        // the rows (per-row scalar loads inside the chain below would each
        // wait out a round trip) and taken lane by lane.
        const size_t mrow = lane < n ? first + ph + size_t(lane) * kPhases : 0;
        const float mean_l = mean[mrow];
        const float rstd_l = rstd[mrow];
        Comp acc[2];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            if (k < n) {
                const float mu = __builtin_bit_cast(
                    float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mean_l), k));
                const float rs = __builtin_bit_cast(
                    float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, rstd_l), k));
                comp_add(acc[0], float(d[k]));
                comp_add_product(acc[1], float(d[k]), mul_rn(sub_rn(xv[k], mu), rs));
            }
        }
        if (ph > 0) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                sums[u][ph - 1][lane] = acc[u].sum;
                errs[u][ph - 1][lane] = acc[u].error;
            }
        }
        __syncthreads();
        if (ph == 0 && live) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
#pragma unroll
                for (int o = 0; o < kPhases - 1; ++o)
                    comp_merge(acc[u], sums[u][o][lane], errs[u][o][lane]);
                float* part = u == 0 ? part0 : part1;
                part[chunk * 2 * cols + col] = acc[u].sum;
                part[(chunk * 2 + 1) * cols + col] = acc[u].error;
            }
        }
        __syncthreads();
    }
}

__global__ void __launch_bounds__(kPhases * 64)
column_partials2(float* part0, float* part1, const _Float16* __restrict__ dy,
                 const float* __restrict__ x, const float* __restrict__ mean,
                 const float* __restrict__ rstd, size_t rows, int cols, size_t chunks,
                 size_t blocks) {
    partials2_units(part0, part1, dy, x, mean, rstd, rows, cols, chunks, blocks, blockIdx.x,
                    gridDim.x);
}

hipError_t launch_partials(float* partial, const void* dy, size_t rows, size_t cols,
                           hipStream_t stream) {
    const size_t chunks = (rows + kChunkRows - 1) / kChunkRows;
    // The "partials_cpl" override, 1 | 2 | 4, forces the columns per lane
    // (tuning sweeps).
    int cpl = 1;
    if (const char* e = tuning(Tune::kPartialsCpl)) {
        const int v = std::atoi(e);
        cpl = v == 2 || v == 4 ? v : 1;
    }
    const int tiles = int((cols + 64 * cpl - 1) / (64 * cpl));
    const size_t blocks = chunks * size_t(tiles);
    const dim3 grid(unsigned(std::min<size_t>(blocks, kMaxBlocks)));
    const auto* dyh = static_cast<const _Float16*>(dy);
#define FLINT_PARTIALS(CPL)                                                                    \
    hipLaunchKernelGGL(column_partials<CPL>, grid, dim3(kPhases * 64), 0, stream, partial, dyh, \
                       rows, int(cols), chunks, blocks)
    if (cpl == 1) FLINT_PARTIALS(1);
    else if (cpl == 2) FLINT_PARTIALS(2);
    else FLINT_PARTIALS(4);
#undef FLINT_PARTIALS
    return hipGetLastError();
}

// ------------------------------------------------------------ LayerNorm dx

// The merge of dbeta's and dgamma's chunk partials (column_finish's, for two
// outputs): by the dx kernel's first half-waves before their rows when the
// partials come from the launch before it (the kernel boundary orders them),
// or by ln_params_finish / linear_grads_finish after the one-launch plan.

__device__ __forceinline__ void finish_columns(const ColumnFinish& f, int cols) {
    const int quads = cols / 4;
    for (int job = int(blockIdx.x) * 8 + int(threadIdx.x >> 5); job < 2 * quads;
         job += int(gridDim.x) * 8) {
        const bool second = job >= quads;
        finish_quad(second ? f.out1 : f.out0, second ? f.part1 : f.part0, f.chunks, cols,
                    f.accumulate, second ? job - quads : job, threadIdx.x & 31);
    }
}

// One 32-lane half-wave per row: lane l takes pieces l, l + 32, ... (up to PPL
// of them, 8 columns each), adds g = dy gamma and g xhat over them in order
// with plain FP32 adds, and a 32-lane butterfly totals them. The second pass
// reuses the registers. With dx_half, RN16 of every dx value written goes
// there too (the model's FP16 copy of the residual gradient).
// Rows of workgroup `block` of `blocks` (RPB rows, one per half-wave, each).
template <int PPL, int RPB>
__device__ __forceinline__ void dx_rows(float* __restrict__ dx, const _Float16* __restrict__ dy,
                                        const float* __restrict__ x,
                                        const float* __restrict__ mean,
                                        const float* __restrict__ rstd,
                                        const float* __restrict__ gamma, size_t rows, int cols,
                                        int accumulate, _Float16* __restrict__ dx_half,
                                        size_t block, size_t blocks) {
    for (size_t row = block * RPB + (threadIdx.x >> 5); row < rows; row += blocks * RPB) {
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
            if (dx_half != nullptr) {
                h8 hv;
#pragma unroll
                for (int j = 0; j < 8; ++j) hv[j] = to_half(o[j]);
                *reinterpret_cast<h8*>(dx_half + row * cols + p * 8) = hv;
            }
        }
    }
    }
}

template <int PPL>
__global__ void __launch_bounds__(256)
layernorm_backward_dx(float* __restrict__ dx, const _Float16* __restrict__ dy,
                      const float* __restrict__ x, const float* __restrict__ mean,
                      const float* __restrict__ rstd, const float* __restrict__ gamma,
                      size_t rows, int cols, int accumulate, _Float16* __restrict__ dx_half,
                      ColumnFinish finish) {
    finish_columns(finish, cols);
    dx_rows<PPL, 8>(dx, dy, x, mean, rstd, gamma, rows, cols, accumulate, dx_half, blockIdx.x,
                    gridDim.x);
}

// LayerNorm backward's two passes in one launch: workgroups [0, units) take
// the dbeta / dgamma chunk partials (column_partials2's), the rest dx one row
// per half-wave (layernorm_backward_dx's), so that the latency-bound partials
// overlap the bandwidth-bound rows; ln_params_finish merges the partials
// after it. The same arithmetic in the same order as the two-launch path.
template <int PPL>
__global__ void __launch_bounds__(kPhases * 64)
layernorm_backward_fused(float* part0, float* part1, float* __restrict__ dx,
                         const _Float16* __restrict__ dy, const float* __restrict__ x,
                         const float* __restrict__ mean, const float* __restrict__ rstd,
                         const float* __restrict__ gamma, size_t rows, int cols, size_t chunks,
                         size_t items, unsigned units, int accumulate,
                         _Float16* __restrict__ dx_half) {
    if (blockIdx.x < units) {
        partials2_units(part0, part1, dy, x, mean, rstd, rows, cols, chunks, items, blockIdx.x,
                        units);
        return;
    }
    dx_rows<PPL, kPhases * 2>(dx, dy, x, mean, rstd, gamma, rows, cols, accumulate, dx_half,
                              blockIdx.x - units, gridDim.x - units);
}

__global__ void __launch_bounds__(256) ln_params_finish(ColumnFinish finish, int cols) {
    finish_columns(finish, cols);
}

// Any cols (multiple of 8): the same order, two passes over memory.
__global__ void __launch_bounds__(256)
layernorm_backward_dx_any(float* __restrict__ dx, const _Float16* __restrict__ dy,
                          const float* __restrict__ x, const float* __restrict__ mean,
                          const float* __restrict__ rstd, const float* __restrict__ gamma,
                          size_t rows, int cols, int accumulate, _Float16* __restrict__ dx_half,
                          ColumnFinish finish) {
    finish_columns(finish, cols);
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
            if (dx_half != nullptr) dx_half[row * cols + c] = to_half(v);
        }
    }
    }
}

// ------------------------------------------------------------ causal softmax

constexpr int kSmRowsPerBlock = 4;   // waves per workgroup, one row group each
constexpr int kSmRowsPerWave = 1;   // 96 x 1024: 58.6 us, against 60.3 at 2 rows and 75.1 at 4

// One wave per row of length L <= 1024: lane l holds chunks l and l + 64
// (the row arithmetic is softmax_rows.h's, shared with the fused attention
// passes). Row t sees columns 0..t; masked chunks are written as zeros and
// never read. The zeros go out with the row's values, after its reductions:
// stored first, under the loads, they made the pass slower (60.5 -> 64.7 us
// at 96 x 1024, and 74.2 -> 76.5 for the backward pass).
// A wave takes R consecutive rows and loads all of them before the first
// reduction, so R times the bytes are in flight; each row's arithmetic is
// the one-row order.
template <int R>
__global__ void __launch_bounds__(256)
causal_softmax_forward(h8* __restrict__ p, const h8* __restrict__ s, size_t rows, int length,
                       int zero_span) {
    for (size_t row0 = (size_t(blockIdx.x) * kSmRowsPerBlock + (threadIdx.x >> 6)) * R;
         row0 < rows; row0 += size_t(gridDim.x) * kSmRowsPerBlock * R) {
    const int lane = threadIdx.x & 63;
    const int chunks = length >> 3;
    h8 raw[R][2];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const size_t row = row0 + r;
        const int t = int(row % size_t(length));
        const int visible_chunks = row < rows ? (t >> 3) + 1 : 0;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = lane + i * 64;
            if (c < visible_chunks) raw[r][i] = load_stream(s + row * chunks + c);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const size_t row = row0 + r;
        if (row >= rows) break;
        const int t = int(row % size_t(length));
        softmax_forward_row(p + row * chunks, raw[r], t, chunks, lane, zero_span);
    }
    }
}

// ds = scale * p * ((dp - D.sum) - D.error) over the visible columns, with D
// the compensated sum of the exact products p * dp (softmax_backward_row).
// Each lane reads all of its dp before the butterfly and writes only its own
// chunks afterwards, so ds may alias dp.
__global__ void __launch_bounds__(256)
causal_softmax_backward(h8* ds, const h8* __restrict__ p, const h8* dp, size_t rows, int length,
                        float scale, int zero_span) {
    for (size_t row = size_t(blockIdx.x) * kSmRowsPerBlock + (threadIdx.x >> 6); row < rows;
         row += size_t(gridDim.x) * kSmRowsPerBlock) {
    const int lane = threadIdx.x & 63;
    const int chunks = length >> 3;
    const int t = int(row % size_t(length));
    const int visible_chunks = (t >> 3) + 1;
    h8 ph[2], dh[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = lane + i * 64;
        if (c < visible_chunks) {
            ph[i] = load_stream(p + row * chunks + c);
            dh[i] = load_stream(dp + row * chunks + c);
        }
    }
    softmax_backward_row(ds + row * chunks, ph, dh, t, chunks, lane, scale, zero_span);
    }
}

// --------------------------------------------------- softmax + cross-entropy

// One workgroup of THREADS per row; thread t holds vocab chunks t, t + THREADS,
// ... (up to CPT of them) from a single HBM read, as FP16 (4 VGPRs a chunk).
// Columns at or past vocab are loaded as -inf, so they drop out of the max and
// add exp(-inf) = 0 to the sum.
//   1. mx = max over the row: packed FP16 maximum per chunk, then wave and
//      workgroup. The maximum propagates NaN (the reference's fmaxf skips it),
//      which changes no output: a NaN logit makes the reference's sum, loss and
//      every dlogit NaN through expf(NaN), and a NaN mx does the same here.
//   2. sum = sum of e = exp(l - mx), as 2^((l - mx) log2 e) on v_exp_f32. The
//      gap l - mx is exact for FP16 inputs, so the row's maximum gets e = 1
//      exactly; elsewhere e is within about |l - mx| * 7e-8 relative plus an
//      ulp. Each chunk's 8 values are added pairwise and the chunk total
//      enters a compensated (TwoSum) sum, merged lane -> wave -> workgroup in
//      a fixed order.
//   3. e is formed again from the registers (cheaper than holding 8 FP32
//      values a chunk, which would halve the rows in flight per CU), and
//      dlogits = RN16(scale RN(RN(e / sum) - [c == target])), 0 past vocab;
//      row_loss = log(sum) - (l_target - mx) when target < vocab
//      (ref cross_entropy.cu:106-172 for the formulas).
// Only the lane holding the target's chunk or the partial last chunk takes the
// per-column branch.
template <int THREADS, int CPT, bool POW2_SCALE>
__global__ void __launch_bounds__(THREADS)
softmax_cross_entropy(h8* __restrict__ dlogits, float* __restrict__ row_loss,
                      const h8* __restrict__ logits, const uint16_t* __restrict__ targets,
                      float scale, float one, int vocab, int cols) {
    constexpr int kWaves = THREADS / 64;
    constexpr float kLog2e = 1.44269502162933349609375f;
    __shared__ float red_a[kWaves];
    __shared__ float red_b[kWaves];
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const size_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int chunks = cols >> 3;
    const int vocab_chunks = (vocab + 7) >> 3;
    const int last = vocab_chunks - 1;
    const int last_count = vocab - last * 8;   // 1..8 values of the last chunk count
    const h8* lr = logits + row * chunks;
    h8* dr = dlogits + row * chunks;
    const _Float16 neg_inf = -__builtin_huge_valf16();

    // l - mx rounded once, as an fma with the FP16 value as a mixed-precision
    // operand (one v_fma_mix_f32); `one` is 1.0f passed at run time so that the
    // compiler keeps the fma instead of a convert and a subtract.
    float mx_g = 0.0f;
    auto gap = [&](_Float16 l) { return __builtin_fmaf(float(l), one, -mx_g); };

    h8 raw[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = tid + i * THREADS;
        raw[i] = c < vocab_chunks ? load_stream(lr + c) : h8(neg_inf);
    }
    if (last_count < 8 && last >= tid && (last - tid) % THREADS == 0) {
        const int i = (last - tid) / THREADS;
#pragma unroll
        for (int k = 0; k < CPT; ++k)
            if (k == i) {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (j >= last_count) raw[k][j] = neg_inf;
            }
    }

    // 1. Row max.
    h8 m8 = raw[0];
#pragma unroll
    for (int i = 1; i < CPT; ++i) m8 = __builtin_elementwise_maximum(m8, raw[i]);
    h2 m2 = __builtin_elementwise_maximum(h2{m8[0], m8[1]}, h2{m8[2], m8[3]});
    m2 = __builtin_elementwise_maximum(m2, __builtin_elementwise_maximum(h2{m8[4], m8[5]},
                                                                          h2{m8[6], m8[7]}));
    float mx = __builtin_elementwise_maximum(float(m2[0]), float(m2[1]));
    mx = maximum_reduce<64>(mx);
    if (lane == 0) red_a[wave] = mx;
    __syncthreads();
    mx = red_a[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) mx = __builtin_elementwise_maximum(mx, red_a[w]);
    __syncthreads();
    mx_g = mx;

    // 2. Compensated sum of e.
    Comp s;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = tid + i * THREADS;
        if (c < vocab_chunks) {
            float e[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                e[j] = __builtin_amdgcn_exp2f(mul_rn(gap(raw[i][j]), kLog2e));
            comp_add(s, add_rn(add_rn(add_rn(e[0], e[1]), add_rn(e[2], e[3])),
                               add_rn(add_rn(e[4], e[5]), add_rn(e[6], e[7]))));
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
    for (int w = 1; w < kWaves; ++w) comp_merge(tot, red_a[w], red_b[w]);
    const float sum = add_rn(tot.sum, tot.error);
    const float inv = __fdiv_rn(1.0f, sum);
    // With a power-of-two scale, RN(RN(e inv) scale) = RN(e (inv scale)): both
    // scalings are exact unless the value falls below FP32's normal range,
    // far under FP16's smallest subnormal, where both round to 0 in FP16.
    const float inv_scale = mul_rn(inv, scale);

    // 3. Loss and dlogits.
    const int target = targets[row];
    if (tid == 0 && target < vocab) {
        const float gap_t = gap(reinterpret_cast<const _Float16*>(lr)[target]);
        row_loss[row] = sub_rn(logf(sum), gap_t);
    }
    const int tchunk = target >> 3;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = tid + i * THREADS;
        if (c >= vocab_chunks) continue;
        // An empty asm on the chunk keeps the compiler from carrying pass 2's
        // FP32 gaps (8 VGPRs a chunk) over to here instead of the FP16 chunk
        // (holding pass 2's e instead, 154 VGPRs, one workgroup per CU, ran
        // no faster).
        asm volatile("" : "+v"(raw[i]));
        float e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) e[j] = __builtin_amdgcn_exp2f(mul_rn(gap(raw[i][j]), kLog2e));
        float o[8];
        if (c != tchunk && c != last) {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                o[j] = POW2_SCALE ? mul_rn(e[j], inv_scale) : mul_rn(mul_rn(e[j], inv), scale);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float p = mul_rn(e[j], inv);
                if (c * 8 + j == target) p = sub_rn(p, 1.0f);
                o[j] = c * 8 + j < vocab ? mul_rn(p, scale) : 0.0f;
            }
        }
        store_stream(dr + c, pack8(o));
    }
    for (int c = vocab_chunks + tid; c < chunks; c += THREADS) store_stream(dr + c, h8{});
}

}  // namespace

// ---------------------------------------------------------------- launchers

hipError_t launch_layernorm_forward(void* y, void* mean, void* rstd, const void* x,
                                    const void* gamma, const void* beta, size_t rows, size_t cols,
                                    float eps, hipStream_t stream) {
    // One row per wave (8192 x 768: 9.7 us, against 10.6 with the grid the GPU
    // holds at once and 11.6 with two rows per wave); the kernels stride over
    // rows past the grid's limit.
    const size_t row_blocks = (rows + kLnRowsPerBlock - 1) / kLnRowsPerBlock;
    const unsigned blocks = unsigned(std::min<size_t>(row_blocks, kMaxBlocks));
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

hipError_t launch_bias_partials(void* workspace, const void* dy, size_t rows, size_t cols,
                                hipStream_t stream) {
    return launch_partials(static_cast<float*>(workspace), dy, rows, cols, stream);
}

hipError_t launch_linear_grads_finish(void* dw, const void* dw_partials, size_t m, size_t n,
                                      int splits, bool accumulate_w, void* db,
                                      const void* db_workspace, size_t rows, size_t cols,
                                      bool accumulate_b, hipStream_t stream,
                                      const ParamsMerge* also) {
    const size_t quads = m * n / 4;
    const unsigned reduce_blocks =
        splits > 1 ? unsigned(std::clamp<size_t>((quads + 255) / 256, 1, 8192)) : 0u;
    const size_t chunks = (rows + kChunkRows - 1) / kChunkRows;
    const unsigned finish_blocks = unsigned((cols / 4 + 7) / 8);
    ColumnFinish ln{};
    int ln_cols = 0;
    unsigned ln_blocks = 0;
    if (also != nullptr && also->cols > 0) {
        ln = ColumnFinish{also->dbeta, also->dgamma, also->part0, also->part1, also->chunks,
                          also->accumulate};
        ln_cols = also->cols;
        ln_blocks = unsigned((2 * (ln_cols / 4) + 7) / 8);
    }
    hipLaunchKernelGGL(linear_grads_finish, dim3(reduce_blocks + finish_blocks + ln_blocks),
                       dim3(256), 0, stream, static_cast<float*>(dw),
                       static_cast<const float*>(dw_partials), quads, splits,
                       accumulate_w ? 1 : 0, reduce_blocks, static_cast<float*>(db),
                       static_cast<const float*>(db_workspace), chunks, int(cols),
                       accumulate_b ? 1 : 0, finish_blocks, ln, ln_cols);
    return hipGetLastError();
}

hipError_t launch_params_merge(const ParamsMerge& merge, hipStream_t stream) {
    if (merge.cols <= 0) return hipSuccess;
    const ColumnFinish finish{merge.dbeta, merge.dgamma, merge.part0, merge.part1, merge.chunks,
                              merge.accumulate};
    const unsigned fin = unsigned(std::min<size_t>((2 * (size_t(merge.cols) / 4) + 7) / 8,
                                                   kMaxBlocks));
    hipLaunchKernelGGL(ln_params_finish, dim3(fin), dim3(256), 0, stream, finish, merge.cols);
    return hipGetLastError();
}

hipError_t launch_bias_gradient(void* dbias, const void* dy, size_t rows, size_t cols,
                                bool accumulate, void* workspace, hipStream_t stream) {
    if (hipError_t e = launch_partials(static_cast<float*>(workspace), dy, rows, cols, stream);
        e != hipSuccess) {
        return e;
    }
    return launch_bias_gradient_finish(dbias, workspace, rows, cols, accumulate, stream);
}

hipError_t launch_layernorm_backward(void* dx, void* dgamma, void* dbeta, const void* dy,
                                     const void* x, const void* mean, const void* rstd,
                                     const void* gamma, size_t rows, size_t cols,
                                     bool accumulate_dx, bool accumulate_params, void* workspace,
                                     hipStream_t stream, void* dx_half, ParamsMerge* deferred) {
    if (deferred != nullptr) *deferred = ParamsMerge{};
    if (cols == 0 || cols % 8 != 0 || rows == 0) return hipErrorInvalidValue;
    const size_t chunks = (rows + kChunkRows - 1) / kChunkRows;
    const size_t region = chunks * 2 * cols;   // floats
    auto* part0 = static_cast<float*>(workspace);
    auto* part1 = part0 + region;
    const auto* dyh = static_cast<const _Float16*>(dy);
    const auto* xf = static_cast<const float*>(x);
    const auto* mf = static_cast<const float*>(mean);
    const auto* rf = static_cast<const float*>(rstd);
    const int c = int(cols);
    const size_t items = chunks * ((cols + 63) / 64);
    const ColumnFinish finish{static_cast<float*>(dbeta), static_cast<float*>(dgamma), part0,
                              part1, chunks, accumulate_params ? 1 : 0};
    auto* dxf = static_cast<float*>(dx);
    const auto* gf = static_cast<const float*>(gamma);
    const int acc = accumulate_dx ? 1 : 0;
    auto* dxh = static_cast<_Float16*>(dx_half);
    const size_t pieces = cols / 8;
    // One launch for the partials and dx, then the merge ("ln_fused" = "0":
    // the partials, then dx with the merge; the same bits).
    const bool fused = pieces <= 256 && !tuning_off(Tune::kLnFused);
    if (fused) {
        const size_t units = std::min<size_t>(items, 1u << 20);
        const size_t row_blocks = std::min<size_t>((rows + 15) / 16, kMaxBlocks);
        const dim3 grid(unsigned(units + row_blocks));
#define FLINT_LNF(PPL)                                                                         \
    hipLaunchKernelGGL(layernorm_backward_fused<PPL>, grid, dim3(kPhases * 64), 0, stream,     \
                       part0, part1, dxf, dyh, xf, mf, rf, gf, rows, c, chunks, items,         \
                       unsigned(units), acc, dxh)
        if (pieces <= 32) FLINT_LNF(1);
        else if (pieces <= 64) FLINT_LNF(2);
        else if (pieces <= 96) FLINT_LNF(3);
        else if (pieces <= 128) FLINT_LNF(4);
        else FLINT_LNF(8);
#undef FLINT_LNF
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
        const ParamsMerge merge{static_cast<float*>(dbeta), static_cast<float*>(dgamma), part0,
                                part1, chunks, c, accumulate_params ? 1 : 0};
        if (deferred != nullptr) {
            *deferred = merge;
            return hipSuccess;
        }
        return launch_params_merge(merge, stream);
    }
    // dbeta and dgamma partials, one pass over dy and x.
    hipLaunchKernelGGL(column_partials2, dim3(unsigned(std::min<size_t>(items, kMaxBlocks))),
                       dim3(kPhases * 64), 0, stream, part0, part1, dyh, xf, mf, rf, rows, c,
                       chunks, items);
    // dx, whose first half-waves also merge the partials.
    const unsigned blocks = unsigned(std::min<size_t>((rows + 7) / 8, kMaxBlocks));
#define FLINT_DX(PPL)                                                                        \
    hipLaunchKernelGGL(layernorm_backward_dx<PPL>, dim3(blocks), dim3(256), 0, stream, dxf, dyh, \
                       xf, mf, rf, gf, rows, c, acc, dxh, finish)
    if (pieces <= 32) FLINT_DX(1);
    else if (pieces <= 64) FLINT_DX(2);
    else if (pieces <= 96) FLINT_DX(3);
    else if (pieces <= 128) FLINT_DX(4);
    else if (pieces <= 256) FLINT_DX(8);
    else
        hipLaunchKernelGGL(layernorm_backward_dx_any, dim3(blocks), dim3(256), 0, stream, dxf,
                           dyh, xf, mf, rf, gf, rows, c, acc, dxh, finish);
#undef FLINT_DX
    return hipGetLastError();
}

hipError_t launch_causal_softmax_forward(void* p, const void* s, size_t rows, size_t length,
                                         hipStream_t stream, int zero_span) {
    if (zero_span < 0 || zero_span % 8 != 0) return hipErrorInvalidValue;
    constexpr size_t kRowsPerBlock = size_t(kSmRowsPerBlock) * kSmRowsPerWave;
    const unsigned blocks =
        unsigned(std::min<size_t>((rows + kRowsPerBlock - 1) / kRowsPerBlock, kMaxBlocks));
    hipLaunchKernelGGL(causal_softmax_forward<kSmRowsPerWave>, dim3(blocks), dim3(256), 0, stream,
                       static_cast<h8*>(p), static_cast<const h8*>(s), rows, int(length),
                       zero_span);
    return hipGetLastError();
}

hipError_t launch_causal_softmax_backward(void* ds, const void* p, const void* dp, size_t rows,
                                          size_t length, float scale, hipStream_t stream,
                                          int zero_span) {
    if (zero_span < 0 || zero_span % 8 != 0) return hipErrorInvalidValue;
    const unsigned blocks = unsigned(std::min<size_t>((rows + kSmRowsPerBlock - 1) / kSmRowsPerBlock, kMaxBlocks));
    hipLaunchKernelGGL(causal_softmax_backward, dim3(blocks), dim3(256), 0, stream,
                       static_cast<h8*>(ds), static_cast<const h8*>(p),
                       static_cast<const h8*>(dp), rows, int(length), scale, zero_span);
    return hipGetLastError();
}

hipError_t launch_softmax_cross_entropy(void* dlogits, void* row_loss, const void* logits,
                                        const void* targets, float scale, size_t rows,
                                        size_t vocab, size_t cols, hipStream_t stream) {
    const size_t vc = (vocab + 7) / 8;
    auto* d = static_cast<h8*>(dlogits);
    auto* l = static_cast<float*>(row_loss);
    const auto* lg = static_cast<const h8*>(logits);
    const auto* tg = static_cast<const uint16_t*>(targets);
    // The "ce_threads" override, 256 | 512 | 1024, forces the workgroup size
    // (tuning sweeps);
    // the chunks per thread follow from it.
    // 256 threads while a row fits 25 chunks a thread (GPT-2's 50,257: 305.9
    // to 307.8 us against 309.8 to 309.9 at 512, two runs, the same bits).
    int threads = vc <= 256 * 25 ? 256 : 512;
    if (const char* e = tuning(Tune::kCeThreads)) {
        const int t = std::atoi(e);
        if (t == 256 || t == 512 || t == 1024) threads = t;
    }
    const size_t per = (vc + threads - 1) / threads;
    // A power of two (of either sign) in FP32's normal range.
    int exp2_of_scale = 0;
    const bool pow2 = std::isfinite(scale) && scale != 0.0f &&
                      std::fabs(std::frexp(scale, &exp2_of_scale)) == 0.5f &&
                      std::fpclassify(scale) == FP_NORMAL;
    // Grid x holds up to 2^31 - 1 rows per launch; larger row counts go in slices.
    for (size_t done = 0; done < rows;) {
        const size_t n = std::min<size_t>(rows - done, size_t{1} << 22);
#define FLINT_CE(THREADS, CPT)                                                                   \
    if (pow2)                                                                                    \
        hipLaunchKernelGGL((softmax_cross_entropy<THREADS, CPT, true>), dim3(unsigned(n)),       \
                           dim3(THREADS), 0, stream, d + done * (cols / 8), l + done,            \
                           lg + done * (cols / 8), tg + done, scale, 1.0f, int(vocab),           \
                           int(cols));                                                           \
    else                                                                                         \
        hipLaunchKernelGGL((softmax_cross_entropy<THREADS, CPT, false>), dim3(unsigned(n)),      \
                           dim3(THREADS), 0, stream, d + done * (cols / 8), l + done,            \
                           lg + done * (cols / 8), tg + done, scale, 1.0f, int(vocab),           \
                           int(cols))
#define FLINT_CE_PER(THREADS)                                                                    \
    if (per <= 1) FLINT_CE(THREADS, 1);                                                          \
    else if (per <= 2) FLINT_CE(THREADS, 2);                                                     \
    else if (per <= 4) FLINT_CE(THREADS, 4);                                                     \
    else if (per <= 8) FLINT_CE(THREADS, 8);                                                     \
    else if (per <= 13) FLINT_CE(THREADS, 13);                                                   \
    else if (per <= 16) FLINT_CE(THREADS, 16);                                                   \
    else if (per <= 25) FLINT_CE(THREADS, 25);                                                   \
    else FLINT_CE(THREADS, 32);
        if (threads == 256) { FLINT_CE_PER(256) }
        else if (threads == 512) { FLINT_CE_PER(512) }
        else { FLINT_CE_PER(1024) }
#undef FLINT_CE_PER
#undef FLINT_CE
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
        done += n;
    }
    return hipSuccess;
}

}  // namespace flint

// ---- the bias gradient without a caller's workspace ------------------------
//
// flint_bias_gradient_noalloc keeps the column partials in `scratch`, a
// device array of kBiasGradientScratchBytes that every device the library
// runs on holds until the process ends. The array's name is only a host-side
// handle: host code uses the address hipGetSymbolAddress returns for the
// current device, read once per device on that device's first call. Calls on
// one device share the array, so calls that overlap in time on one device
// (two streams, two threads) race on it; calls in one stream's order do not.
// The partials pass writes every partial the finish pass reads, so nothing
// needs clearing between calls.
static __device__ __align__(256) unsigned char scratch[flint::kBiasGradientScratchBytes];

namespace flint {
namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_lock;
std::atomic<void*> g_scratch[kScratchDevices];

hipError_t scratch_address(void** out) {
    int device = 0;
    if (hipError_t e = hipGetDevice(&device); e != hipSuccess) return e;
    if (device < 0 || device >= kScratchDevices) return hipErrorInvalidDevice;
    void* p = g_scratch[device].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> guard(g_scratch_lock);
        p = g_scratch[device].load(std::memory_order_relaxed);
        if (p == nullptr) {
            if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); e != hipSuccess) return e;
            g_scratch[device].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return hipSuccess;
}

}  // namespace

hipError_t launch_bias_gradient_noalloc(void* dbias, const void* dy, size_t rows, size_t cols,
                                        bool accumulate, hipStream_t stream) {
    if (bias_gradient_workspace(rows, cols) > kBiasGradientScratchBytes) return hipErrorInvalidValue;
    void* ws = nullptr;
    if (hipError_t e = scratch_address(&ws); e != hipSuccess) return e;
    return launch_bias_gradient(dbias, dy, rows, cols, accumulate, ws, stream);
}

}  // namespace flint
