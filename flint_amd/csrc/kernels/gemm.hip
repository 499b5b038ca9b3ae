// The GEMM family on gfx950 matrix cores: FP16 operands, FP32 accumulation in
// v_mfma_f32_32x32x16_f16, one rounding per output.
//
// Layouts (ref src/kernels/gemm.cu:1-12 for the semantics):
//   NT  y(m x n) = x(m x k) w(n x k)^T     forward linear layer
//   NN  y(m x n) = x(m x k) w(k x n)       input gradient
//   TN  y(m x n) = x(k x m)^T w(k x n)     weight gradient, FP32 out, split-K
//
// Design (MI355X-first, not a translation of the reference's warp tiling):
//  * A workgroup of 256 threads (4 wave64s, WAVES_M x WAVES_N) owns a BM x BN
//    macro-tile and walks k in steps of BK (32 or 64). Both operands sit in
//    LDS as k-contiguous rows, so a lane's MFMA fragment is one ds_read_b128.
//    16-byte chunks are XOR-swizzled per row so that any 8 (32-bank) or 16
//    (64-bank) consecutive lanes of a fragment read hit distinct banks.
//  * Whole NT tiles stream global -> LDS with global_load_lds_dwordx4 (no
//    register staging) through a ring of STAGES buffers, STAGES - 1 k-steps
//    ahead of the MFMAs: one barrier per k-step, global latency hidden by
//    up to three k-steps of math.
//  * Operands stored k-major (NN's w, both TN operands), and edge tiles that
//    need bounds checks, go through registers: 8x8 blocks of halves are read
//    as 8 rows of 16 bytes, transposed in registers and written as 8 LDS rows
//    one k-step ahead, so the LDS layout and the MFMA loop are the same.
//  * The MFMA's A operand is the w tile and its B operand the x tile, so a
//    lane's 16 accumulators are 4 runs of 4 consecutive output columns of one
//    output row: 8-byte (FP16) / 16-byte (FP32) stores and 16-byte bias and
//    residual loads in the epilogue.
//  * Workgroup ids are remapped so each of the 8 XCDs (which take workgroups
//    round-robin) owns a contiguous, grouped block of tiles and reuses operand
//    rows from its own L2.
//  * Epilogues (bias, bias+GELU writing pre and y, bias+residual into FP32,
//    dGELU, scale) run on the FP32 accumulators before the single rounding.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "common/common.h"
#include "common/tuning.h"
#include "kernels/kernels.h"
#include "kernels/gemm_common.h"
#include "kernels/split_sum.h"

namespace flint {
namespace {

// Streams a ROWS x BK tile of a k-contiguous matrix straight into LDS with
// buffer_load_dwordx4 ... lds. The buffer resource covers the tile's rows (base
// = its first row, every k); the k-step goes in the scalar offset, so a lane's
// address is one 32-bit vector offset computed once. Instruction i of wave w
// fills 1 KB of LDS, rows [(4i + w) R, +R) with R = 512 / BK; lane l writes the
// 16 bytes at position l % C of row l / C (C = BK / 8 chunks a row), so it
// loads the global chunk the swizzle puts there.
// (Buffer rather than global addressing: on MI355X the global form stalled the
// address unit on the L1 for a large share of the GEMM's cycles.)
template <int ROWS, int BK, int THREADS>
struct LdsTile {
    static constexpr int kWaves = THREADS / 64;
    static constexpr int kC = BK / 8;
    static constexpr int kRowsPerInstr = 64 / kC;
    static constexpr int kInstr = ROWS * kC / THREADS;   // per thread
    static_assert(ROWS * kC % THREADS == 0, "whole wave instructions");

    _Float16* base;
    unsigned voff[kInstr];

    __device__ __forceinline__ void init(const _Float16* tile_base, size_t ld, int tid) {
        base = uniform_ptr(tile_base);
        const int lane = tid & 63;
        const int wave = tid >> 6;
#pragma unroll
        for (int i = 0; i < kInstr; ++i) {
            const int row = (i * kWaves + wave) * kRowsPerInstr + lane / kC;
            const int kc = swizzle<BK>(row, lane % kC);
            voff[i] = unsigned((size_t(row) * ld + kc * 8) * sizeof(_Float16));
        }
    }
    // Instruction i of load(): k columns [k0, k0 + BK) of its rows.
    __device__ __forceinline__ void load_one(int i, int k0, lds_half* lds, int tid) const {
#if defined(__HIP_DEVICE_COMPILE__)
        const auto rsrc = __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7fffffff, 0x00020000);
        const int row0 = (i * kWaves + (tid >> 6)) * kRowsPerInstr;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsrc, (__attribute__((address_space(3))) void*)(lds + row0 * BK), 16, voff[i],
            unsigned(k0) * 2u, 0, 0);
#endif
    }
    // Loads k columns [k0, k0 + BK) (k0 in elements) into `lds`.
    __device__ __forceinline__ void load(int k0, lds_half* lds, int tid) const {
        // The host pass of this file never runs kernel code; it only has to
        // see a kernel it can emit a launch stub for, which the buffer-resource
        // builtins (device-only types) would prevent.
#if defined(__HIP_DEVICE_COMPILE__)
        // 0x00020000: 32-bit data format, the raw-buffer word 3 of gfx9 parts.
        const auto rsrc = __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7fffffff, 0x00020000);
        const int wave = tid >> 6;
#pragma unroll
        for (int i = 0; i < kInstr; ++i) {
            const int row0 = (i * kWaves + wave) * kRowsPerInstr;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rsrc, (__attribute__((address_space(3))) void*)(lds + row0 * BK), 16, voff[i],
                unsigned(k0) * 2u, 0, 0);
        }
#endif
    }
};



// Waits until at most `tiles` tiles of PER loads each are outstanding.
template <int PER, int MAX>
__device__ __forceinline__ void wait_tiles(int tiles) {
    if constexpr (MAX <= 0) {
        wait_vmcnt<0>();
    } else {
        if (tiles >= MAX) wait_vmcnt<MAX * PER>();
        else wait_tiles<PER, MAX - 1>(tiles);
    }
}

// Copies a ROWS x BK tile of a k-contiguous matrix into LDS rows through
// registers (16-byte chunks), with optional bounds checks.
template <int ROWS, int BK, bool CHECK, int THREADS>
struct DirectTile {
    static constexpr int kC = BK / 8;
    static constexpr int kChunks = ROWS * kC;
    static constexpr int kPer = (kChunks + THREADS - 1) / THREADS;
    f16x8 r[kPer];

    __device__ __forceinline__ void load(const _Float16* __restrict__ base, size_t ld,
                                         int rows_valid, int k_valid, int tid) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int c = tid + i * THREADS;
            if (kChunks % THREADS != 0 && c >= kChunks) continue;
            const int row = c / kC;
            const int kc = c % kC;
            const _Float16* p = base + size_t(row) * ld + kc * 8;
            if (CHECK) {
                r[i] = (row < rows_valid && kc * 8 < k_valid) ? *reinterpret_cast<const f16x8*>(p)
                                                             : f16x8{};
            } else {
                r[i] = *reinterpret_cast<const f16x8*>(p);
            }
        }
    }
    __device__ __forceinline__ void store(_Float16* lds, int tid) const {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int c = tid + i * THREADS;
            if (kChunks % THREADS != 0 && c >= kChunks) continue;
            const int row = c / kC;
            const int kc = c % kC;
            *reinterpret_cast<f16x8*>(lds + row * BK + swizzle<BK>(row, kc) * 8) = r[i];
        }
    }
};

// Copies the transpose of a BK x ROWS tile of a matrix stored with k as its row
// index (element (k, c) at base + k*ld + c) into ROWS LDS rows of BK k values:
// 8x8 blocks of halves are read as 8 rows of 16 bytes and transposed in
// registers.
template <int ROWS, int BK, bool CHECK, int THREADS>
struct TransposedTile {
    static constexpr int kColBlocks = ROWS / 8;
    static constexpr int kBlocks = kColBlocks * (BK / 8);
    static constexpr int kPer = (kBlocks + THREADS - 1) / THREADS;
    f16x8 r[kPer][8];

    __device__ __forceinline__ void load(const _Float16* __restrict__ base, size_t ld,
                                         int cols_valid, int k_valid, int tid) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int b = tid + i * THREADS;
            if (kBlocks % THREADS != 0 && b >= kBlocks) continue;
            const int cb = b % kColBlocks;
            const int kb = b / kColBlocks;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int kr = kb * 8 + e;
                const _Float16* p = base + size_t(kr) * ld + cb * 8;
                if (CHECK) {
                    r[i][e] = (kr < k_valid && cb * 8 < cols_valid)
                                  ? *reinterpret_cast<const f16x8*>(p)
                                  : f16x8{};
                } else {
                    r[i][e] = *reinterpret_cast<const f16x8*>(p);
                }
            }
        }
    }
    __device__ __forceinline__ void store(_Float16* lds, int tid) const {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int b = tid + i * THREADS;
            if (kBlocks % THREADS != 0 && b >= kBlocks) continue;
            const int cb = b % kColBlocks;
            const int kb = b / kColBlocks;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                f16x8 o;
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = r[i][e][j];
                const int row = cb * 8 + j;
                *reinterpret_cast<f16x8*>(lds + row * BK + swizzle<BK>(row, kb) * 8) = o;
            }
        }
    }
};


// Registers a lane may hold: 512 (one wave per SIMD) when its accumulators
// alone take 192 or more, else 256 (two waves per SIMD, or two workgroups).
template <int BM, int BN, int WAVES_M, int NW>
constexpr int waves_per_simd() {
    return NW == 8 || (BM / WAVES_M) * (BN / (NW / WAVES_M)) / 64 < 192 ? 2 : 1;
}

// NW wave64s per workgroup (4 or 8) in a WAVES_M x (NW / WAVES_M) grid.
template <int BM, int BN, int BK, int STAGES, int WAVES_M, int NW, Layout L, Store S, bool CHECK>
__global__ void __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu(waves_per_simd<BM, BN, WAVES_M, NW>())))
gemm_kernel(Operands op, TileArgs ta) {
    constexpr int kThreads = NW * 64;
    constexpr int WAVES_N = NW / WAVES_M;
    constexpr int WTM = BM / WAVES_M;   // wave tile rows (m)
    constexpr int WTN = BN / WAVES_N;   // wave tile cols (n)
    constexpr int FM = WTM / 32;
    constexpr int FN = WTN / 32;
    constexpr int KK = BK / 16;         // MFMA k sub-steps per k-step
    // STAGES 0 selects the register-staged pipeline for NT as well.
    constexpr bool kDirect = L == Layout::kNT && !CHECK && STAGES >= 2;
    constexpr int kStages = kDirect ? STAGES : 2;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tiles are whole 32x32 MFMA blocks");
    static_assert(kStages >= 2, "at least double buffering");

    using TileA =
        typename std::conditional<L == Layout::kTN, TransposedTile<BM, BK, CHECK, kThreads>,
                                  DirectTile<BM, BK, CHECK, kThreads>>::type;
    using TileB =
        typename std::conditional<L == Layout::kNT, DirectTile<BN, BK, CHECK, kThreads>,
                                  TransposedTile<BN, BK, CHECK, kThreads>>::type;

    // Stage s: A tile (BM rows) then B tile (BN rows), BK halves per row.
    __shared__ __attribute__((aligned(16))) _Float16 lds[kStages][(BM + BN) * BK];

    const int tid = threadIdx.x;
    const int m = op.m, n = op.n;
    const unsigned total = unsigned(ta.tiles_per_slice) * unsigned(ta.slices);
    if (blockIdx.x >= total) return;

    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N;
    const int wn = wave % WAVES_N;
    const int frag_row = lane & 31;
    const int frag_chunk = lane >> 5;

    // A tile's place: its slice (a batch, or a TN split of k), output corner,
    // operand pointers at its first k and its k range.
    struct Geo {
        int slice, m0, n0, k_len;
        size_t y_batch;
        const _Float16* a;
        const _Float16* b;
    };
    size_t a_ld, b_ld, a_step, b_step;
    if (L == Layout::kTN) { a_ld = m; a_step = size_t(BK) * m; }
    else { a_ld = op.k; a_step = BK; }
    if (L == Layout::kNT) { b_ld = op.k; b_step = BK; }
    else { b_ld = n; b_step = size_t(BK) * n; }
    auto geo = [&](unsigned id) {
        Geo g;
        int tm, tn;
        map_tile(ta, id, &g.slice, &tm, &tn);
        g.m0 = tm * BM;
        g.n0 = tn * BN;
        const _Float16* x = op.x;
        const _Float16* w = op.w;
        int k_begin = 0, k_end = op.k;
        g.y_batch = 0;
        if (S == Store::kTn && op.partials != nullptr) {
            k_begin = g.slice * ta.split_len;
            k_end = min(op.k, k_begin + ta.split_len);
        } else if (ta.slices > 1) {
            x += size_t(g.slice) * m * op.k;
            w += size_t(g.slice) * n * op.k;
            g.y_batch = size_t(g.slice) * m * n;
        }
        g.a = L == Layout::kTN ? x + size_t(k_begin) * m + g.m0 : x + size_t(g.m0) * op.k + k_begin;
        g.b = L == Layout::kNT ? w + size_t(g.n0) * op.k + k_begin : w + size_t(k_begin) * n + g.n0;
        g.k_len = k_end - k_begin;
        return g;
    };

    f32x16 acc[FN][FM];
    auto zero_acc = [&]() {
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FM; ++j) acc[i][j] = f32x16{};
    };
    zero_acc();

    // Fragment reads of k16 sub-step kk from LDS stage `st`.
    auto read_frags = [&](int st, int kk, f16x8 (&xa)[FM], f16x8 (&wb)[FN]) {
        const _Float16* la = lds[st];
        const _Float16* lb = lds[st] + BM * BK;
        const int chunk = kk * 2 + frag_chunk;
#pragma unroll
        for (int j = 0; j < FM; ++j) {
            const int row = wm * WTM + j * 32 + frag_row;
            xa[j] = *reinterpret_cast<const f16x8*>(la + row * BK + swizzle<BK>(row, chunk) * 8);
        }
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            const int row = wn * WTN + i * 32 + frag_row;
            wb[i] = *reinterpret_cast<const f16x8*>(lb + row * BK + swizzle<BK>(row, chunk) * 8);
        }
    };
    // One k-step of MFMAs from LDS stage `st`. Fragments are double-buffered
    // in registers: sub-step kk + 1's reads are issued before sub-step kk's
    // MFMAs, and scheduling fences keep the compiler from sinking them back
    // next to their uses (it otherwise reuses one register set and waits on
    // every read). `between(kk)` runs after sub-step kk's MFMAs.
    auto compute_step = [&](int st, auto&& between, auto&& early) {
        f16x8 xa[2][FM];
        f16x8 wb[2][FN];
        read_frags(st, 0, xa[0], wb[0]);
        // The first kLead MFMAs of sub-step kk go out before sub-step kk + 1's
        // reads, so the wait those reads need lands behind the rest of kk's
        // MFMAs rather than in front of them.
        constexpr int kLead = FM * FN > 2 ? 2 : 1;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            const int cb = kk & 1;
#pragma unroll
            for (int q = 0; q < FM * FN; ++q) {
                const int i = q / FM, j = q % FM;
                if (q == kLead) {
                    __builtin_amdgcn_sched_barrier(0);
                    if (kk + 1 < KK) read_frags(st, kk + 1, xa[cb ^ 1], wb[cb ^ 1]);
                    early(kk);
                    __builtin_amdgcn_sched_barrier(0);
                }
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wb[cb][i], xa[cb][j], acc[i][j],
                                                                   0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            between(kk);
        }
    };

    // Residual epilogue of the direct path: the tile's residual values and
    // bias go into registers when its k-loop starts (prefetch()), so their HBM
    // reads overlap the MFMAs instead of stalling the store stage.
    // Bias epilogues of the direct path prefetch their bias the same way, so
    // the store stage issues no loads: a load there would make the waves wait
    // (in-order vmcnt) for the next tile's prefetched k-steps as well.
    constexpr bool kPrefetch = S == Store::kBiasResidual && kDirect;
    constexpr bool kPrefetchBias =
        kDirect && (S == Store::kBias || S == Store::kBiasGelu || S == Store::kBiasResidual);
    struct Prefetched {
        f32x4 res[kPrefetch ? FM : 1][kPrefetch ? FN : 1][4];
        f32x4 bias[kPrefetchBias ? FN : 1][4];
    } pre;
    auto prefetch = [&](const Geo& t) {
        const int col_lane = (lane >> 5) * 4;
        if constexpr (kPrefetchBias) {
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    pre.bias[i][g] = *reinterpret_cast<const f32x4*>(
                        op.bias + t.n0 + wn * WTN + i * 32 + g * 8 + col_lane);
        }
        if constexpr (kPrefetch) {
            const float* res = static_cast<const float*>(op.aux);
#pragma unroll
            for (int j = 0; j < FM; ++j) {
                const int row = t.m0 + wm * WTM + j * 32 + frag_row;
#pragma unroll
                for (int i = 0; i < FN; ++i)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int col = t.n0 + wn * WTN + i * 32 + g * 8 + col_lane;
                        pre.res[j][i][g] = *reinterpret_cast<const f32x4*>(
                            res + t.y_batch + size_t(row) * n + col);
                    }
            }
        }
    };

    // Store stage for tile `t` (the accumulators hold its sums).
    auto store_tile = [&](const Geo& t) {
        const int slice = t.slice, m0 = t.m0, n0 = t.n0;
        const size_t y_batch = t.y_batch;
        // Store stage. Lane holds output row m0 + wm*WTM + j*32 + (lane & 31) and,
        // for each group g, 4 consecutive columns n0 + wn*WTN + i*32 + 8g + 4*(lane>>5).
        const int col_lane = (lane >> 5) * 4;
    #pragma unroll
        for (int j = 0; j < FM; ++j) {
            const int row = m0 + wm * WTM + j * 32 + frag_row;
            if (CHECK && row >= m) continue;
    #pragma unroll
            for (int i = 0; i < FN; ++i) {
    #pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int col = n0 + wn * WTN + i * 32 + g * 8 + col_lane;
                    float v[4] = {acc[i][j][g * 4 + 0], acc[i][j][g * 4 + 1], acc[i][j][g * 4 + 2],
                                  acc[i][j][g * 4 + 3]};
                    const size_t at = y_batch + size_t(row) * n + col;
                    const bool whole = !CHECK || (col + 3 < n && (n & 3) == 0);
                    if (CHECK && col >= n) continue;
                    if (S == Store::kTn) {
                        float* out = op.partials ? op.partials + size_t(slice) * m * n
                                                 : static_cast<float*>(op.y);
                        const bool add = op.partials == nullptr && op.accumulate;
                        if (whole) {
                            f32x4* p = reinterpret_cast<f32x4*>(out + at);
                            f32x4 r = {v[0], v[1], v[2], v[3]};
                            if (add) r = *p + r;
                            *p = r;
                        } else {
                            for (int q = 0; q < 4; ++q)
                                if (col + q < n) out[at + q] = add ? out[at + q] + v[q] : v[q];
                        }
                        continue;
                    }
                    if (S == Store::kBias || S == Store::kBiasGelu || S == Store::kBiasResidual) {
                        if constexpr (kPrefetchBias) {
                            const f32x4 b = pre.bias[kPrefetchBias ? i : 0][g];
                            v[0] += b[0]; v[1] += b[1]; v[2] += b[2]; v[3] += b[3];
                        } else if (whole) {
                            const f32x4 b = *reinterpret_cast<const f32x4*>(op.bias + col);
                            v[0] += b[0]; v[1] += b[1]; v[2] += b[2]; v[3] += b[3];
                        } else {
                            for (int q = 0; q < 4; ++q) v[q] += col + q < n ? op.bias[col + q] : 0.0f;
                        }
                    }
                    if (S == Store::kBiasResidual) {
                        float* out = static_cast<float*>(op.y);
                        const float* res = static_cast<const float*>(op.aux);
                        if constexpr (kPrefetch) {
                            const f32x4 r = pre.res[kPrefetch ? j : 0][kPrefetch ? i : 0][g];
                            f32x4 o = {r[0] + v[0], r[1] + v[1], r[2] + v[2], r[3] + v[3]};
                            *reinterpret_cast<f32x4*>(out + at) = o;
                        } else if (whole) {
                            const f32x4 r = *reinterpret_cast<const f32x4*>(res + at);
                            f32x4 o = {r[0] + v[0], r[1] + v[1], r[2] + v[2], r[3] + v[3]};
                            *reinterpret_cast<f32x4*>(out + at) = o;
                        } else {
                            for (int q = 0; q < 4; ++q)
                                if (col + q < n) out[at + q] = res[at + q] + v[q];
                        }
                        continue;
                    }
                    if (S == Store::kScale) {
                        for (int q = 0; q < 4; ++q) v[q] *= op.scale;
                    }
                    if (S == Store::kDGelu) {
                        const _Float16* pre = static_cast<const _Float16*>(op.aux);
                        if (whole) {
                            const f16x4 p = *reinterpret_cast<const f16x4*>(pre + at);
                            for (int q = 0; q < 4; ++q) v[q] *= gelu_grad(float(p[q]));
                        } else {
                            for (int q = 0; q < 4; ++q)
                                if (col + q < n) v[q] *= gelu_grad(float(pre[at + q]));
                        }
                    }
                    _Float16* out = static_cast<_Float16*>(op.y);
                    if (S == Store::kBiasGelu) {
                        _Float16* pre = static_cast<_Float16*>(op.aux);
                        if (whole) {
                            f16x4 p = {_Float16(v[0]), _Float16(v[1]), _Float16(v[2]), _Float16(v[3])};
                            *reinterpret_cast<f16x4*>(pre + at) = p;
                        } else {
                            for (int q = 0; q < 4; ++q)
                                if (col + q < n) pre[at + q] = _Float16(v[q]);
                        }
                        for (int q = 0; q < 4; ++q) v[q] = gelu(v[q]);
                    }
                    if (whole) {
                        f16x4 o = {_Float16(v[0]), _Float16(v[1]), _Float16(v[2]), _Float16(v[3])};
                        *reinterpret_cast<f16x4*>(out + at) = o;
                    } else {
                        for (int q = 0; q < 4; ++q)
                            if (col + q < n) out[at + q] = _Float16(v[q]);
                    }
                }
            }
        }

    };

    if constexpr (kDirect) {
        // One stream of k-steps over all of this workgroup's tiles (ids
        // blockIdx.x, + gridDim.x, ...; NT has no k splits, so every tile has
        // `steps` of them). Step g of the stream lives in stage g % STAGES and
        // is issued STAGES - 1 steps ahead, across tile boundaries: the next
        // tile's first loads are in flight while this one's epilogue stores.
        const int steps = (op.k + BK - 1) / BK;
        const unsigned n_tiles = (total - 1 - blockIdx.x) / gridDim.x + 1;
        const int total_steps = int(n_tiles) * steps;
        constexpr int kPer = LdsTile<BM, BK, kThreads>::kInstr + LdsTile<BN, BK, kThreads>::kInstr;
        // Vector stores one store stage issues per lane.
        constexpr int kStoreInstr = FM * FN * 4 * (S == Store::kBiasGelu ? 2 : 1);
        constexpr int kAfterStore = (STAGES - 2) * kPer + kStoreInstr < 63
                                        ? (STAGES - 2) * kPer + kStoreInstr : 63;
        // Not with the residual prefetch: its extra branch led the compiler to
        // drain vmcnt before every barrier (seen in the ISA), which costs more
        // than the drained stores.
        constexpr bool kWaitPastStores = !kPrefetch;
        Geo cur = geo(blockIdx.x);
        LdsTile<BM, BK, kThreads> tile_a;
        LdsTile<BN, BK, kThreads> tile_b;
        tile_a.init(cur.a, a_ld, tid);
        tile_b.init(cur.b, b_ld, tid);
        int iss_tile = 0;   // tile (index in this workgroup's list) being issued
        auto issue = [&](int g) {
            const int t = g / steps;
            if (t != iss_tile) {
                iss_tile = t;
                const Geo ng = geo(blockIdx.x + unsigned(t) * gridDim.x);
                tile_a.base = uniform_ptr(ng.a);
                tile_b.base = uniform_ptr(ng.b);
            }
            const int k0 = (g - t * steps) * BK;
            _Float16* st = lds[g % STAGES];
            tile_a.load(k0, (lds_half*)st, tid);
            tile_b.load(k0, (lds_half*)(st + BM * BK), tid);
        };
#pragma unroll
        for (int g = 0; g < STAGES - 1; ++g)
            if (g < total_steps) issue(g);
        int g = 0;   // position in the stream
        for (unsigned t = 0; t < n_tiles; ++t) {
            if (t > 0) cur = geo(blockIdx.x + t * gridDim.x);
            prefetch(cur);
            for (int s = 0; s < steps; ++s, ++g) {
                // Step g has landed once only the steps issued after it remain
                // (and, right after a store stage, its stores: vmcnt retires in
                // issue order, so the stores need not drain first).
                if (kWaitPastStores && s == 0 && t > 0 && total_steps - 1 - g >= STAGES - 2)
                    wait_vmcnt<kAfterStore>();
                else
                    wait_tiles<kPer, STAGES - 2>(min(total_steps - 1 - g, STAGES - 2));
                block_sync();   // step g visible; stage (g - 1) % STAGES idle
                if (g + STAGES - 1 < total_steps) issue(g + STAGES - 1);
                compute_step(g % STAGES, [](int) {}, [](int) {});
            }
            store_tile(cur);
            zero_acc();
        }
    } else {
        for (unsigned id = blockIdx.x; id < total; id += gridDim.x) {
            const Geo cur = geo(id);
            const int a_rows_valid = m - cur.m0;
            const int b_rows_valid = n - cur.n0;
            const int k_len = cur.k_len;
            const int steps = (k_len + BK - 1) / BK;
            // Register-staged: tile s + 1 is written to the idle stage during
            // sub-step 0 of step s, and tile s + 2's global loads go out after it.
            TileA ta_regs;
            TileB tb_regs;
            ta_regs.load(cur.a, a_ld, a_rows_valid, k_len, tid);
            tb_regs.load(cur.b, b_ld, b_rows_valid, k_len, tid);
            ta_regs.store(lds[0], tid);
            tb_regs.store(lds[0] + BM * BK, tid);
            if (steps > 1) {
                const int k_left = k_len - BK;
                ta_regs.load(cur.a + a_step, a_ld, a_rows_valid, k_left, tid);
                tb_regs.load(cur.b + b_step, b_ld, b_rows_valid, k_left, tid);
            }
            block_sync();
            for (int s = 0; s < steps; ++s) {
                const int c = s & 1;
                compute_step(c, [&](int kk) {
                    if (kk == 0 && s + 1 < steps) {
                        ta_regs.store(lds[c ^ 1], tid);
                        tb_regs.store(lds[c ^ 1] + BM * BK, tid);
                        if (s + 2 < steps) {
                            const int k_left = k_len - (s + 2) * BK;
                            ta_regs.load(cur.a + (s + 2) * a_step, a_ld, a_rows_valid, k_left,
                                         tid);
                            tb_regs.load(cur.b + (s + 2) * b_step, b_ld, b_rows_valid, k_left,
                                         tid);
                        }
                    }
                }, [](int) {});
                block_sync();
            }
            store_tile(cur);
            zero_acc();
        }
    }
}

// Adds a split TN's partials in split order: y = old + (p0 + p1 + ...), or
// y = p0 + p1 + ... (add_split_partials).
__global__ void __launch_bounds__(256)
tn_reduce(float* __restrict__ y, const float* __restrict__ partials, size_t quads, int splits,
          int accumulate) {
    add_split_partials(y, partials, quads, splits, accumulate,
                       size_t(blockIdx.x) * blockDim.x + threadIdx.x,
                       size_t(gridDim.x) * blockDim.x);
}

struct Config {
    int bm, bn, bk, stages, waves_m, waves;
};

// Every instantiated tile configuration. `occ` is how many workgroups of it
// share one CU (LDS and register limits), `eff` its measured throughput per
// unit of tile area at that occupancy, relative to 128x192 (GPT-2 shapes at
// 8,192 tokens on MI355X; the selector below uses both).
struct Cand {
    Config c;
    int occ;
    double eff;
    bool pick;   // considered by the selector (the rest: FLINT_GEMM_CONFIG only)
};
constexpr Cand kCands[] = {
    {{128, 192, 64, 2, 2, 4}, 2, 1.00, true},  {{256, 192, 64, 2, 2, 4}, 1, 0.93, true},
    {{128, 128, 64, 2, 2, 4}, 2, 0.92, true},  {{64, 128, 64, 2, 1, 4}, 3, 0.70, true},
    {{128, 64, 64, 2, 4, 4}, 3, 0.70, true},   {{128, 256, 64, 2, 2, 4}, 1, 0.90, true},
    {{128, 192, 64, 3, 2, 4}, 1, 0.80, false},
#ifdef FLINT_GEMM_SWEEP
    // Tuning-sweep configurations (FLINT_GEMM_CONFIG only), built with
    // -DFLINT_GEMM_SWEEP so the product library stays quick to compile.
    {{256, 128, 64, 2, 2, 4}, 1, 0.85, false},
    {{128, 128, 64, 4, 2, 4}, 1, 0.70, false}, {{256, 192, 32, 4, 2, 4}, 1, 0.85, false},
    {{128, 192, 32, 4, 2, 4}, 2, 0.90, false}, {{128, 192, 64, 0, 2, 4}, 2, 1.00, false},
    {{256, 192, 64, 0, 2, 4}, 1, 0.90, false}, {{256, 256, 64, 2, 2, 4}, 1, 0.85, false},
    {{256, 256, 64, 2, 2, 8}, 1, 1.00, false}, {{256, 256, 64, 2, 4, 8}, 1, 1.00, false},
    {{256, 128, 64, 2, 4, 8}, 1, 1.00, false}, {{128, 256, 64, 2, 2, 8}, 1, 1.00, false},
    {{256, 256, 32, 4, 2, 8}, 1, 1.00, false}, {{128, 192, 32, 6, 2, 4}, 1, 1.00, false},
    {{256, 192, 32, 5, 2, 4}, 1, 1.00, false}, {{128, 192, 64, 3, 4, 8}, 1, 1.00, false},
#endif
};

// Workgroups of configuration c that share a CU.
int occupancy(const Config& c) {
    for (const Cand& k : kCands)
        if (k.c.bm == c.bm && k.c.bn == c.bn && k.c.bk == c.bk && k.c.stages == c.stages &&
            k.c.waves_m == c.waves_m && k.c.waves == c.waves)
            return k.occ;
    return 1;
}

// The "gemm_config" override, "bm,bn,bk,stages,waves_m[,waves]", forces one of
// the instantiated configurations (tuning sweeps); unset or unknown, the cost
// model below picks.
bool forced_config(Config* out) {
    const char* e = tuning(Tune::kGemmConfig);
    if (e == nullptr) return false;
    Config c{};
    c.waves = 4;
    const int got = std::sscanf(e, "%d,%d,%d,%d,%d,%d", &c.bm, &c.bn, &c.bk, &c.stages,
                                &c.waves_m, &c.waves);
    if (got != 5 && got != 6) return false;
    for (const Cand& k : kCands) {
        if (k.c.bm == c.bm && k.c.bn == c.bn && k.c.bk == c.bk && k.c.stages == c.stages &&
            k.c.waves_m == c.waves_m && k.c.waves == c.waves) {
            *out = c;
            return true;
        }
    }
    return false;
}

// The macro-tile for an m x n output with `slices` independent slices:
// minimises (rounds of tiles over CUs x occupancy) x (tile area x occupancy /
// efficiency). Epilogue-heavy GELU output prefers the 256x192 tile (one
// workgroup per CU), and TN's transposed loads the 128x256 one.
Config pick_config(size_t m, size_t n, size_t slices, int cus, bool gelu, bool tn,
                   bool residual = false) {
    Config forced;
    if (forced_config(&forced)) return forced;
    // The residual epilogue holds its prefetched residual and bias in
    // registers, which leaves one 128x192 workgroup per CU: three stages then
    // keep two k-steps of loads in flight (measured 17-20% faster at 8192 x
    // 768 with k = 768 and 3,072).
    if (residual && m % 128 == 0 && n % 192 == 0) return Config{128, 192, 64, 3, 2, 4};
    Config best = kCands[0].c;
    double best_cost = 1e300;
    for (const Cand& k : kCands) {
        if (!k.pick) continue;
        const Config& c = k.c;
        if (c.bn > 64 && n <= 64) continue;
        double eff = k.eff;
        if (gelu && c.bm == 256 && c.bn == 192) eff = 1.15;
        if (tn && c.bm == 128 && c.bn == 256) eff = 1.15;
        const double tiles = double((m + c.bm - 1) / c.bm) * double((n + c.bn - 1) / c.bn) *
                             double(slices);
        const double rounds = std::ceil(tiles / (double(cus) * k.occ));
        const double cost = rounds * double(c.bm) * double(c.bn) * k.occ / eff;
        if (cost < best_cost * 0.999) {
            best_cost = cost;
            best = c;
        }
    }
    return best;
}

template <Layout L, Store S, bool CHECK>
hipError_t dispatch(const Config& c, dim3 grid, const Operands& op, const TileArgs& ta,
                    hipStream_t stream) {
#define FLINT_GEMM_CASE(BM_, BN_, BK_, ST_, WM_, NW_)                                       \
    if (c.bm == BM_ && c.bn == BN_ && c.bk == BK_ && c.stages == ST_ && c.waves_m == WM_ &&   \
        c.waves == NW_) {                                                                     \
        hipLaunchKernelGGL((gemm_kernel<BM_, BN_, BK_, ST_, WM_, NW_, L, S, CHECK>), grid,    \
                           dim3(NW_ * 64), 0, stream, op, ta);                                \
        return hipGetLastError();                                                             \
    }
    FLINT_GEMM_CASE(128, 192, 64, 2, 2, 4)
    FLINT_GEMM_CASE(256, 192, 64, 2, 2, 4)
    FLINT_GEMM_CASE(128, 128, 64, 2, 2, 4)
    FLINT_GEMM_CASE(64, 128, 64, 2, 1, 4)
    FLINT_GEMM_CASE(128, 64, 64, 2, 4, 4)
    FLINT_GEMM_CASE(128, 256, 64, 2, 2, 4)
    FLINT_GEMM_CASE(128, 192, 64, 3, 2, 4)
#ifdef FLINT_GEMM_SWEEP
    FLINT_GEMM_CASE(256, 128, 64, 2, 2, 4)
    FLINT_GEMM_CASE(128, 128, 64, 4, 2, 4)
    FLINT_GEMM_CASE(256, 192, 32, 4, 2, 4)
    FLINT_GEMM_CASE(128, 192, 32, 4, 2, 4)
    FLINT_GEMM_CASE(128, 192, 64, 0, 2, 4)
    FLINT_GEMM_CASE(256, 192, 64, 0, 2, 4)
    FLINT_GEMM_CASE(256, 256, 64, 2, 2, 4)
    FLINT_GEMM_CASE(256, 256, 64, 2, 2, 8)
    FLINT_GEMM_CASE(256, 256, 64, 2, 4, 8)
    FLINT_GEMM_CASE(256, 128, 64, 2, 4, 8)
    FLINT_GEMM_CASE(128, 256, 64, 2, 2, 8)
    FLINT_GEMM_CASE(256, 256, 32, 4, 2, 8)
    FLINT_GEMM_CASE(128, 192, 32, 6, 2, 4)
    FLINT_GEMM_CASE(256, 192, 32, 5, 2, 4)
    FLINT_GEMM_CASE(128, 192, 64, 3, 4, 8)
#endif
#undef FLINT_GEMM_CASE
    return hipErrorInvalidValue;
}

template <Layout L, Store S>
hipError_t run(Operands op, size_t slices, int split_len, hipStream_t stream) {
    int cus = 256;
    if (hipError_t e = device_cus(&cus); e != hipSuccess) return e;
    const bool split = S == Store::kTn && op.partials != nullptr;
    // A TN split's tile shape is the one gemm_tn_splits planned with.
    const Config c = pick_config(op.m, op.n, S == Store::kTn ? 1 : slices, cus,
                                 S == Store::kBiasGelu, L == Layout::kTN,
                                 S == Store::kBiasResidual);
    TileArgs ta{};
    ta.tiles_m = (op.m + c.bm - 1) / c.bm;
    ta.tiles_n = (op.n + c.bn - 1) / c.bn;
    ta.tiles_per_slice = ta.tiles_m * ta.tiles_n;
    ta.slices = int(slices);
    ta.group_m = 8;
    if (const char* e = tuning(Tune::kGemmGroupM)) ta.group_m = std::max(1, std::atoi(e));
    ta.split_len = split_len;
    // Persistent workgroups: as many as fit on the GPU at once (a multiple of
    // 8, so a workgroup keeps its XCD's share of the tiles), each walking ids
    // blockIdx.x, + gridDim.x, ...
    const size_t total = size_t(ta.tiles_per_slice) * slices;
    size_t slots = size_t(cus) * size_t(occupancy(c));
    if (const char* e = tuning(Tune::kGemmSlots)) slots = std::max(1, std::atoi(e));
    size_t gx = std::min(total, slots);
    if (gx >= 8) gx -= gx % 8;
    const dim3 grid(static_cast<unsigned>(gx), 1, 1);
    // The unchecked kernel needs whole tiles and whole k-steps in every slice.
    const int k_piece = split ? split_len : op.k;
    const bool exact = op.m % c.bm == 0 && op.n % c.bn == 0 && k_piece % c.bk == 0 &&
                       op.k % c.bk == 0;
    return exact ? dispatch<L, S, false>(c, grid, op, ta, stream)
                 : dispatch<L, S, true>(c, grid, op, ta, stream);
}

Operands make_ops(void* y, const void* x, const void* w, size_t m, size_t n, size_t k) {
    Operands op{};
    op.y = y;
    op.x = static_cast<const _Float16*>(x);
    op.w = static_cast<const _Float16*>(w);
    op.m = int(m);
    op.n = int(n);
    op.k = int(k);
    op.scale = 1.0f;
    return op;
}

// TN's split of k. The count is the smallest that keeps at least 3/4 of the
// CUs busy over all waves of tiles (or the fullest, up to 16 splits), each split
// at least 1,024 long and a multiple of 64; the last split takes the rest.
// (Policy follows ref src/kernels/gemm.cu:737-784, with CUs for slots.)
constexpr int kMinSplitK = 1024;
constexpr int kMaxSplits = 16;

}  // namespace

hipError_t gemm_tn_splits(size_t m, size_t n, size_t k, int* splits, int* split_len) {
    int cus = 256;
    if (hipError_t e = device_cus(&cus); e != hipSuccess) return e;
    const Config c = pick_config(m, n, 1, cus, false, true);
    const double tiles = double((m + c.bm - 1) / c.bm) * double((n + c.bn - 1) / c.bn);
    const int most = std::min<int>(kMaxSplits, std::max<int>(1, int(k / kMinSplitK)));
    int want = 1;
    double best = 0;
    for (int s = 1; s <= most; ++s) {
        const double blocks = tiles * s;
        const double waves = std::ceil(blocks / cus);
        const double fill = blocks / (waves * cus);
        if (fill > best) {
            best = fill;
            want = s;
        }
        if (fill >= 0.75) {
            want = s;
            break;
        }
    }
    const size_t per = (k + want - 1) / want;
    const size_t len = (per + 63) / 64 * 64;
    *split_len = int(len);
    *splits = int((k + len - 1) / len);
    return hipSuccess;
}

hipError_t gemm_tn_workspace(size_t m, size_t n, size_t k, size_t* bytes) {
    int splits = 1, len = 0;
    if (hipError_t e = gemm_tn_splits(m, n, k, &splits, &len); e != hipSuccess) return e;
    *bytes = splits > 1 ? size_t(splits) * m * n * sizeof(float) : 0;
    return hipSuccess;
}

hipError_t launch_gemm_nt(void* y, const void* x, const void* w, const void* bias, void* aux,
                          Epilogue e, size_t m, size_t n, size_t k, hipStream_t stream) {
    if (gemm_pipe_eligible(GemmLayout::kNT, e, m, n, k))
        return launch_gemm_pipe(GemmLayout::kNT, e, y, x, w, bias, aux, 1.0f, 1, m, n, k, false,
                                nullptr, 0, stream);
    Operands op = make_ops(y, x, w, m, n, k);
    op.bias = static_cast<const float*>(bias);
    op.aux = aux;
    switch (e) {
    case Epilogue::kNone: return run<Layout::kNT, Store::kNone>(op, 1, 0, stream);
    case Epilogue::kBias: return run<Layout::kNT, Store::kBias>(op, 1, 0, stream);
    case Epilogue::kBiasGelu: return run<Layout::kNT, Store::kBiasGelu>(op, 1, 0, stream);
    case Epilogue::kBiasResidual: return run<Layout::kNT, Store::kBiasResidual>(op, 1, 0, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm_nn(void* y, const void* x, const void* w, const void* aux, Epilogue e,
                          size_t m, size_t n, size_t k, hipStream_t stream) {
    if (gemm_pipe_eligible(GemmLayout::kNN, e, m, n, k))
        return launch_gemm_pipe(GemmLayout::kNN, e, y, x, w, nullptr, const_cast<void*>(aux), 1.0f,
                                1, m, n, k, false, nullptr, 0, stream);
    Operands op = make_ops(y, x, w, m, n, k);
    op.aux = const_cast<void*>(aux);
    switch (e) {
    case Epilogue::kNone: return run<Layout::kNN, Store::kNone>(op, 1, 0, stream);
    case Epilogue::kDGelu: return run<Layout::kNN, Store::kDGelu>(op, 1, 0, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm_tn_split(void* y, const void* x, const void* w, size_t m, size_t n,
                                size_t k, bool accumulate, void* workspace, int* splits_used,
                                hipStream_t stream) {
    int splits = 1, len = 0;
    if (hipError_t e = gemm_tn_splits(m, n, k, &splits, &len); e != hipSuccess) return e;
    Operands op = make_ops(y, x, w, m, n, k);
    op.accumulate = accumulate ? 1 : 0;
    op.partials = splits > 1 ? static_cast<float*>(workspace) : nullptr;
    hipError_t err;
    if (gemm_pipe_eligible(GemmLayout::kTN, kTnFloat, m, n, k)) {
        // The pipeline picks its own split count, at most the plan's.
        int used = 1;
        err = launch_gemm_pipe_tn(y, x, w, m, n, k, accumulate, op.partials, splits, &used, stream);
        splits = used;
    } else {
        err = run<Layout::kTN, Store::kTn>(op, size_t(splits), len, stream);
    }
    *splits_used = splits;
    return err;
}

hipError_t launch_tn_reduce(void* y, const void* partials, size_t m, size_t n, int splits,
                            bool accumulate, hipStream_t stream) {
    const size_t quads = m * n / 4;
    const unsigned blocks = unsigned(std::clamp<size_t>((quads + 255) / 256, 1, 8192));
    hipLaunchKernelGGL(tn_reduce, dim3(blocks), dim3(256), 0, stream, static_cast<float*>(y),
                       static_cast<const float*>(partials), quads, splits, accumulate ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_gemm_tn(void* y, const void* x, const void* w, size_t m, size_t n, size_t k,
                          bool accumulate, void* workspace, hipStream_t stream) {
    int splits = 1;
    if (hipError_t e = launch_gemm_tn_split(y, x, w, m, n, k, accumulate, workspace, &splits,
                                            stream);
        e != hipSuccess || splits == 1) {
        return e;
    }
    return launch_tn_reduce(y, workspace, m, n, splits, accumulate, stream);
}

hipError_t launch_gemm_nt_batched(void* y, const void* x, const void* w, size_t batches,
                                  size_t m, size_t n, size_t k, float scale, hipStream_t stream,
                                  bool causal) {
    if (gemm_pipe_eligible(GemmLayout::kNT, Epilogue::kScale, m, n, k))
        return launch_gemm_pipe(GemmLayout::kNT, Epilogue::kScale, y, x, w, nullptr, nullptr, scale,
                                batches, m, n, k, false, nullptr, 0, stream, causal && m == n);
    Operands op = make_ops(y, x, w, m, n, k);
    op.scale = scale;
    return run<Layout::kNT, Store::kScale>(op, batches, 0, stream);
}

bool gemm_batched_causal_taken(GemmLayout l, size_t m, size_t n, size_t k) {
    const Epilogue e = l == GemmLayout::kNT ? Epilogue::kScale : Epilogue::kNone;
    return gemm_pipe_eligible(l, e, m, n, k) && (l == GemmLayout::kNT ? m == n : m == k);
}

hipError_t launch_gemm_nn_batched(void* y, const void* x, const void* w, size_t batches,
                                  size_t m, size_t n, size_t k, hipStream_t stream, bool causal) {
    if (gemm_pipe_eligible(GemmLayout::kNN, Epilogue::kNone, m, n, k))
        return launch_gemm_pipe(GemmLayout::kNN, Epilogue::kNone, y, x, w, nullptr, nullptr, 1.0f,
                                batches, m, n, k, false, nullptr, 0, stream, causal && m == k);
    Operands op = make_ops(y, x, w, m, n, k);
    return run<Layout::kNN, Store::kNone>(op, batches, 0, stream);
}

hipError_t launch_gemm_nn_batched_views(void* y, const void* x, const void* w, size_t batches,
                                        size_t m, size_t n, size_t k, const HeadView& wv,
                                        const HeadView& yv, hipStream_t stream, bool causal) {
    if (!gemm_pipe_eligible(GemmLayout::kNN, Epilogue::kNone, m, n, k)) return hipErrorInvalidValue;
    return launch_gemm_pipe(GemmLayout::kNN, Epilogue::kNone, y, x, w, nullptr, nullptr, 1.0f,
                            batches, m, n, k, false, nullptr, 0, stream, causal && m == k, &wv,
                            &yv);
}

hipError_t launch_gemm_tn_batched_views(void* y, const void* x, const void* w, size_t batches,
                                        size_t m, size_t n, size_t k, const HeadView& wv,
                                        const HeadView& yv, hipStream_t stream, bool causal) {
    if (!gemm_pipe_eligible(GemmLayout::kTN, Epilogue::kNone, m, n, k)) return hipErrorInvalidValue;
    return launch_gemm_pipe(GemmLayout::kTN, Epilogue::kNone, y, x, w, nullptr, nullptr, 1.0f,
                            batches, m, n, k, false, nullptr, 0, stream, causal && m == k, &wv,
                            &yv);
}

hipError_t launch_gemm_tn_batched(void* y, const void* x, const void* w, size_t batches,
                                  size_t m, size_t n, size_t k, hipStream_t stream, bool causal) {
    if (gemm_pipe_eligible(GemmLayout::kTN, Epilogue::kNone, m, n, k))
        return launch_gemm_pipe(GemmLayout::kTN, Epilogue::kNone, y, x, w, nullptr, nullptr, 1.0f,
                                batches, m, n, k, false, nullptr, 0, stream, causal && m == k);
    Operands op = make_ops(y, x, w, m, n, k);
    return run<Layout::kTN, Store::kTnHalf>(op, batches, 0, stream);
}

}  // namespace flint
