// NT GEMM on gfx950 with one wave per SIMD and large wave tiles: the path for
// whole k-steps of 32 and rows of 16-byte multiples (n % 8 == 0, k % 32 == 0),
// which covers every NT shape of GPT-2 (forward linear layers, logits, and the
// batched QK^T). Other NT shapes, and the NN / TN layouts, run gemm.hip's
// kernels.
//
// Why this shape of kernel (measured on MI355X):
//  * A CU pulls about 110 GB/s (~45 B/clk) from L2 through the vector memory
//    path, with direct-to-LDS or register loads alike. Feeding 4,096 FLOP/clk
//    needs at least ~90 FLOP per loaded byte, i.e. a 256 x 192 (110 FLOP/B) or
//    256 x 256 (128 FLOP/B) macro-tile. A workgroup of 4 waves then holds
//    128 x 96 or 128 x 128 accumulators per wave (192 / 256 AGPRs), so one
//    wave runs per SIMD and overlap has to come from the instruction stream,
//    not from other waves.
//  * The k-loop takes k-steps of 32 through S = 4 LDS stages (256 x 256: 32 KB
//    a stage). The loads of step g + 3 are issued half during the first and
//    half during the second k16 sub-step of the steps before it, one
//    buffer_load ... lds after every second MFMA, and the fragment reads of the
//    next sub-step one after every MFMA: no burst of loads stalls the wave, and
//    three steps of latency are covered. One barrier per step sits between the
//    two sub-steps, after the last fragment read of the step.
//  * The epilogue stages the tile through LDS (the stages are free by then) so
//    that every global store instruction writes whole rows: 64 lanes x 16 B.
//    Stores straight from the MFMA layout cover 32 rows x 16 B each and ran the
//    output at under 2 TB/s; the staged form more than doubles that.
//  * Edge tiles need no separate path: each operand's buffer resource ends at
//    the last valid row, so loads past it read zeros (and a row of A or B only
//    ever meets its own output row or column), and the stores are masked.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>

#include "common/common.h"
#include "kernels/gemm_common.h"
#include "kernels/kernels.h"

namespace flint {
namespace {

constexpr int kPipeBK = 32;

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int cap63(int n) { return n < 63 ? n : 63; }

// s_waitcnt vmcnt(N) lgkmcnt(0) (expcnt at its maximum).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

// Key of the 64-byte LDS rows (4 chunks of 16 B): rows r and r + 4 differ, so
// the 16 lanes a ds_read_b128 serves per cycle (16 rows, one chunk) cover all
// four chunk positions four times and no 16-byte bank group twice in a row of 4.
__device__ __forceinline__ int pipe_key(int row) { return ((row >> 1) ^ (row >> 2)) & 3; }

// Per-wave C staging of the epilogue: a wave turns one 32-row block of its
// accumulators into [32][WTN + pad] elements (FP16, or FP32 for the residual
// epilogue; the pad moves consecutive rows by 16 bytes, 4 banks) and stores it
// back as whole 16-byte row chunks.
template <int BN, bool F32>
struct PipeStaging {
    static constexpr int kWtn = BN / 2;
    static constexpr int kElem = F32 ? 4 : 2;              // bytes per element
    static constexpr int kPerChunk = 16 / kElem;           // elements per 16-byte chunk
    static constexpr int kLdw = kWtn + kPerChunk;          // row stride (elements)
    static constexpr int kHalves = 32 * kLdw * kElem / 2;  // one wave's block, in halves
    static constexpr int kCpr = kWtn / kPerChunk;          // chunks per row
    static constexpr int kPerLane = 32 * kCpr / 64;        // chunks per lane per block
    static_assert(32 * kCpr % 64 == 0, "whole store instructions");
};

template <int BM, int BN, int S, Store ST>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_nt_pipe(Operands op, TileArgs ta) {
    // The host pass only needs a kernel to emit a launch stub for; the buffer
    // resource builtins below exist on the device side only.
#if defined(__HIP_DEVICE_COMPILE__)
    constexpr int BK = kPipeBK;
    constexpr int WTM = BM / 2, WTN = BN / 2;   // 2 x 2 waves
    constexpr int FM = WTM / 32, FN = WTN / 32;
    constexpr int IA = BM / 64, IB = BN / 64;   // loads (16 rows each) per thread per step
    constexpr int PER = IA + IB;
    constexpr int HALF = PER / 2;
    constexpr bool kBias =
        ST == Store::kBias || ST == Store::kBiasGelu || ST == Store::kBiasResidual;
    constexpr bool kF32 = ST == Store::kBiasResidual;   // y = residual + (sum + bias), FP32
    using C = PipeStaging<BN, kF32>;
    constexpr int kStageHalves = S * (BM + BN) * BK;
    constexpr int kCHalves = C::kHalves;   // one wave's staging block
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "whole 32 x 32 blocks per wave");
    static_assert((S - 2) * PER + PER < 64, "vmcnt range");
    static_assert(ST == Store::kNone || ST == Store::kBias || ST == Store::kBiasGelu ||
                      ST == Store::kScale || ST == Store::kBiasResidual, "NT epilogues");
    // One LDS object for everything: with a second one, the compiler's LDS-DMA
    // alias tracking put a vmcnt(0) in front of every fragment read.
    __shared__ __attribute__((aligned(16))) _Float16 lds[kStageHalves + 4 * kCHalves];
    auto stage = [&](int st) { return lds + st * (BM + BN) * BK; };
    // Epilogue: per 32-row block of a wave, C::kPerLane stores a lane per
    // output (GELU writes two).
    constexpr int kPasses = ST == Store::kBiasGelu ? 2 : 1;
    constexpr int kStores = FM * C::kPerLane * kPasses;   // buffer stores per wave per tile
    constexpr int kBiasLoads = kBias ? FN * 4 : 0;       // buffer loads per wave per tile

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int m = op.m, n = op.n, K = op.k;
    _Float16* const cst = lds + kStageHalves + wave * kCHalves;

    // This workgroup's tiles: ids blockIdx.x, + gridDim.x, ... (gridDim.x is a
    // multiple of 8 when there are 8 or more tiles, so they stay on one XCD).
    const unsigned total = unsigned(ta.tiles_per_slice) * unsigned(ta.slices);
    const int n_tiles = int((total - 1 - blockIdx.x) / gridDim.x) + 1;
    const int steps = K / BK;
    struct Tile {
        int m0, n0;
        size_t y_batch;
        const _Float16* a;
        const _Float16* b;
        unsigned a_bytes, b_bytes;
    };
    auto tile = [&](int i) {
        Tile t;
        int slice, tm, tn;
        map_tile(ta, blockIdx.x + unsigned(i) * gridDim.x, &slice, &tm, &tn);
        t.m0 = tm * BM;
        t.n0 = tn * BN;
        t.a = op.x;
        t.b = op.w;
        t.y_batch = 0;
        if (ta.slices > 1) {
            t.a += size_t(slice) * m * K;
            t.b += size_t(slice) * n * K;
            t.y_batch = size_t(slice) * m * n;
        }
        t.a += size_t(t.m0) * K;
        t.b += size_t(t.n0) * K;
        // Each operand's resource ends at its last valid row of the tile.
        t.a_bytes = unsigned(min(BM, m - t.m0)) * unsigned(K) * 2u;
        t.b_bytes = unsigned(min(BN, n - t.n0)) * unsigned(K) * 2u;
        return t;
    };

    // Load instruction q of a step: 16 rows x 64 bytes; lane l fills LDS row
    // l / 4 of the group, slot l % 4, with the global chunk the key puts there.
    const int lrow = lane >> 2;
    const unsigned lane_off = unsigned((lrow * K + ((lane & 3) ^ pipe_key(lrow)) * 8) * 2);
    unsigned voff[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        const int row0 = ((q < IA ? q : q - IA) * 4 + wave) * 16;
        voff[q] = lane_off + unsigned(row0 * K * 2);
    }
    // The issue side walks one stream of k-steps over all of the workgroup's
    // tiles, S steps ahead of the MFMAs; past the last one it reloads the last
    // step (into a stage nobody reads), so every wait counts the same loads.
    struct Issue {
        int tile, k0, st;
        __amdgpu_buffer_rsrc_t ra, rb;
    };
    auto rsrc_of = [&](Issue& is) {
        const Tile t = tile(is.tile);
        is.ra = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(t.a), 0, t.a_bytes, 0x00020000);
        is.rb = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(t.b), 0, t.b_bytes, 0x00020000);
    };
    auto advance = [&](Issue& is) {
        is.st = is.st + 1 == S ? 0 : is.st + 1;
        if (is.k0 + BK < K) {
            is.k0 += BK;
        } else if (is.tile + 1 < n_tiles) {
            is.k0 = 0;
            ++is.tile;
            rsrc_of(is);
        }
    };
    auto issue_q = [&](const Issue& is, int q) {
        const int row0 = ((q < IA ? q : q - IA) * 4 + wave) * 16;
        lds_half* dst = (lds_half*)(stage(is.st) + (q < IA ? 0 : BM * BK) + row0 * BK);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(q < IA ? is.ra : is.rb,
                                                 (__attribute__((address_space(3))) void*)dst, 16,
                                                 voff[q], unsigned(is.k0) * 2u, 0, 0);
    };

    f32x16 acc[FN][FM];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = f32x16{};

    const int fr = lane & 31, fc = lane >> 5;
    auto frag = [&](int row, int kk) { return row * BK + (((kk * 2 + fc) ^ pipe_key(row)) * 8); };
    // Fragment read idx (< FM: an x fragment, else a w fragment) of sub-step kk.
    auto read_one = [&](int st, int kk, int idx, f16x8 (&xf)[FM], f16x8 (&wf)[FN]) {
        const _Float16* s0 = stage(st);
        if (idx < FM) {
            xf[idx] = *reinterpret_cast<const f16x8*>(s0 + frag(wm * WTM + idx * 32 + fr, kk));
        } else {
            const int i = idx - FM;
            wf[i] = *reinterpret_cast<const f16x8*>(s0 + BM * BK + frag(wn * WTN + i * 32 + fr, kk));
        }
    };
    // The MFMAs of one k16 sub-step, with `between(q)` after MFMA q; the
    // scheduling fences keep this interleave exactly as written.
    auto mfmas = [&](f16x8 (&xf)[FM], f16x8 (&wf)[FN], auto&& between) {
#pragma unroll
        for (int q = 0; q < FM * FN; ++q) {
            const int i = q / FM, j = q % FM;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[i], xf[j], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            between(q);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Prologue: stream steps 0 .. S-2 and the first half of step S-1.
    Issue cur;
    cur.tile = 0;
    cur.k0 = 0;
    cur.st = 0;
    rsrc_of(cur);
#pragma unroll
    for (int j = 0; j < S - 1; ++j) {
#pragma unroll
        for (int q = 0; q < PER; ++q) issue_q(cur, q);
        advance(cur);
    }
#pragma unroll
    for (int q = 0; q < HALF; ++q) issue_q(cur, q);
    wait_vm_lgkm0<(S - 2) * PER + HALF>();
    block_sync();

    f16x8 xf[2][FM], wf[2][FN];
#pragma unroll
    for (int q = 0; q < FM + FN; ++q) read_one(0, 0, q, xf[0], wf[0]);
    int st = 0;
    // `cur` is the step whose second half goes out in the next sub-step 0.
    for (int i = 0; i < n_tiles; ++i) {
        const Tile t = tile(i);
        // Bias of this lane's columns, for the epilogue (48 or 64 VGPRs). Buffer
        // loads with the resource ending at n: columns past it read 0, and
        // every wave issues exactly FN * 4 of them (the waits below count them).
        f32x4 bias[kBias ? FN : 1][4];
        if constexpr (kBias) {
            const auto rbias = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(op.bias), 0, unsigned(n) * 4u, 0x00020000);
#pragma unroll
            for (int ii = 0; ii < FN; ++ii)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const int c = t.n0 + wn * WTN + ii * 32 + g4 * 8 + fc * 4;
                    bias[ii][g4] = __builtin_bit_cast(
                        f32x4, __builtin_amdgcn_raw_buffer_load_b128(rbias, unsigned(c) * 4u, 0, 0));
                }
        }
        for (int s = 0; s < steps; ++s) {
            Issue nxt = cur;
            advance(nxt);
            // Sub-step 0: reads of sub-step 1, second half of step `cur`.
            mfmas(xf[0], wf[0], [&](int q) {
                if (q < FM + FN) read_one(st, 1, q, xf[1], wf[1]);
                if ((q & 1) && HALF + q / 2 < PER) issue_q(cur, HALF + q / 2);
            });
            // The next step has landed once only the loads of the S - 2 steps
            // after it remain outstanding. For the first S - 2 steps of a tile
            // the previous tile's stores and this tile's bias loads went out
            // after the step as well (vmcnt retires in issue order), so they may
            // stay in flight too: the stores drain while the MFMAs run. After
            // the barrier nobody reads stage st any more.
            if (s <= S - 3) {
                if (i == 0) wait_vm_lgkm0<cap63((S - 2) * PER + kBiasLoads)>();
                else wait_vm_lgkm0<cap63((S - 2) * PER + kBiasLoads + kStores)>();
            } else {
                wait_vm_lgkm0<(S - 2) * PER>();
            }
            block_sync();
            const int st_next = st + 1 == S ? 0 : st + 1;
            // Sub-step 1: reads of the next step's sub-step 0, first half of `nxt`.
            mfmas(xf[1], wf[1], [&](int q) {
                if (q < FM + FN) read_one(st_next, 0, q, xf[0], wf[0]);
                if ((q & 1) && q / 2 < HALF) issue_q(nxt, q / 2);
            });
            st = st_next;
            cur = nxt;
        }

        // ---- epilogue: per 32-row block, registers -> this wave's staging
        // block -> whole 16-byte row chunks to HBM. Buffer stores: a chunk
        // outside the output gets an offset past the resource's end and is
        // dropped, so every wave issues exactly kStores of them. They drain
        // while the next tile's k-loop runs on its prefetched steps.
        const int row_base = t.m0 + wm * WTM;
        const int col_base = t.n0 + wn * WTN;
        const unsigned out_bytes = unsigned(m) * unsigned(n) * unsigned(C::kElem);
        // Byte offset of chunk q of this lane in 32-row block j (past the end
        // of the output when the chunk is outside it; n % 8 == 0 on this path,
        // so a chunk is whole once it starts).
        auto chunk_off = [&](int j, int q, int* r, int* cc) {
            const int c = q * 64 + lane;
            *r = c / C::kCpr;
            *cc = c % C::kCpr;
            const int gr = row_base + j * 32 + *r, gc = col_base + *cc * C::kPerChunk;
            return gr < m && gc < n ? (unsigned(gr) * unsigned(n) + unsigned(gc)) * unsigned(C::kElem)
                                    : 0xfffffff0u;
        };
#pragma unroll
        for (int j = 0; j < FM; ++j) {
            // Residual: this block's chunks are loaded first, so their latency
            // overlaps the staging writes.
            f32x4 res[kF32 ? C::kPerLane : 1];
            if constexpr (kF32) {
                const auto rres = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<float*>(static_cast<const float*>(op.aux) + t.y_batch), 0,
                    out_bytes, 0x00020000);
#pragma unroll
                for (int q = 0; q < C::kPerLane; ++q) {
                    int r, cc;
                    res[q] = __builtin_bit_cast(
                        f32x4, __builtin_amdgcn_raw_buffer_load_b128(rres, chunk_off(j, q, &r, &cc), 0, 0));
                }
            }
#pragma unroll
            for (int pass = 0; pass < kPasses; ++pass) {
                // GELU: pass 0 writes pre = RN16(s), pass 1 y = RN16(gelu(s)).
                const bool gelu_pass = ST == Store::kBiasGelu && pass == 1;
#pragma unroll
                for (int ii = 0; ii < FN; ++ii) {
#pragma unroll
                    for (int g4 = 0; g4 < 4; ++g4) {
                        f32x4 v = {acc[ii][j][g4 * 4 + 0], acc[ii][j][g4 * 4 + 1],
                                   acc[ii][j][g4 * 4 + 2], acc[ii][j][g4 * 4 + 3]};
                        if constexpr (kBias) v += bias[ii][g4];
                        if constexpr (ST == Store::kScale) v *= op.scale;
                        const int at = fr * C::kLdw + ii * 32 + g4 * 8 + fc * 4;
                        if constexpr (kF32) {
                            *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(cst) + at) = v;
                        } else {
                            if (gelu_pass) {
#pragma unroll
                                for (int e = 0; e < 4; ++e) v[e] = gelu(v[e]);
                            }
                            const f16x4 h = {_Float16(v[0]), _Float16(v[1]), _Float16(v[2]),
                                             _Float16(v[3])};
                            *reinterpret_cast<f16x4*>(cst + at) = h;
                        }
                    }
                }
                void* out = ST == Store::kBiasGelu && pass == 0 ? op.aux : op.y;
                out = static_cast<char*>(out) + t.y_batch * C::kElem;
                const auto rout = __builtin_amdgcn_make_buffer_rsrc(out, 0, out_bytes, 0x00020000);
#pragma unroll
                for (int q = 0; q < C::kPerLane; ++q) {
                    int r, cc;
                    const unsigned off = chunk_off(j, q, &r, &cc);
                    i32x4 v;
                    if constexpr (kF32) {
                        // y = residual + (sum + bias): one FP32 add, as the
                        // unstaged epilogue does it.
                        const f32x4 sb = *reinterpret_cast<const f32x4*>(
                            reinterpret_cast<const float*>(cst) + r * C::kLdw + cc * 4);
                        v = __builtin_bit_cast(i32x4, res[q] + sb);
                    } else {
                        v = __builtin_bit_cast(
                            i32x4, *reinterpret_cast<const f16x8*>(cst + r * C::kLdw + cc * 8));
                    }
                    __builtin_amdgcn_raw_buffer_store_b128(v, rout, off, 0, 0);
                }
            }
        }
#pragma unroll
        for (int ii = 0; ii < FN; ++ii)
#pragma unroll
            for (int j = 0; j < FM; ++j) acc[ii][j] = f32x16{};
    }
    // Outstanding loads (the tail's reloads) land before the workgroup's LDS
    // is released.
    wait_vmcnt<0>();
#endif
}

struct PipeConfig {
    int bm, bn, stages;
};

constexpr PipeConfig kPipeConfigs[] = {{256, 256, 3}, {256, 192, 4}, {128, 192, 4}};

// FLINT_GEMM_PIPE: "0" routes every NT call to gemm.hip's kernels;
// "bm,bn,stages" forces one of kPipeConfigs (tuning sweeps; read per call).
bool pipe_forced(PipeConfig* out, bool* disabled) {
    *disabled = false;
    const char* e = std::getenv("FLINT_GEMM_PIPE");
    if (e == nullptr) return false;
    if (e[0] == '0' && e[1] == '\0') {
        *disabled = true;
        return false;
    }
    PipeConfig c{};
    if (std::sscanf(e, "%d,%d,%d", &c.bm, &c.bn, &c.stages) != 3) return false;
    for (const PipeConfig& k : kPipeConfigs) {
        if (k.bm == c.bm && k.bn == c.bn && k.stages == c.stages) {
            *out = c;
            return true;
        }
    }
    return false;
}

// The macro-tile: whole waves of tiles over the CUs weigh most (a K = 768
// tile is short, so a partial last wave costs nearly a full one); among
// equal wave counts the larger tile needs fewer bytes per FLOP.
// LDS bytes of a configuration: its stages plus four per-wave staging blocks.
constexpr size_t pipe_lds_bytes(int bm, int bn, int stages, bool f32) {
    const int wtn = bn / 2, per_chunk = f32 ? 4 : 8;
    return size_t(stages) * (bm + bn) * kPipeBK * 2 + 4 * 32 * size_t(wtn + per_chunk) * (f32 ? 4 : 2);
}
constexpr size_t kPipeMaxLds = 160 * 1024;

PipeConfig pick_pipe(size_t m, size_t n, size_t slices, int cus, bool f32) {
    PipeConfig best = kPipeConfigs[0];
    double best_cost = 1e300;
    for (const PipeConfig& c : kPipeConfigs) {
        if (pipe_lds_bytes(c.bm, c.bn, c.stages, f32) > kPipeMaxLds) continue;
        const double tiles = double((m + c.bm - 1) / c.bm) * double((n + c.bn - 1) / c.bn) *
                             double(slices);
        const double rounds = std::ceil(tiles / cus);
        // Relative time of one tile: its area over its measured throughput per
        // unit area (256 x 256 as 1; the smaller tiles move more bytes per FLOP).
        const double eff = c.bm == 128 ? 0.80 : (c.bn == 256 ? 1.0 : 0.97);
        const double cost = rounds * double(c.bm) * double(c.bn) / eff;
        if (cost < best_cost * 0.999) {
            best_cost = cost;
            best = c;
        }
    }
    return best;
}

template <Store ST>
hipError_t launch_pipe(const PipeConfig& c, const Operands& op, size_t slices, int cus,
                       hipStream_t stream) {
    TileArgs ta{};
    ta.tiles_m = (op.m + c.bm - 1) / c.bm;
    ta.tiles_n = (op.n + c.bn - 1) / c.bn;
    ta.tiles_per_slice = ta.tiles_m * ta.tiles_n;
    ta.slices = int(slices);
    ta.group_m = 8;
    ta.split_len = 0;
    const size_t total = size_t(ta.tiles_per_slice) * slices;
    if (total == 0 || total > 0x7fffffffu) return hipErrorInvalidValue;
    // Persistent: one workgroup per CU (a multiple of 8, so each keeps its
    // XCD's share of the tiles), each walking ids blockIdx.x, + gridDim.x, ...
    size_t gx = std::min(total, size_t(cus));
    if (gx >= 8) gx -= gx % 8;
    const dim3 grid(unsigned(gx), 1, 1);
    constexpr bool kF32 = ST == Store::kBiasResidual;
#define FLINT_PIPE_CASE(BM_, BN_, S_)                                                         \
    if constexpr (pipe_lds_bytes(BM_, BN_, S_, kF32) <= kPipeMaxLds) {                        \
        if (c.bm == BM_ && c.bn == BN_ && c.stages == S_) {                                   \
            hipLaunchKernelGGL((gemm_nt_pipe<BM_, BN_, S_, ST>), grid, dim3(256), 0, stream, op, \
                               ta);                                                           \
            return hipGetLastError();                                                         \
        }                                                                                     \
    }
    FLINT_PIPE_CASE(256, 256, 3)
    FLINT_PIPE_CASE(256, 192, 4)
    FLINT_PIPE_CASE(128, 192, 4)
#undef FLINT_PIPE_CASE
    return hipErrorInvalidValue;
}

}  // namespace

bool gemm_nt_pipe_eligible(Epilogue e, size_t m, size_t n, size_t k) {
    bool disabled = false;
    PipeConfig forced;
    const bool force = pipe_forced(&forced, &disabled);
    if (disabled || m == 0 || n == 0 || n % 8 != 0 || k % kPipeBK != 0 || k < kPipeBK) return false;
    // The epilogue's buffer stores address one slice's output with 32-bit
    // offsets (FP32 for the residual epilogue).
    if (m * n * (e == Epilogue::kBiasResidual ? 4 : 2) >= (size_t{1} << 31)) return false;
    if (e != Epilogue::kNone && e != Epilogue::kBias && e != Epilogue::kBiasGelu &&
        e != Epilogue::kScale && e != Epilogue::kBiasResidual) {
        return false;
    }
    // The residual outputs of GPT-2 are 768 wide: 128-row tiles are needed to
    // fill the CUs there, and gemm.hip's 128 x 192 x 64 kernel with the
    // residual prefetched into registers measured as fast as this one's.
    return force || e != Epilogue::kBiasResidual || n >= 1024;
}

hipError_t launch_gemm_nt_pipe(void* y, const void* x, const void* w, const void* bias, void* aux,
                               Epilogue e, float scale, size_t slices, size_t m, size_t n,
                               size_t k, hipStream_t stream) {
    int cus = 256;
    if (hipError_t err = device_cus(&cus); err != hipSuccess) return err;
    Operands op{};
    op.y = y;
    op.x = static_cast<const _Float16*>(x);
    op.w = static_cast<const _Float16*>(w);
    op.bias = static_cast<const float*>(bias);
    op.aux = aux;
    op.scale = scale;
    op.m = int(m);
    op.n = int(n);
    op.k = int(k);
    PipeConfig c;
    bool disabled = false;
    const bool f32 = e == Epilogue::kBiasResidual;
    if (!pipe_forced(&c, &disabled) || pipe_lds_bytes(c.bm, c.bn, c.stages, f32) > kPipeMaxLds)
        c = pick_pipe(m, n, slices, cus, f32);
    switch (e) {
    case Epilogue::kNone: return launch_pipe<Store::kNone>(c, op, slices, cus, stream);
    case Epilogue::kBias: return launch_pipe<Store::kBias>(c, op, slices, cus, stream);
    case Epilogue::kBiasGelu: return launch_pipe<Store::kBiasGelu>(c, op, slices, cus, stream);
    case Epilogue::kScale: return launch_pipe<Store::kScale>(c, op, slices, cus, stream);
    case Epilogue::kBiasResidual:
        return launch_pipe<Store::kBiasResidual>(c, op, slices, cus, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace flint
