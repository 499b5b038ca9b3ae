// The GEMM pipeline on gfx950 with one wave per SIMD and large wave tiles,
// for all three layouts (NT, NN, TN, and their batched forms) whenever k is a
// multiple of 32 and the output rows are 16-byte multiples. Other shapes run
// gemm.hip's kernels.
//
// Why this shape of kernel (measured on MI355X):
//  * A CU's L2 -> LDS rate depends on the row piece one load covers: 64-byte
//    pieces of a row (k-steps of 32 FP16) stream at ~64 GB/s per CU, 128-byte
//    pieces (k-steps of 64) at ~124 GB/s. Row-major operands therefore take
//    k-steps of 64 wherever the tile's stages fit in LDS (k-major operands
//    are whole lines either way).
//  * Tiles of 128 x 192 to 256 x 256 load few bytes per FLOP; a workgroup of
//    4 waves then holds 64 x 96 to 128 x 128 accumulators per wave (96 to
//    256 AGPRs), so one wave runs per SIMD and overlap has to come from the
//    instruction stream, not from other waves.
//  * The k-loop takes k-steps of BK (32 or 64) through S LDS stages, each
//    step BK / 16 MFMA sub-steps. The loads of step g + S - 1 are spread over
//    the sub-steps of the steps before it, one buffer_load ... lds after every
//    second MFMA (every MFMA where a sub-step has few MFMAs), and the fragment
//    reads of the next sub-step one after every MFMA: no burst of loads stalls
//    the wave, and about S - 1 steps of latency are covered. One barrier per
//    step sits before its last sub-step, after the step's last fragment read
//    of its own stage. With two stages (256-row tiles at k-steps of 64) a
//    step's loads all go out right after the barrier that frees their stage.
//  * Operands whose rows run along k (NT's x and w, NN's x) sit in LDS as
//    [rows][BK k]. Operands stored k-major (NN's and TN's w, TN's x) are
//    loaded as they lie, [BK k][rows], and their MFMA fragments come from
//    ds_read_b64_tr_b16: within 16 lanes, lane j addresses 4 halves of row
//    k0 + j / 4 at column c0 + 4 (j % 4), and lane i receives column c0 + i of
//    rows k0 .. k0 + 3, so two such reads give a lane its 8 consecutive k.
//    Either way a load instruction fills 1 KB of LDS in one piece, and 16-byte
//    chunks are XOR-swizzled per row against bank conflicts.
//  * Workgroups are persistent and walk their tiles as one stream of k-steps,
//    so the next tile's first steps load under this tile's epilogue.
//  * The epilogue stages each wave's accumulators through LDS, 32 rows (FP16
//    outputs) or 16 rows (FP32 values) at a time (half that where the stages
//    leave too little LDS), so that every global store instruction writes
//    whole row pieces: 64 lanes x 16 B. Stores straight from the MFMA layout
//    cover 32 rows x 16 B each and ran the output at under 2 TB/s. They are
//    non-temporal buffer stores: a chunk outside the output gets an offset
//    past the resource's end and is dropped, so every wave issues the same
//    count, which the k-loop's waits rely on to let them drain under the next
//    tile.
//  * Edge tiles need no separate path: loads past an operand's end read zeros
//    (or, for a k-major operand's last columns, the next row's first values),
//    a row of either operand only ever meets its own output row or column, and
//    the stores are masked.
//  * Causal attention (the GPT-2 model's batched products): NT computes only
//    the output tiles at or below the diagonal; NN and TN cut each tile's
//    k-range to where the square operand can be nonzero.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <type_traits>

#include "common/common.h"
#include "common/tuning.h"
#include "kernels/gemm_common.h"
#include "kernels/kernels.h"

namespace flint {
namespace {

constexpr int kPipeBK = 32;

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

constexpr int cap63(int n) { return n < 63 ? n : 63; }

// The two 4-half results of a pair of ds_read_b64_tr_b16, k 0..3 and 4..7.
struct TrFrag {
    i32x2 lo, hi;
};
__device__ __forceinline__ f16x8 as_f16x8(const f16x8& v) { return v; }
__device__ __forceinline__ f16x8 as_f16x8(const TrFrag& f) {
    return __builtin_shufflevector(__builtin_bit_cast(f16x4, f.lo), __builtin_bit_cast(f16x4, f.hi), 0,
                                   1, 2, 3, 4, 5, 6, 7);
}

// Cache policy of the epilogue's stores: non-temporal (the nt bit). Outputs
// are written once and read by a later kernel, not by this one; marked as
// streaming they delay the next tiles' operand loads less (measured: logits
// 8192 x 50304 x 768 700 -> 645 us, MLP down 50 -> 46 us, training step -2.5%).
constexpr int kStoreAux = 2;

// s_waitcnt vmcnt(N) lgkmcnt(0) (expcnt at its maximum).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

// Key of the [rows][BK] layouts, XORed into a row's 16-byte chunk index. The
// 16 lanes a ds_read_b128 serves per cycle read one chunk of 16 consecutive
// rows, which must land on 16 distinct 16-byte bank groups (64 banks):
//  * BK = 32 (64-byte rows, 4 chunks): rows r, r + 4, r + 8, r + 12 share
//    bank groups before the XOR; ((row >> 1) ^ (row >> 2)) & 3 tells them apart.
//  * BK = 64 (128-byte rows, 8 chunks): the 8 even (odd) rows share 8 bank
//    groups; (row >> 1) & 7 gives each its own.
template <int BK>
__device__ __forceinline__ int row_key(int row) {
    if constexpr (BK == 32) return ((row >> 1) ^ (row >> 2)) & 3;
    else return (row >> 1) & 7;
}
// Key of the [32 k][rows] layout: rows k .. k + 3, which one transposing read
// of 16 lanes touches (2 chunks each), land on 8 distinct chunk positions of an
// aligned group of 8 (the XOR stays inside the group, hence inside the row).
__host__ __device__ constexpr int kmajor_key(int k) { return 2 * (k & 3); }

// Waves of a workgroup along n: 2 x 2 waves, or 4 x 1 for 64-wide tiles.
__host__ __device__ constexpr int pipe_waves_n(int bn) { return bn >= 128 ? 2 : 1; }

// What the epilogue stages per wave (WTN columns) and writes per 16-byte chunk.
// COMPACT halves the rows staged at a time, for tiles whose stages leave too
// little LDS for the full staging.
template <int WTN, Store ST, bool COMPACT = false>
struct PipeEpi {
    // FP32 values are staged when the output is FP32 (residual, TN) or when
    // the rounding needs a value that only the store pass reads (dGELU's pre).
    static constexpr bool kF32 =
        ST == Store::kBiasResidual || ST == Store::kTn || ST == Store::kDGelu;
    static constexpr int kOutElem = ST == Store::kBiasResidual || ST == Store::kTn ? 4 : 2;
    static constexpr int kWtn = WTN;
    // Values per chunk: a chunk is one 16-byte store (8 FP16 or 4 FP32
    // outputs); dGELU stages FP32 but stores FP16, 8 values a chunk.
    static constexpr int kPerChunk = kF32 && ST != Store::kDGelu ? 4 : 8;
    static constexpr int kRows = (kF32 ? 16 : 32) / (COMPACT ? 2 : 1);   // rows staged at a time
    static constexpr int kLdw = kWtn + kPerChunk;             // staged row stride (values)
    static constexpr int kHalves = kRows * kLdw * (kF32 ? 2 : 1);   // per wave, in halves
    static constexpr int kCpr = kWtn / kPerChunk;             // chunks per staged row
    static constexpr int kPerLane = kRows * kCpr / 64;        // chunks per lane per block
    static_assert(kRows * kCpr % 64 == 0, "whole store instructions");
    static constexpr int kPasses = ST == Store::kBiasGelu ? 2 : 1;
    static constexpr int kSubs = 32 / kRows;                  // staged blocks per 32 rows
};

constexpr size_t kPipeMaxLds = 160 * 1024;
constexpr bool is_bias_store(Store st) {
    return st == Store::kBias || st == Store::kBiasGelu || st == Store::kBiasResidual;
}
// Two-stage tiles with 64-deep steps read fragments two sub-steps ahead (four
// fragment buffers) where the accumulators and buffers fit in 320 registers;
// their bias then waits in LDS (1 KB per wave) instead of registers. nw is the
// workgroup's wave count: 4 (one wave per SIMD) or 8 (two).
__host__ __device__ constexpr bool pipe_look2(int bm, int bn, int s, int bk, int nw = 4) {
    const int wn = pipe_waves_n(bn);
    const int fm = bm / (nw / wn) / 32, fn = bn / wn / 32;
    return s == 2 && bk == 64 && fm * fn * 16 + 16 * (fm + fn) <= 320;
}
__host__ __device__ constexpr size_t pipe_bias_lds(int bm, int bn, int s, int bk, Store st,
                                                   int nw = 4) {
    return pipe_look2(bm, bn, s, bk, nw) && is_bias_store(st) ? 1024 * size_t(nw) : 0;
}
// Whether a configuration stages its epilogue compactly (see PipeEpi).
template <int BM, int BN, int S, int BK, Store ST, int NW = 4>
constexpr bool pipe_compact() {
    using E = PipeEpi<BN / pipe_waves_n(BN), ST>;
    return size_t(S) * (BM + BN) * BK * 2 + NW * size_t(E::kHalves) * 2 +
               pipe_bias_lds(BM, BN, S, BK, ST, NW) >
           kPipeMaxLds;
}
template <int BM, int BN, int S, int BK, Layout L, Store ST, int NW = 4>
constexpr size_t pipe_lds_bytes() {
    using E = PipeEpi<BN / pipe_waves_n(BN), ST, pipe_compact<BM, BN, S, BK, ST, NW>()>;
    return size_t(S) * (BM + BN) * BK * 2 + NW * size_t(E::kHalves) * 2 +
           pipe_bias_lds(BM, BN, S, BK, ST, NW);
}

// Tiles of one slice at or below the diagonal of a causal NT output: row
// block tm needs column blocks tn with tn * BN < (tm + 1) * BM.
__host__ __device__ inline int causal_row_tiles(int tm, int bm, int bn, int tiles_n) {
    const int c = ((tm + 1) * bm + bn - 1) / bn;
    return c < tiles_n ? c : tiles_n;
}

// map_tile for a causal NT output: the same XCD remap, then row block by row
// block through the tiles at or below the diagonal (tiles_m is small here:
// attention rows are at most a sequence).
__device__ inline void map_tile_causal(const TileArgs& t, unsigned id, int bm, int bn, int* slice,
                                       int* tm, int* tn) {
    const unsigned total = unsigned(t.tiles_per_slice) * unsigned(t.slices);
    if ((total & 7u) == 0) id = (id & 7u) * (total >> 3) + (id >> 3);
    *slice = int(id / unsigned(t.tiles_per_slice));
    int rest = int(id % unsigned(t.tiles_per_slice));
    int r = 0;
    for (; r + 1 < t.tiles_m; ++r) {
        const int c = causal_row_tiles(r, bm, bn, t.tiles_n);
        if (rest < c) break;
        rest -= c;
    }
    *tm = r;
    *tn = rest;
}

// NW MFMA waves per workgroup: 4 (one per SIMD) or 8 (two per SIMD, each
// wave half the rows of the 4-wave tile's): the same tile and LDS stages.
// LD adds four loader waves (one more per SIMD) that issue every operand load
// and join the k-step barriers, so that twice the waves issue the direct-to-
// LDS loads while the LDS fragment reads stay those of four MFMA waves.
// HV (batched NN / TN only): w and y are heads views (op.wv, op.yv), rows
// op.wv.ld / op.yv.ld apart. A template flag, so that the other instances
// keep their scalar registers: the runtime strides alone spilled SGPRs.
template <int BM, int BN, int S, int BK, Layout L, Store ST, int NW, bool LD = false,
          bool HV = false>
__global__ void __launch_bounds__((NW + (LD ? 4 : 0)) * 64)
__attribute__((amdgpu_waves_per_eu((NW + (LD ? 4 : 0)) / 4, (NW + (LD ? 4 : 0)) / 4)))
gemm_pipe(Operands op, TileArgs ta) {
    // The host pass only needs a kernel to emit a launch stub for; the buffer
    // resource builtins below exist on the device side only.
#if defined(__HIP_DEVICE_COMPILE__)
    static_assert(BK == 32 || BK == 64, "k-step");
    static_assert(kCausalZeroSpan % BM == 0 && kCausalZeroSpan % BK == 0,
                  "causal tiles must stay inside the softmax's zero span");
    constexpr int NS = BK / 16;                 // k16 sub-steps per k-step
    static_assert(NW == 4 || NW == 8, "waves per workgroup");
    static_assert(!LD || NW == 4, "loader waves serve four MFMA waves");
    static_assert(!HV || (L != Layout::kNT && (ST == Store::kNone || ST == Store::kTnHalf)),
                  "heads views: batched NN / TN, FP16 outputs");
    constexpr int WAVES_N = pipe_waves_n(BN);
    constexpr int WTM = BM / (NW / WAVES_N), WTN = BN / WAVES_N;
    constexpr int FM = WTM / 32, FN = WTN / 32;
    // The waves that issue the operand loads: the MFMA waves, or the loaders.
    constexpr int NLW = LD ? 4 : NW;
    // 1 KB loads per loading wave per step (each operand's stage is BM (BN)
    // rows of BK halves, 1 KB a load, spread over NLW waves).
    static_assert(BM * BK % (512 * NLW) == 0 && BN * BK % (512 * NLW) == 0, "whole loads per wave");
    constexpr int IA = BM * BK / (512 * NLW), IB = BN * BK / (512 * NLW);
    constexpr int PER = IA + IB;
    // A step's loads: POST of them in the sub-step after the barrier, the rest
    // PRE at a time in the NS - 1 sub-steps before the next one. With two
    // stages all of them go out after the barrier (the stage is free from
    // there on, and the step after is all the lead there is).
    static_assert(S >= 2 && (S > 2 || BK == 64), "stages");
    constexpr bool kAllPost = S == 2;
    constexpr int POST = kAllPost ? PER : PER / NS;
    constexpr int PRE = kAllPost ? 0 : (PER - POST + NS - 2) / (NS - 1);
    constexpr int kMaxLoads = POST > PRE ? POST : PRE;
    // A sub-step's loads go out after every second MFMA, or after every one
    // when the sub-step has too few MFMAs for that (64-wide tiles, two-stage
    // tiles); every load must get a slot, or the waits below would count
    // loads never issued. Two-stage tiles issue what has no slot right after
    // the sub-step's MFMAs.
    constexpr int kLoadEvery = FM * FN >= 2 * kMaxLoads ? 2 : 1;
    static_assert(kAllPost || FM * FN >= kMaxLoads * kLoadEvery, "a slot for every load");
    // x side (rows m, the MFMA's B operand) and w side (rows n, its A operand)
    // are k-major ([32 k][rows] in LDS) or row-major ([rows][32 k]).
    constexpr bool kXM = L == Layout::kTN;
    constexpr bool kWM = L != Layout::kNT;
    // A k-major fragment stays as the two halves its transposing reads wrote
    // until the MFMA that uses it (after the lgkmcnt wait): joining them
    // earlier could make the compiler copy registers the reads have not
    // filled yet, since it cannot see that asm results are still in flight.
    using XFrag = std::conditional_t<kXM, TrFrag, f16x8>;
    using WFrag = std::conditional_t<kWM, TrFrag, f16x8>;
    constexpr bool kBias =
        ST == Store::kBias || ST == Store::kBiasGelu || ST == Store::kBiasResidual;
    using E = PipeEpi<WTN, ST, pipe_compact<BM, BN, S, BK, ST, NW>()>;
    constexpr int kStageHalves = S * (BM + BN) * BK;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "whole 32 x 32 blocks per wave");
    static_assert(pipe_lds_bytes<BM, BN, S, BK, L, ST, NW>() <= kPipeMaxLds, "LDS");
    static_assert((S - 2) * PER + PER < 64, "vmcnt range");
    // Buffer stores per wave per tile, bias loads per wave per tile.
    constexpr int kStores = FM * E::kSubs * E::kPerLane * E::kPasses;
    constexpr bool kLook2 = pipe_look2(BM, BN, S, BK, NW);
    constexpr bool kBiasLds = kBias && kLook2;
    // Bias loads per wave per tile: FN * 4 into registers, or one 1 KB load
    // into the wave's LDS bias block.
    constexpr int kBiasLoads = kBiasLds ? 1 : (kBias ? FN * 4 : 0);
    // The residual is loaded into registers at tile start where it fits in
    // 128 VGPRs (128 x 192: 96), so that its latency hides under the k-loop.
    constexpr int kResAll = FM * E::kSubs * E::kPerLane;
    constexpr bool kResEarly =
        ST == Store::kBiasResidual && kResAll <= (NW == 4 && !LD ? 32 : 8);
    // dGELU's pre: the first staged block's chunks load at tile start, and
    // each later block's while the block before it is stored, so that no
    // block waits out a load's full latency.
    constexpr bool kPreEarly = ST == Store::kDGelu;
    constexpr int kEarlyLoads =
        kBiasLoads + (kResEarly ? kResAll : 0) + (kPreEarly ? E::kPerLane : 0);
    // One LDS object for everything: with a second one, the compiler's LDS-DMA
    // alias tracking put a vmcnt(0) in front of every fragment read.
    __shared__ __attribute__((aligned(16)))
    _Float16 lds[kStageHalves + NW * E::kHalves + pipe_bias_lds(BM, BN, S, BK, ST, NW) / 2];
    auto stage = [&](int st) { return lds + st * (BM + BN) * BK; };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool loader = LD && wave >= NW;
    // The wave's index among the waves that load (its loads' positions).
    const int lw = LD ? wave - NW : wave;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int m = op.m, n = op.n, K = op.k;
    const bool split = ST == Store::kTn && op.partials != nullptr;
    // Row strides: k-major operands' rows are the output's columns (w's are
    // op.wv.ld apart in a heads view); y's rows are n apart, or op.yv.ld.
    const int a_ld = kXM ? m : K;
    const int b_ld = kWM ? (HV ? op.wv.ld : n) : K;
    const int y_ld = HV ? op.yv.ld : n;
    _Float16* const cst = lds + kStageHalves + wave * E::kHalves;

    // This workgroup's tiles: ids blockIdx.x, + gridDim.x, ... (gridDim.x is a
    // multiple of 8 when there are 8 or more tiles, so they stay on one XCD).
    const unsigned total = unsigned(ta.tiles_per_slice) * unsigned(ta.slices);
    const int n_tiles = int((total - 1 - blockIdx.x) / gridDim.x) + 1;
    struct Tile {
        int m0, n0, k_begin, k_end, slice;
        size_t y_off;                 // output elements before this tile's slice
        const _Float16* a;            // x side: the tile's first row (k-contiguous) or column
        const _Float16* b;
        unsigned a_bytes, b_bytes;    // each operand's resource length
    };
    auto tile = [&](int i) {
        Tile t;
        int tm, tn;
        if (L == Layout::kNT && op.causal) {
            map_tile_causal(ta, blockIdx.x + unsigned(i) * gridDim.x, BM, BN, &t.slice, &tm, &tn);
        } else if (op.causal) {
            // Causal NN / TN: a tile's k-range grows (NN) or shrinks (TN) with
            // its row block. Tiles go out longest first, each round in the
            // reverse order of the one before, so a workgroup's long tile of
            // one round meets a short one in the next; no XCD remap (these
            // tiles share no operand worth keeping in L2).
            const unsigned total = unsigned(ta.tiles_per_slice) * unsigned(ta.slices);
            const unsigned first = unsigned(i) * gridDim.x;
            const unsigned in_round = min(gridDim.x, total - first);
            const unsigned rank =
                first + ((i & 1) ? in_round - 1 - blockIdx.x : unsigned(blockIdx.x));
            const unsigned per_row = unsigned(ta.slices) * unsigned(ta.tiles_n);
            const int d = int(rank / per_row);
            tm = L == Layout::kNN ? ta.tiles_m - 1 - d : d;
            const unsigned rem = rank % per_row;
            t.slice = int(rem / unsigned(ta.tiles_n));
            tn = int(rem % unsigned(ta.tiles_n));
        } else {
            map_tile(ta, blockIdx.x + unsigned(i) * gridDim.x, &t.slice, &tm, &tn);
        }
        t.m0 = tm * BM;
        t.n0 = tn * BN;
        t.k_begin = 0;
        t.k_end = K;
        // Causal NN / TN: x's row (NN) or column (TN) r is zero past r, so an
        // output row block [m0, m0 + BM) needs k < m0 + BM (NN: keys up to
        // the block's last query) or k >= m0 (TN: queries from the block's
        // first key on), in whole k-steps.
        if (L == Layout::kNN && op.causal) t.k_end = min(K, (t.m0 + BM + BK - 1) / BK * BK);
        if (L == Layout::kTN && op.causal) t.k_begin = t.m0 / BK * BK;
        t.y_off = 0;
        const _Float16* xs = op.x;
        const _Float16* ws = op.w;
        if (split) {
            t.k_begin = t.slice * ta.split_len;
            t.k_end = min(K, t.k_begin + ta.split_len);
            t.y_off = size_t(t.slice) * m * n;
        } else if (ta.slices > 1) {
            xs += size_t(t.slice) * m * K;
            ws += HV ? head_view_offset(op.wv, t.slice) : size_t(t.slice) * n * K;
            t.y_off = HV ? head_view_offset(op.yv, t.slice) : size_t(t.slice) * m * n;
        }
        // Row-major operands: the resource ends at the tile's last valid row.
        // k-major ones: at the end of the slice's matrix.
        if (kXM) {
            t.a = xs + t.m0;
            t.a_bytes = unsigned((size_t(K) * m - t.m0) * 2);
        } else {
            t.a = xs + size_t(t.m0) * K;
            t.a_bytes = unsigned(min(BM, m - t.m0)) * unsigned(K) * 2u;
        }
        if (kWM) {
            // Through the last row's last column (rows b_ld apart).
            t.b = ws + t.n0;
            t.b_bytes = HV ? unsigned((size_t(K - 1) * b_ld + n - t.n0) * 2)
                           : unsigned((size_t(K) * n - t.n0) * 2);
        } else {
            t.b = ws + size_t(t.n0) * K;
            t.b_bytes = unsigned(min(BN, n - t.n0)) * unsigned(K) * 2u;
        }
        return t;
    };

    // Instruction u = q * NLW + lw of an operand fills LDS bytes
    // [u KB, u KB + 1 KB) of its region; lane l writes bytes l * 16 .. + 16.
    // voff: the lane's byte offset in the global operand for k = 0 (the
    // k-step goes in the scalar offset).
    auto lane_voff = [&](int q, int rows, bool kmajor, int ld) {
        const int u = q * NLW + lw;
        if (kmajor) {
            const int p = u * 1024 + lane * 16;       // byte in the [32][rows] tile
            const int r = p / (rows * 2);             // k within the step
            const int pos = (p % (rows * 2)) / 16;    // chunk position in the row
            const int c = pos ^ kmajor_key(r);
            return unsigned((r * ld + c * 8) * 2);
        }
        constexpr int kCpr = BK / 8;              // 16-byte chunks per row
        const int row = u * (64 / kCpr) + lane / kCpr;
        return unsigned((row * ld + ((lane % kCpr) ^ row_key<BK>(row)) * 8) * 2);
    };
    unsigned voff[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q)
        voff[q] = q < IA ? lane_voff(q, BM, kXM, a_ld) : lane_voff(q - IA, BN, kWM, b_ld);

    // The issue side walks one stream of k-steps over all of the workgroup's
    // tiles, S steps ahead of the MFMAs; past the last one it reloads the last
    // step (into a stage nobody reads), so every wait counts the same loads.
    // A raw buffer's range check covers the vector offset, not the scalar one.
    // Row-major operands put the k-step in the scalar offset: it stays inside
    // the row, and the check on the row's vector offset masks rows past the
    // tile's last valid one. k-major operands instead get a resource based at
    // the step's first k row and ending at the operand's end, so that at the
    // last rows a chunk past the last column reads 0 rather than the memory
    // after the operand.
    struct Issue {
        int tile, k0, k_end, st;
        const _Float16 *a, *b;
        unsigned a_bytes, b_bytes;
        __amdgpu_buffer_rsrc_t ra, rb;
    };
    auto make_rsrcs = [&](Issue& is) {
        const unsigned ka = kXM ? unsigned(is.k0) * unsigned(a_ld) : 0u;
        const unsigned kb = kWM ? unsigned(is.k0) * unsigned(b_ld) : 0u;
        is.ra = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(is.a + ka), 0, is.a_bytes - 2u * ka,
                                                  0x00020000);
        is.rb = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(is.b + kb), 0, is.b_bytes - 2u * kb,
                                                  0x00020000);
    };
    auto rsrc_of = [&](Issue& is) {
        const Tile t = tile(is.tile);
        is.k0 = t.k_begin;
        is.k_end = t.k_end;
        is.a = t.a;
        is.b = t.b;
        is.a_bytes = t.a_bytes;
        is.b_bytes = t.b_bytes;
        make_rsrcs(is);
    };
    auto advance = [&](Issue& is) {
        is.st = is.st + 1 == S ? 0 : is.st + 1;
        if (is.k0 + BK < is.k_end) {
            is.k0 += BK;
            if constexpr (kXM || kWM) make_rsrcs(is);
        } else if (is.tile + 1 < n_tiles) {
            ++is.tile;
            rsrc_of(is);
        }
    };
    auto issue_q = [&](const Issue& is, int q) {
        if (LD && !loader) return;   // with loader waves, only they load operands
        const bool xq = q < IA;
        const int u = (xq ? q : q - IA) * NLW + lw;
        lds_half* dst = (lds_half*)(stage(is.st) + (xq ? 0 : BM * BK) + u * 512);
        // Row-major: k0 halves into every row. k-major: in the resource's base.
        const bool kmajor = xq ? kXM : kWM;
        const unsigned soff = kmajor ? 0u : unsigned(is.k0) * 2u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xq ? is.ra : is.rb,
                                                 (__attribute__((address_space(3))) void*)dst, 16,
                                                 voff[q], soff, 0, 0);
    };

    f32x16 acc[FN][FM];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = f32x16{};

    const int fr = lane & 31, fc = lane >> 5;
    // Fragment of operand rows r0 .. r0 + 31, k16 sub-step kk, from an LDS
    // region of `rows` rows: lane l gets row r0 + l % 32, k 8 (l / 32) .. + 8.
    auto frag_rowmajor = [&](const _Float16* region, int r0, int kk) {
        const int row = r0 + fr;
        return *reinterpret_cast<const f16x8*>(region + row * BK +
                                               (((kk * 2 + fc) ^ row_key<BK>(row)) * 8));
    };
    // Lane j of a 16-lane group addresses row k0 + j / 4, columns
    // c0 + 4 (j % 4) .. + 3; the read hands lane i column c0 + i of rows
    // k0 .. k0 + 3. k0 = 16 kk + 8 (l / 32) + 4 t, c0 = r0 + 16 ((l / 16) % 2).
    // The reads are inline asm: the compiler's LDS-DMA alias tracking put a
    // vmcnt(0) in front of every ds_read_b64_tr_b16 builtin (it cannot tell
    // them from the stage being loaded), which serialised the pipeline. The
    // asm results are unknown to its waitcnt pass, so the k-loop waits for
    // lgkmcnt(0) itself before the sub-step that uses them.
    auto frag_kmajor = [&](const _Float16* region, int rows, int r0, int kk) {
        const int j = lane & 15;
        const int col = r0 + 16 * ((lane >> 4) & 1) + 4 * (j & 3);
        const int key = kmajor_key(j >> 2);
        const int chunk = ((col >> 3) ^ key) * 8 + (col & 4);   // halves into the row
        const int k = kk * 16 + 8 * fc + (j >> 2);
        const unsigned a0 = unsigned(reinterpret_cast<uintptr_t>(
            (lds_half*)(region + k * rows + chunk)));
        TrFrag f;
        asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(f.lo) : "v"(a0));
        asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(f.hi) : "v"(a0), "i"(4 * rows * 2));
        return f;
    };
    // lgkmcnt(0) before a sub-step whose fragments include asm reads.
    auto wait_frags = [&]() {
        if constexpr (kXM || kWM) {
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // Fragment read idx (< FM: an x fragment, else a w fragment) of sub-step kk.
    auto read_one = [&](int st, int kk, int idx, XFrag (&xf)[FM], WFrag (&wf)[FN]) {
        const _Float16* s0 = stage(st);
        if (idx < FM) {
            const int r0 = wm * WTM + idx * 32;
            if constexpr (kXM) xf[idx] = frag_kmajor(s0, BM, r0, kk);
            else xf[idx] = frag_rowmajor(s0, r0, kk);
        } else {
            const int r0 = wn * WTN + (idx - FM) * 32;
            if constexpr (kWM) wf[idx - FM] = frag_kmajor(s0 + BM * BK, BN, r0, kk);
            else wf[idx - FM] = frag_rowmajor(s0 + BM * BK, r0, kk);
        }
    };
    // The MFMAs of one k16 sub-step, with `between(q)` after MFMA q; the
    // scheduling fences keep this interleave exactly as written.
    auto mfmas = [&](XFrag (&xf)[FM], WFrag (&wf)[FN], auto&& between) {
#pragma unroll
        for (int q = 0; q < FM * FN; ++q) {
            const int i = q / FM, j = q % FM;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_f16x8(wf[i]), as_f16x8(xf[j]),
                                                               acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            between(q);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Loader waves: the operand loads of every k-step, S steps ahead of the
    // MFMAs, and one barrier per k-step in step with the MFMA waves'. Before
    // the barrier of step g (which frees step g's stage) step g + 1 has
    // landed; right after it step g + S goes into that stage. Past the last
    // step the stream reloads the last step into stages nobody reads.
    if constexpr (LD) {
        if (loader) {
            Issue ld;
            ld.tile = 0;
            ld.st = 0;
            rsrc_of(ld);
#pragma unroll
            for (int j = 0; j < S; ++j) {
#pragma unroll
                for (int q = 0; q < PER; ++q) issue_q(ld, q);
                advance(ld);
            }
            wait_vmcnt<(S - 1) * PER>();
            block_sync();
            for (int i = 0; i < n_tiles; ++i) {
                const Tile t = tile(i);
                const int steps = (t.k_end - t.k_begin) / BK;
                for (int s = 0; s < steps; ++s) {
                    wait_vmcnt<(S - 2) * PER>();
                    block_sync();
#pragma unroll
                    for (int q = 0; q < PER; ++q) issue_q(ld, q);
                    advance(ld);
                }
            }
            wait_vmcnt<0>();
            return;
        }
    }

    // Prologue: stream steps 0 .. S-2 and the post-barrier share of step S-1.
    // (MFMA waves of a loader kernel issue none of these loads.)
    Issue cur;
    cur.tile = 0;
    cur.st = 0;
    rsrc_of(cur);
#pragma unroll
    for (int j = 0; j < S - 1; ++j) {
#pragma unroll
        for (int q = 0; q < PER; ++q) issue_q(cur, q);
        advance(cur);
    }
#pragma unroll
    for (int q = 0; q < POST; ++q) issue_q(cur, q);
    wait_vm_lgkm0<(S - 2) * PER + POST>();
    block_sync();

    // Fragment buffers: two (sub-step kk reads kk + 1) with three or more
    // stages; with two stages, four, indexed by sub-step: kk reads kk + 2, so
    // the step's stage is read out by the end of sub-step NS - 3 and the
    // barrier that frees it sits mid-step, leaving two sub-steps to issue the
    // next step's loads (all of them in one sub-step outran the vector memory
    // path: ~33 cycles per 1 KB load against 32 per MFMA).
    constexpr int NB = kLook2 ? 4 : 2;
    XFrag xf[NB][FM];
    WFrag wf[NB][FN];
#pragma unroll
    for (int q = 0; q < FM + FN; ++q) read_one(0, 0, q, xf[0], wf[0]);
    if constexpr (kLook2) {
#pragma unroll
        for (int q = 0; q < FM + FN; ++q) read_one(0, 1, q, xf[1], wf[1]);
    }
    int st = 0;
    // `cur` is the step whose remaining loads go out in the next sub-steps
    // 0 .. NS - 2.
    for (int i = 0; i < n_tiles; ++i) {
        const Tile t = tile(i);
        // Bias of this lane's columns, for the epilogue: buffer loads with the
        // resource ending at n (columns past it read 0), FN * 4 of them per wave.
        f32x4 bias[kBias ? FN : 1][4];
        float* const bias_lds = reinterpret_cast<float*>(lds + kStageHalves + NW * E::kHalves) +
                                wave * 256;
        if constexpr (kBiasLds) {
            // One load puts columns col0 .. col0 + 255 of the bias in this
            // wave's 1 KB block; the epilogue reads them back once the
            // k-loop's waits have retired it. The column goes in the lane's
            // vector offset, not the scalar one: a raw buffer's range check
            // covers the vector offset only, and it is what makes the lanes
            // past n read 0 instead of the memory after the bias.
            const auto rbias = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(op.bias), 0, unsigned(n) * 4u, 0x00020000);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rbias, (__attribute__((address_space(3))) void*)(lds_half*)bias_lds, 16,
                unsigned(t.n0 + wn * WTN) * 4u + unsigned(lane) * 16u, 0, 0, 0);
        } else if constexpr (kBias) {
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
        // The epilogue's chunk addressing: byte offset (elements of `elem`
        // bytes) of chunk q of this lane in the staged block (j, h), or past
        // the end when the chunk is outside the output (n % 8 == 0 here, so a
        // chunk is whole once it starts).
        const int row_base = t.m0 + wm * WTM;
        const int col_base = t.n0 + wn * WTN;
        const unsigned out_bytes = HV ? unsigned((size_t(m - 1) * y_ld + n) * E::kOutElem)
                                      : unsigned(size_t(m) * n * E::kOutElem);
        auto chunk_at = [&](int j, int h, int q, int elem, int* r, int* cc) {
            const int c = q * 64 + lane;
            *r = c / E::kCpr;
            *cc = c % E::kCpr;
            const int gr = row_base + j * 32 + h * E::kRows + *r;
            const int gc = col_base + *cc * E::kPerChunk;
            return gr < m && gc < n ? (unsigned(gr) * unsigned(y_ld) + unsigned(gc)) * unsigned(elem)
                                    : 0xfffffff0u;
        };
        f32x4 res_all[kResEarly ? FM : 1][kResEarly ? E::kSubs : 1][kResEarly ? E::kPerLane : 1];
        if constexpr (kResEarly) {
            const auto rs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(static_cast<const float*>(op.aux) + t.y_off), 0, out_bytes,
                0x00020000);
#pragma unroll
            for (int j = 0; j < FM; ++j)
#pragma unroll
                for (int h = 0; h < E::kSubs; ++h)
#pragma unroll
                    for (int q = 0; q < E::kPerLane; ++q) {
                        int r, cc;
                        res_all[j][h][q] = __builtin_bit_cast(
                            f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                       rs, chunk_at(j, h, q, 4, &r, &cc), 0, 0));
                    }
        }
        // Block (j, h)'s pre chunks, 8 FP16 each.
        auto load_pre = [&](int j, int h, f16x8 (&dst)[E::kPerLane]) {
            const auto rs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<void*>(static_cast<const void*>(
                    static_cast<const _Float16*>(op.aux) + t.y_off)),
                0, out_bytes, 0x00020000);
#pragma unroll
            for (int q = 0; q < E::kPerLane; ++q) {
                int r, cc;
                dst[q] = __builtin_bit_cast(
                    f16x8, __builtin_amdgcn_raw_buffer_load_b128(rs, chunk_at(j, h, q, 2, &r, &cc),
                                                                 0, 0));
            }
        };
        f16x8 pre_next[kPreEarly ? E::kPerLane : 1];
        if constexpr (kPreEarly) load_pre(0, 0, pre_next);
        const int steps = (t.k_end - t.k_begin) / BK;
        for (int s = 0; s < steps; ++s) {
            Issue nxt = cur;
            advance(nxt);
          if constexpr (kLook2) {
            static_assert(NS == 4, "two-stage tiles take 64-deep steps");
            static_assert(FM * FN >= FM + FN, "a slot for every fragment read");
            // Sub-steps 0 and 1: read sub-steps 2 and 3 of this step.
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                wait_frags();
                mfmas(xf[kk], wf[kk], [&](int q) {
                    if (q < FM + FN) read_one(st, kk + 2, q, xf[kk + 2], wf[kk + 2]);
                });
            }
            // Step s + 1 (loaded during the second half of the step before)
            // has landed; at a tile's first step the previous tile's stores
            // and this tile's bias (and residual) loads, issued after it, may
            // stay in flight. After the barrier stage st is free.
            if constexpr (!LD) {
                if (s == 0) {
                    if (i == 0) wait_vm_lgkm0<cap63(kEarlyLoads)>();
                    else wait_vm_lgkm0<cap63(kEarlyLoads + kStores)>();
                } else {
                    wait_vm_lgkm0<0>();
                }
            }
            block_sync();
            const int st_next = st + 1 == S ? 0 : st + 1;
            // Sub-steps 2 and 3: read sub-steps 0 and 1 of the next step, and
            // issue the loads of the step after it into stage st, half in each.
            constexpr int kHalf = (PER + 1) / 2;
#pragma unroll
            for (int kk = 2; kk < 4; ++kk) {
                wait_frags();
                mfmas(xf[kk], wf[kk], [&](int q) {
                    if (q < FM + FN) read_one(st_next, kk - 2, q, xf[kk - 2], wf[kk - 2]);
                    const int li = (kk - 2) * kHalf + q;
                    if (q < kHalf && li < PER) issue_q(nxt, li);
                });
                // Loads without a slot (fewer MFMAs than loads) go out here.
#pragma unroll
                for (int q = FM * FN; q < kHalf; ++q)
                    if ((kk - 2) * kHalf + q < PER) issue_q(nxt, (kk - 2) * kHalf + q);
            }
            st = st_next;
            cur = nxt;
          } else {
            // Sub-steps 0 .. NS - 2: reads of the sub-step after, the rest of
            // step `cur`'s loads.
#pragma unroll
            for (int kk = 0; kk < NS - 1; ++kk) {
                wait_frags();
                mfmas(xf[kk & 1], wf[kk & 1], [&](int q) {
                    if (q < FM + FN) read_one(st, kk + 1, q, xf[(kk + 1) & 1], wf[(kk + 1) & 1]);
                    const int li = POST + kk * PRE + q / kLoadEvery;
                    if (q % kLoadEvery == kLoadEvery - 1 && q / kLoadEvery < PRE && li < PER)
                        issue_q(cur, li);
                });
                // Fragments without an MFMA slot (a wave tile of one 32-row
                // block: fewer MFMAs than fragments per sub-step).
#pragma unroll
                for (int q = FM * FN; q < FM + FN; ++q)
                    read_one(st, kk + 1, q, xf[(kk + 1) & 1], wf[(kk + 1) & 1]);
            }
            // The next step has landed once only the loads of the S - 2 steps
            // after it remain outstanding. For the first S - 2 steps of a tile
            // (S - 1 with kAllPost, where no loads follow the stores before
            // the step after) the previous tile's stores and this tile's bias
            // (and residual) loads went out after the step as well (vmcnt
            // retires in issue order), so they may stay in flight too: the
            // stores drain while the MFMAs run. After the barrier nobody reads
            // stage st any more.
            if constexpr (!LD) {
                if (s <= S - (kAllPost ? 2 : 3)) {
                    if (i == 0) wait_vm_lgkm0<cap63((S - 2) * PER + kEarlyLoads)>();
                    else wait_vm_lgkm0<cap63((S - 2) * PER + kEarlyLoads + kStores)>();
                } else {
                    wait_vm_lgkm0<(S - 2) * PER>();
                }
            }
            block_sync();
            const int st_next = st + 1 == S ? 0 : st + 1;
            // Sub-step NS - 1: reads of the next step's sub-step 0, the first
            // POST loads of `nxt` (into stage st, free since the barrier).
            mfmas(xf[1], wf[1], [&](int q) {
                if (q < FM + FN) read_one(st_next, 0, q, xf[0], wf[0]);
                if (q % kLoadEvery == kLoadEvery - 1 && q / kLoadEvery < POST)
                    issue_q(nxt, q / kLoadEvery);
            });
#pragma unroll
            for (int q = FM * FN; q < FM + FN; ++q) read_one(st_next, 0, q, xf[0], wf[0]);
            if constexpr (kAllPost) {
#pragma unroll
                for (int q = FM * FN / kLoadEvery; q < POST; ++q) issue_q(nxt, q);
            }
            st = st_next;
            cur = nxt;
          }
        }

        // ---- epilogue: per staged block of a wave, registers -> staging ->
        // whole 16-byte row chunks to HBM.
        // The bias block's load (kBiasLds) retired at the second step's wait;
        // a one-step tile waits for it here. Its values are read where they
        // are added, so that they take no registers across the epilogue (the
        // next tile's first fragments are live there).
        if constexpr (kBiasLds) {
            // With loader waves nothing else of this wave's retires it first.
            if (LD || steps == 1) wait_vmcnt<0>();
        }
        auto bias_of = [&](int ii, int g4) {
            if constexpr (kBiasLds)
                return *reinterpret_cast<const f32x4*>(bias_lds + ii * 32 + g4 * 8 + fc * 4);
            else
                return bias[ii][g4];
        };
        const bool accumulate = ST == Store::kTn && !split && op.accumulate;
        // FP32 values the store pass reads back: the residual (where it was
        // not loaded at tile start) and the old y of an accumulating TN. Block
        // (j, h)'s go out while the block before it is stored; the first
        // block's at the epilogue's start. Every one of them is used within
        // this epilogue, so the k-loop's wait counts do not see them.
        constexpr bool kReadsAhead =
            (ST == Store::kBiasResidual && !kResEarly) || ST == Store::kTn;
        auto load_rd = [&](int j, int h, f32x4 (&dst)[E::kPerLane]) {
            const float* src = ST == Store::kTn ? static_cast<const float*>(op.y)
                                                : static_cast<const float*>(op.aux);
            const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(src + t.y_off),
                                                              0, out_bytes, 0x00020000);
#pragma unroll
            for (int q = 0; q < E::kPerLane; ++q) {
                int r, cc;
                if (ST == Store::kTn && !accumulate) {
                    dst[q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                } else {
                    dst[q] = __builtin_bit_cast(
                        f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                   rs, chunk_at(j, h, q, 4, &r, &cc), 0, 0));
                }
            }
        };
        f32x4 rd_next[kReadsAhead ? E::kPerLane : 1];
        if constexpr (kReadsAhead) load_rd(0, 0, rd_next);
#pragma unroll
        for (int j = 0; j < FM; ++j) {
#pragma unroll
            for (int h = 0; h < E::kSubs; ++h) {
                constexpr bool kReads = ST == Store::kBiasResidual || ST == Store::kTn;
                f32x4 rd[kReads ? E::kPerLane : 1];
                if constexpr (kResEarly) {
#pragma unroll
                    for (int q = 0; q < E::kPerLane; ++q) rd[q] = res_all[j][h][q];
                } else if constexpr (kReadsAhead) {
#pragma unroll
                    for (int q = 0; q < E::kPerLane; ++q) rd[q] = rd_next[q];
                    const int nb = j * E::kSubs + h + 1;
                    if (nb < FM * E::kSubs) load_rd(nb / E::kSubs, nb % E::kSubs, rd_next);
                }
                f16x8 pre8[ST == Store::kDGelu ? E::kPerLane : 1];
                if constexpr (ST == Store::kDGelu) {
#pragma unroll
                    for (int q = 0; q < E::kPerLane; ++q) pre8[q] = pre_next[q];
                    const int nb = j * E::kSubs + h + 1;
                    if (nb < FM * E::kSubs) load_pre(nb / E::kSubs, nb % E::kSubs, pre_next);
                }
                f16x4 ykeep[ST == Store::kBiasGelu ? FN : 1][4];
#pragma unroll
                for (int pass = 0; pass < E::kPasses; ++pass) {
                    // GELU: pass 0 writes pre = RN16(s), pass 1 y = RN16(gelu(s)).
                    const bool gelu_pass = ST == Store::kBiasGelu && pass == 1;
                    // The lanes holding the block's rows (each lane holds one row).
                    const bool mine = E::kRows == 32 || fr / E::kRows == h;
                    if (mine) {
                        const int srow = fr % E::kRows;
#pragma unroll
                        for (int ii = 0; ii < FN; ++ii) {
#pragma unroll
                            for (int g4 = 0; g4 < 4; ++g4) {
                                const int at = srow * E::kLdw + ii * 32 + g4 * 8 + fc * 4;
                                if (gelu_pass) {
                                    // Formed with pre in pass 0.
                                    *reinterpret_cast<f16x4*>(cst + at) = ykeep[ii][g4];
                                    continue;
                                }
                                f32x4 v = {acc[ii][j][g4 * 4 + 0], acc[ii][j][g4 * 4 + 1],
                                           acc[ii][j][g4 * 4 + 2], acc[ii][j][g4 * 4 + 3]};
                                if constexpr (kBias) v += bias_of(ii, g4);
                                if constexpr (ST == Store::kScale) v *= op.scale;
                                if constexpr (E::kF32) {
                                    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(cst) + at) = v;
                                } else {
                                    if constexpr (ST == Store::kBiasGelu) {
                                        // y = RN16(gelu(v)) from the same biased sum, kept in
                                        // registers for pass 1 (the accumulator is read and
                                        // biased once).
                                        ykeep[ii][g4] = f16x4{_Float16(gelu(v[0])), _Float16(gelu(v[1])),
                                                              _Float16(gelu(v[2])), _Float16(gelu(v[3]))};
                                    }
                                    const f16x4 hv = {_Float16(v[0]), _Float16(v[1]),
                                                      _Float16(v[2]), _Float16(v[3])};
                                    *reinterpret_cast<f16x4*>(cst + at) = hv;
                                }
                            }
                        }
                    }
                    // Other lanes read what these lanes wrote: keep the reads
                    // below (out of the branch). The compiler moved them into
                    // it once, for the lanes that wrote only.
                    __builtin_amdgcn_wave_barrier();
                    asm volatile("" ::: "memory");
                    void* out = ST == Store::kBiasGelu && pass == 0 ? op.aux : op.y;
                    if (split) out = op.partials;
                    out = static_cast<char*>(out) + t.y_off * E::kOutElem;
                    const auto rout = __builtin_amdgcn_make_buffer_rsrc(out, 0, out_bytes,
                                                                        0x00020000);
#pragma unroll
                    for (int q = 0; q < E::kPerLane; ++q) {
                        int r, cc;
                        if constexpr (ST == Store::kDGelu) {
                            // y = RN16(sum * GELU'(pre)), 8 outputs = 16 bytes.
                            const unsigned off = chunk_at(j, h, q, 2, &r, &cc);
                            const float* sp = reinterpret_cast<const float*>(cst) + r * E::kLdw + cc * 8;
                            const f32x4 s0 = *reinterpret_cast<const f32x4*>(sp);
                            const f32x4 s1 = *reinterpret_cast<const f32x4*>(sp + 4);
                            f16x8 o;
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                o[e] = _Float16(s0[e] * gelu_grad(float(pre8[q][e])));
                                o[e + 4] = _Float16(s1[e] * gelu_grad(float(pre8[q][e + 4])));
                            }
                            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, o), rout,
                                                                   off, 0, kStoreAux);
                        } else if constexpr (E::kF32) {
                            // Residual: y = residual + (sum + bias). TN: y = sum,
                            // y = old + sum, or a split's partial.
                            const unsigned off = chunk_at(j, h, q, 4, &r, &cc);
                            const f32x4 sv = *reinterpret_cast<const f32x4*>(
                                reinterpret_cast<const float*>(cst) + r * E::kLdw + cc * 4);
                            f32x4 o = sv;
                            if (ST == Store::kBiasResidual || accumulate) o = rd[q] + sv;
                            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, o), rout,
                                                                   off, 0, kStoreAux);
                        } else {
                            const unsigned off = chunk_at(j, h, q, 2, &r, &cc);
                            const f16x8 v = *reinterpret_cast<const f16x8*>(cst + r * E::kLdw + cc * 8);
                            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), rout,
                                                                   off, 0, kStoreAux);
                        }
                    }
                    // The next block's writes go after these reads.
                    __builtin_amdgcn_wave_barrier();
                    asm volatile("" ::: "memory");
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
    int bm, bn, stages, bk;
    int waves = 4;         // MFMA waves: 4, or 8 (two per SIMD; NT layouts only)
    int loaders = 0;       // 1: four more waves issue the operand loads

    bool same(const PipeConfig& o) const {
        return bm == o.bm && bn == o.bn && stages == o.stages && bk == o.bk &&
               waves == o.waves && loaders == o.loaders;
    }
};

constexpr PipeConfig kPipeConfigs[] = {
    {256, 256, 3, 32}, {256, 192, 4, 32}, {128, 192, 4, 32}, {256, 64, 4, 32},
    {128, 192, 3, 64}, {256, 128, 3, 64}, {256, 256, 2, 64}, {256, 192, 2, 64},
    {256, 192, 2, 64, 8}, {128, 192, 3, 64, 4, 1}, {256, 128, 3, 64, 4, 1}, {128, 64, 4, 32},
    {128, 64, 3, 64}, {256, 64, 3, 64}};

// The "gemm_pipe" override: "0" routes every call to gemm.hip's kernels;
// "bm,bn,stages[,bk[,waves[,loaders]]]" forces one of kPipeConfigs (tests and
// tuning sweeps; bk defaults to 32, waves to 4, loaders to 0).
bool pipe_forced(PipeConfig* out, bool* disabled) {
    *disabled = false;
    const char* e = tuning(Tune::kGemmPipe);
    if (e == nullptr) return false;
    if (e[0] == '0' && e[1] == '\0') {
        *disabled = true;
        return false;
    }
    PipeConfig c{};
    c.bk = 32;
    c.waves = 4;
    c.loaders = 0;
    const int got = std::sscanf(e, "%d,%d,%d,%d,%d,%d", &c.bm, &c.bn, &c.stages, &c.bk, &c.waves,
                                &c.loaders);
    if (got < 3) return false;
    for (const PipeConfig& k : kPipeConfigs) {
        if (k.same(c)) {
            *out = c;
            return true;
        }
    }
    return false;
}

// LDS bytes of a configuration at run time (the kernel's own static_assert
// checks the same sum).
size_t lds_bytes(const PipeConfig& c, Store st) {
    const bool f32 = st == Store::kBiasResidual || st == Store::kTn || st == Store::kDGelu;
    const int wtn = c.bn / pipe_waves_n(c.bn), per = f32 && st != Store::kDGelu ? 4 : 8,
              rows = f32 ? 16 : 32;
    const size_t stages = size_t(c.stages) * (c.bm + c.bn) * c.bk * 2 +
                          pipe_bias_lds(c.bm, c.bn, c.stages, c.bk, st, c.waves);
    const size_t staging = size_t(c.waves) * rows * (wtn + per) * (f32 ? 4 : 2);
    return stages + staging <= kPipeMaxLds ? stages + staging : stages + staging / 2;
}

// Whether a configuration can run an epilogue over k: it fits in LDS and k is
// whole k-steps; the 8-wave configuration serves the NT layout only.
bool usable(const PipeConfig& c, Store st, size_t k, Layout l) {
    return lds_bytes(c, st) <= kPipeMaxLds && k % size_t(c.bk) == 0 &&
           (c.waves == 4 || l == Layout::kNT);
}

// Relative throughput per unit of tile area, measured on the GPT-2 shapes at
// many tiles per CU (256 x 256 x 32 as 1). Larger tiles load fewer bytes per
// FLOP; 64-deep k-steps load whole 128-byte lines of row-major operands, which
// the vector memory path delivers at twice the rate of 64-byte pieces.
// (256 x 64: 51 FLOP per loaded byte, worth it only where n <= 64.) TN's
// operands are k-major, whole lines at either depth; there the 64-deep steps
// gain from half the barriers, most in 128 x 192 tiles.
double pipe_eff(const PipeConfig& c, Store st, Layout l) {
    // Loader waves pay where the MFMA waves' own stream is the bottleneck:
    // TN, whose fragments come from transposing LDS reads with a full LDS
    // wait per sub-step (3072 x 768 x 8192: 64.2 -> 55.2 us, 768 x 3072: 60.2
    // -> 55.1, 2304 x 768: 46.0 -> 43.6, same process; the logits dW 50304 x
    // 768 x 8192: 744 -> 671 us at 256 x 128), and NT + bias at 128 x 192
    // (the bias epilogue's stores retire on the MFMA waves' counter, apart
    // from the loads: qkv 8192 x 2304 x 768 34.0 -> 31.6 us, 8192 x 768 x 768
    // 13.8 -> 13.0, 8192 x 3072 x 768 43.1 -> 40.9, 8192 x 768 x 3072 37.9 ->
    // 36.1, same process), and plain NT (8192 x 3072 x 768 43.7 -> 42.1 us,
    // 8192 x 768 x 3072 38.3 -> 36.9; the logits 8192 x 50304 x 768 636.0 ->
    // 617.6 at 256 x 128, which pick_pipe admits only for outputs that
    // large). Other NT and NN epilogues ran as fast or slower (MLP down +
    // residual 43.8 -> 52.3 us: its residual no longer loads at tile start;
    // MLP up + GELU 54.7 -> 55.0; NN 8192 x 768 x 3072 38.2 -> 43.8), so
    // there they are taken only when forced.
    if (c.loaders) {
        if (st == Store::kTn || st == Store::kTnHalf) return 1.0;
        if (st == Store::kBias && c.bm == 128) return 1.1;
        if (st == Store::kNone && l == Layout::kNT) return c.bm == 128 ? 1.1 : 1.15;
        return 0.01;
    }
    // The 8-wave tile: same bits as the 4-wave 256 x 192 x 2 x 64; faster only
    // for plain NT products of many tile rounds (logits 8192 x 50304 x 768:
    // 632.6 -> 608.0 us, same process, five rounds); slower at two rounds with
    // an epilogue (MLP up + GELU 53.9 -> 58.1 us). pick_pipe admits it only
    // for plain NT products of at least kPipe8MinRounds rounds.
    if (c.waves == 8) return 1.04;
    // 64 wide: 64-deep steps, whole 128-byte lines a load (the causal
    // attention products' 128 x 64 tiles: the default model's training step
    // 13.36 -> 13.07 ms; the full batched NN 96 x 1024 x 64 x 1024 at 256 x
    // 64: 53.1 -> 41.9 us, TN the same; same process, the same bits).
    if (c.bn == 64) return c.bk == 64 ? 0.56 : 0.55;
    // Two stages: worth it for 256 x 192 outside TN (MLP up 59 -> 56 us,
    // dGELU 77 -> 74 us); 256 x 256 measured no better than at 32-deep steps.
    if (c.stages == 2)
        return c.bn == 192 && st != Store::kTn && st != Store::kTnHalf ? 1.0 : 0.5;
    if (st == Store::kTn || st == Store::kTnHalf) {
        if (c.bk == 64) return c.bm == 128 ? 0.86 : 0.80;
    } else if (c.bk == 64) {
        return c.bm == 128 ? 0.84 : 0.94;
    }
    return c.bm == 128 ? 0.80 : (c.bn == 256 ? 1.0 : 0.97);
}

// The macro-tile: whole waves of tiles over the CUs weigh most (a K = 768
// tile is short, so a partial last wave costs nearly a full one); among equal
// wave counts the larger tile needs fewer bytes per FLOP.
constexpr double kPipe8MinRounds = 8.0;

PipeConfig pick_pipe(size_t m, size_t n, size_t k, size_t slices, int cus, Store st, Layout l,
                     bool causal = false) {
    PipeConfig best = kPipeConfigs[0];
    double best_cost = 1e300;
    for (const PipeConfig& c : kPipeConfigs) {
        if (!usable(c, st, k, l)) continue;
        // 64-wide tiles only for outputs that narrow: elsewhere a round of
        // them costs as much as one of the wider tiles and loads far more.
        if (c.bn == 64 && n > 64) continue;
        // 128 x 64 only for the causal attention products, whose tiles' work
        // grows with their row block: three rounds of the shorter tiles
        // balance better than one and a half of 256 x 64 (the default GPT-2
        // model's step 13.78 -> 13.60 ms, same process, the same bits). On
        // full products 256 x 64 is faster (96 x 1024 x 64 x 1024 NN: 41.8
        // against 44.8 us).
        if (c.bm == 128 && c.bn == 64 && !causal) continue;
        const double tiles = double((m + c.bm - 1) / c.bm) * double((n + c.bn - 1) / c.bn) *
                             double(slices);
        const double rounds = std::ceil(tiles / cus);
        if (c.waves == 8 && (st != Store::kNone || rounds < kPipe8MinRounds)) continue;
        // The 256 x 128 loader tile: plain NT only on the logits' size of
        // output (8192 x 3072 x 768: 42.7 against 42.1 us for 128 x 192).
        if (c.loaders && c.bm == 256 && l != Layout::kTN && double(m) * double(n) < 1e8)
            continue;
        const double cost = rounds * double(c.bm) * double(c.bn) / pipe_eff(c, st, l);
        if (cost < best_cost * 0.999) {
            best_cost = cost;
            best = c;
        }
    }
    return best;
}

// TN's tile and split count together. The ABI plan (gemm_tn_splits, which the
// workspace size follows) caps the split count; any count up to it fits the
// caller's workspace. Cost: rounds of (tile, split) units over the CUs times a
// unit's work, plus the partials' reduce pass when there is more than one
// split ((splits + 1 or 2) * m * n * 4 bytes at ~5 TB/s, and a launch).
// `only`, when given, is the one configuration considered.
void plan_tn(size_t m, size_t n, size_t k, int max_splits, int cus, bool accumulate,
             const PipeConfig* only, PipeConfig* best_c, int* best_s) {
    const Store st = Store::kTn;
    double best = 1e300;
    *best_c = only != nullptr ? *only : pick_pipe(m, n, k, 1, cus, st, Layout::kTN);
    *best_s = 1;
    for (const PipeConfig& c : kPipeConfigs) {
        if (!usable(c, st, k, Layout::kTN)) continue;
        if (only != nullptr && !c.same(*only)) continue;
        if (only == nullptr && c.bn == 64 && (n > 64 || c.bm == 128)) continue;
        // The 256 x 128 loader tile won only on the logits' size of output.
        if (only == nullptr && c.loaders && c.bm == 256 && double(m) * double(n) < 8e6) continue;
        const double eff = pipe_eff(c, st, Layout::kTN);
        const double tiles = double((m + c.bm - 1) / c.bm) * double((n + c.bn - 1) / c.bn);
        for (int sp = 1; sp <= max_splits; ++sp) {
            const size_t len = (k + sp - 1) / sp;
            const size_t len32 = (len + c.bk - 1) / c.bk * c.bk;
            if (size_t(sp - 1) * len32 >= k) continue;   // the last split would be empty
            const double rounds = std::ceil(tiles * sp / cus);
            // One 256 x 256 x 32 step of a unit is ~0.5 us at the pipeline's rate.
            const double t_compute = rounds * double(c.bm) * double(c.bn) * double(len32) /
                                     (256.0 * 256.0 * 32.0) * 0.5e-6 / eff;
            const double t_reduce = sp > 1 ? double(sp + 1 + (accumulate ? 1 : 0)) * double(m) *
                                                 double(n) * 4.0 / 5e12 + 3e-6
                                           : 0.0;
            const double t = t_compute + t_reduce;
            if (t < best * 0.999) {
                best = t;
                *best_c = c;
                *best_s = sp;
            }
        }
    }
}

template <Layout L, Store ST>
hipError_t launch_pipe(const PipeConfig& c, const Operands& op, size_t slices, int split_len,
                       int cus, hipStream_t stream) {
    constexpr bool kViews = L != Layout::kNT && (ST == Store::kNone || ST == Store::kTnHalf);
    const bool hv = op.wv.heads != 0;
    TileArgs ta{};
    ta.tiles_m = (op.m + c.bm - 1) / c.bm;
    ta.tiles_n = (op.n + c.bn - 1) / c.bn;
    ta.tiles_per_slice = ta.tiles_m * ta.tiles_n;
    if (L == Layout::kNT && op.causal) {
        ta.tiles_per_slice = 0;
        for (int r = 0; r < ta.tiles_m; ++r)
            ta.tiles_per_slice += causal_row_tiles(r, c.bm, c.bn, ta.tiles_n);
    }
    ta.slices = int(slices);
    ta.group_m = 8;
    ta.split_len = split_len;
    const size_t total = size_t(ta.tiles_per_slice) * slices;
    if (total == 0 || total > 0x7fffffffu) return hipErrorInvalidValue;
    // Persistent: one workgroup per CU (a multiple of 8, so each keeps its
    // XCD's share of the tiles), each walking ids blockIdx.x, + gridDim.x, ...
    size_t gx = std::min(total, size_t(cus));
    if (gx >= 8) gx -= gx % 8;
    const dim3 grid(unsigned(gx), 1, 1);
#define FLINT_PIPE_CASE(BM_, BN_, S_, BK_, NW_, LD_)                                           \
    if constexpr (pipe_lds_bytes<BM_, BN_, S_, BK_, L, ST, NW_>() <= kPipeMaxLds) {            \
        if (c.same(PipeConfig{BM_, BN_, S_, BK_, NW_, LD_})) {                                 \
            if constexpr (kViews) {                                                            \
                if (hv) {                                                                      \
                    hipLaunchKernelGGL((gemm_pipe<BM_, BN_, S_, BK_, L, ST, NW_, LD_ != 0,     \
                                                  true>),                                      \
                                       grid, dim3((NW_ + 4 * LD_) * 64), 0, stream, op, ta);   \
                    return hipGetLastError();                                                  \
                }                                                                              \
            }                                                                                  \
            if (hv) return hipErrorInvalidValue;                                               \
            hipLaunchKernelGGL((gemm_pipe<BM_, BN_, S_, BK_, L, ST, NW_, LD_ != 0>), grid,     \
                               dim3((NW_ + 4 * LD_) * 64), 0, stream, op, ta);                 \
            return hipGetLastError();                                                          \
        }                                                                                      \
    }
    FLINT_PIPE_CASE(256, 256, 3, 32, 4, 0)
    FLINT_PIPE_CASE(256, 192, 4, 32, 4, 0)
    FLINT_PIPE_CASE(128, 192, 4, 32, 4, 0)
    FLINT_PIPE_CASE(256, 64, 4, 32, 4, 0)
    FLINT_PIPE_CASE(128, 64, 4, 32, 4, 0)
    FLINT_PIPE_CASE(128, 64, 3, 64, 4, 0)
    FLINT_PIPE_CASE(256, 64, 3, 64, 4, 0)
    FLINT_PIPE_CASE(128, 192, 3, 64, 4, 0)
    FLINT_PIPE_CASE(256, 128, 3, 64, 4, 0)
    FLINT_PIPE_CASE(256, 256, 2, 64, 4, 0)
    FLINT_PIPE_CASE(256, 192, 2, 64, 4, 0)
    FLINT_PIPE_CASE(128, 192, 3, 64, 4, 1)
    FLINT_PIPE_CASE(256, 128, 3, 64, 4, 1)
    if constexpr (L == Layout::kNT) {
        FLINT_PIPE_CASE(256, 192, 2, 64, 8, 0)
    }
#undef FLINT_PIPE_CASE
    return hipErrorInvalidValue;
}

Store store_of(Epilogue e, Layout l) {
    if (e == kTnFloat) return Store::kTn;
    switch (e) {
    case Epilogue::kNone: return l == Layout::kTN ? Store::kTnHalf : Store::kNone;
    case Epilogue::kBias: return Store::kBias;
    case Epilogue::kBiasGelu: return Store::kBiasGelu;
    case Epilogue::kBiasResidual: return Store::kBiasResidual;
    case Epilogue::kDGelu: return Store::kDGelu;
    case Epilogue::kScale: return Store::kScale;
    }
    return Store::kNone;
}

Layout layout_of(GemmLayout l) {
    return l == GemmLayout::kNT ? Layout::kNT : (l == GemmLayout::kNN ? Layout::kNN : Layout::kTN);
}

template <Layout L>
hipError_t dispatch_pipe(const PipeConfig& c, Store st, const Operands& op, size_t slices,
                         int split_len, int cus, hipStream_t stream) {
    if constexpr (L == Layout::kNT) {
        switch (st) {
        case Store::kNone: return launch_pipe<L, Store::kNone>(c, op, slices, split_len, cus, stream);
        case Store::kBias: return launch_pipe<L, Store::kBias>(c, op, slices, split_len, cus, stream);
        case Store::kBiasGelu:
            return launch_pipe<L, Store::kBiasGelu>(c, op, slices, split_len, cus, stream);
        case Store::kBiasResidual:
            return launch_pipe<L, Store::kBiasResidual>(c, op, slices, split_len, cus, stream);
        case Store::kScale:
            return launch_pipe<L, Store::kScale>(c, op, slices, split_len, cus, stream);
        default: break;
        }
    } else if constexpr (L == Layout::kNN) {
        switch (st) {
        case Store::kNone: return launch_pipe<L, Store::kNone>(c, op, slices, split_len, cus, stream);
        case Store::kDGelu:
            return launch_pipe<L, Store::kDGelu>(c, op, slices, split_len, cus, stream);
        default: break;
        }
    } else {
        switch (st) {
        case Store::kTn: return launch_pipe<L, Store::kTn>(c, op, slices, split_len, cus, stream);
        case Store::kTnHalf:
            return launch_pipe<L, Store::kTnHalf>(c, op, slices, split_len, cus, stream);
        default: break;
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_gemm_pipe_tn(void* y, const void* x, const void* w, size_t m, size_t n,
                               size_t k, bool accumulate, void* workspace, int max_splits,
                               int* splits, hipStream_t stream) {
    int cus = 256;
    if (hipError_t err = device_cus(&cus); err != hipSuccess) return err;
    PipeConfig c;
    int sp = 1;
    bool disabled = false;
    PipeConfig forced;
    const bool force = pipe_forced(&forced, &disabled) && usable(forced, Store::kTn, k, Layout::kTN);
    plan_tn(m, n, k, workspace != nullptr ? max_splits : 1, cus, accumulate,
            force ? &forced : nullptr, &c, &sp);
    const size_t len = ((k + sp - 1) / sp + c.bk - 1) / c.bk * c.bk;
    Operands op{};
    op.y = y;
    op.x = static_cast<const _Float16*>(x);
    op.w = static_cast<const _Float16*>(w);
    op.partials = sp > 1 ? static_cast<float*>(workspace) : nullptr;
    op.accumulate = accumulate ? 1 : 0;
    op.scale = 1.0f;
    op.m = int(m);
    op.n = int(n);
    op.k = int(k);
    *splits = sp;
    return launch_pipe<Layout::kTN, Store::kTn>(c, op, size_t(sp), int(len), cus, stream);
}

bool gemm_pipe_eligible(GemmLayout gl, Epilogue e, size_t m, size_t n, size_t k) {
    bool disabled = false;
    PipeConfig forced;
    pipe_forced(&forced, &disabled);
    if (disabled || m == 0 || n == 0 || n % 8 != 0 || k % kPipeBK != 0 || k < kPipeBK) return false;
    const Layout l = layout_of(gl);
    const Store st = store_of(e, l);
    // Only the epilogues each layout serves.
    const bool served = l == Layout::kNT ? (st == Store::kNone || st == Store::kBias ||
                                            st == Store::kBiasGelu || st == Store::kBiasResidual ||
                                            st == Store::kScale)
                        : l == Layout::kNN ? (st == Store::kNone || st == Store::kDGelu)
                                           : (st == Store::kTn || st == Store::kTnHalf);
    if (!served) return false;
    // k-major operands come in 16-byte chunks of their columns.
    if (l == Layout::kTN && m % 8 != 0) return false;
    // Buffer offsets are 32-bit: one slice's output and each operand.
    const size_t out_elem = st == Store::kBiasResidual || st == Store::kTn ? 4 : 2;
    if (m * n * out_elem >= (size_t{1} << 31) || m * k * 2 >= (size_t{1} << 31) ||
        n * k * 2 >= (size_t{1} << 31)) {
        return false;
    }
    return true;
}

hipError_t launch_gemm_pipe(GemmLayout gl, Epilogue e, void* y, const void* x, const void* w,
                            const void* bias, void* aux, float scale, size_t slices, size_t m,
                            size_t n, size_t k, bool accumulate, void* partials, int split_len,
                            hipStream_t stream, bool causal, const HeadView* wv,
                            const HeadView* yv) {
    // Heads views: batched NN / TN with FP16 outputs only, every slice a
    // whole (sequence, head) pair.
    if (wv != nullptr || yv != nullptr) {
        const bool ok_layout = gl != GemmLayout::kNT && e == Epilogue::kNone && slices > 1 &&
                               split_len == 0 && partials == nullptr && !accumulate;
        // A slice's rows, ld apart, must stay within the 32-bit buffer range.
        auto ok_view = [&](const HeadView* v, size_t rows) {
            return v == nullptr ||
                   (v->heads > 0 && slices % size_t(v->heads) == 0 && v->ld >= 0 &&
                    size_t(v->ld) >= n && v->seq >= 0 && v->head >= 0 &&
                    ((rows - 1) * size_t(v->ld) + n) * 2 < (size_t{1} << 31));
        };
        if (!ok_layout || !ok_view(wv, k) || !ok_view(yv, m)) return hipErrorInvalidValue;
    }
    int cus = 256;
    if (hipError_t err = device_cus(&cus); err != hipSuccess) return err;
    Operands op{};
    op.y = y;
    op.x = static_cast<const _Float16*>(x);
    op.w = static_cast<const _Float16*>(w);
    op.bias = static_cast<const float*>(bias);
    op.aux = aux;
    op.partials = static_cast<float*>(partials);
    op.scale = scale;
    op.accumulate = accumulate ? 1 : 0;
    op.m = int(m);
    op.n = int(n);
    op.k = int(k);
    const Layout l = layout_of(gl);
    // Causal needs the square operand, and no TN split (k-ranges of its own).
    op.causal = causal && split_len == 0 &&
                        (l == Layout::kNT ? m == n : m == k) ? 1 : 0;
    // Both views set (heads != 0 selects the view kernels); a missing one is
    // the plain [slices][rows][cols] layout as a view of one head.
    if (wv != nullptr || yv != nullptr) {
        auto plain = [](size_t rows, size_t cols) {
            HeadView v;
            v.heads = 1;
            v.ld = int(cols);
            v.seq = (long long)(rows * cols);
            v.head = 0;
            return v;
        };
        op.wv = wv != nullptr ? *wv : plain(k, n);
        op.yv = yv != nullptr ? *yv : plain(m, n);
    }
    const Store st = store_of(e, l);
    PipeConfig c;
    bool disabled = false;
    if (!pipe_forced(&c, &disabled) || !usable(c, st, k, l))
        c = pick_pipe(m, n, k, slices, cus, st, l, op.causal != 0);
    switch (l) {
    case Layout::kNT: return dispatch_pipe<Layout::kNT>(c, st, op, slices, split_len, cus, stream);
    case Layout::kNN: return dispatch_pipe<Layout::kNN>(c, st, op, slices, split_len, cus, stream);
    case Layout::kTN: return dispatch_pipe<Layout::kTN>(c, st, op, slices, split_len, cus, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace flint
