// The NT GEMM as an eight-wave ping-pong for gfx950: two waves per SIMD take
// turns, one issuing its MFMAs while the other reads its next fragments from
// LDS, streams the next k-step into LDS and runs its epilogue.
//
// Why this shape of kernel (measured on MI355X, counters of the one-wave-per-
// SIMD pipeline in gemm_pipe.hip on MLP up 8192 x 3072 x 768 + bias + GELU):
// the matrix cores were busy 28% of the kernel's cycles. With one wave per
// SIMD every wait of that wave (for a k-step's loads, at a barrier, for LDS)
// and every instruction of its epilogue (about 6,000 VALU instructions per
// wave for bias + GELU over its two tiles) leaves the MFMA pipe idle. With two
// waves per SIMD in alternating roles the other wave has its MFMAs ready
// while one waits.
//
// Layout of the work:
//  * A workgroup of 8 waves owns a BM x BN output tile (BM = 256). Waves w and
//    w + 4 run on SIMD w % 4; wave w computes rows (w % 4) BM/4 .. + BM/4 and
//    columns (w / 4) BN/2 .. + BN/2 of the tile: group 0 (waves 0-3) the left
//    half, group 1 (waves 4-7) the right half, both from the same x rows.
//  * k-steps of 64 through two LDS stages, each holding BM + BN rows of 128
//    bytes (x rows, then w rows), 16-byte chunks XOR-swizzled per row. A
//    step's loads (1 KB direct-to-LDS buffer loads, (BM + BN) / 8 of them) are
//    shared by all 8 waves.
//  * Each wave alternates slots separated by workgroup barriers: a compute
//    slot (the MFMAs of one k32 unit: two k16 sub-steps) and a memory slot
//    (the next unit's fragment reads, its share of a k-step's loads, and at a
//    tile's end its epilogue). Group 1 starts one slot later, so in every slot
//    one wave of each SIMD computes while the other does memory work.
//  * The loads of step t + 1 go out in the memory slot that reads step t's
//    first unit, right after the last reads of step t - 1 (whose stage they
//    overwrite) are past a barrier; each wave waits for its own share three to
//    four slots later, before the barrier ahead of the first read of step t + 1.
//  * Workgroups are persistent: the k-step stream runs across the tiles of a
//    workgroup, so the next tile's first steps load under this tile's
//    epilogue.
//  * The epilogue stages each wave's accumulators through its own LDS block,
//    a few rows at a time, so that every store instruction writes whole
//    16-byte chunks of rows (non-temporal buffer stores; chunks outside the
//    output get an offset past the resource's end and are dropped).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>

#include "common/common.h"
#include "kernels/gemm_common.h"
#include "kernels/kernels.h"

namespace flint {
namespace {

constexpr int kPpBK = 64;
constexpr int kPpThreads = 512;
constexpr size_t kPpLds = 160 * 1024;
constexpr int kPpStoreAux = 2;    // the nt bit: outputs are read by a later kernel

typedef int i32x4 __attribute__((ext_vector_type(4)));

// s_waitcnt vmcnt(N) lgkmcnt(0).
template <int N>
__device__ __forceinline__ void pp_wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

// Key XORed into the 16-byte chunk index of a 128-byte LDS row: the 16 lanes
// one LDS cycle of a ds_read_b128 serves read one chunk of 16 consecutive
// rows; an even and an odd row fill the two halves of the 64 banks, and
// (row >> 1) & 7 gives each pair its own chunk position.
__device__ __forceinline__ int pp_key(int row) { return (row >> 1) & 7; }

// The epilogue's staging of one wave's WTN-wide rows, ROWS rows at a time.
template <int WTN, Store ST, int ROWS>
struct PpEpi {
    static constexpr bool kF32 = ST == Store::kBiasResidual;
    static constexpr int kOutElem = kF32 ? 4 : 2;
    static constexpr int kPerChunk = kF32 ? 4 : 8;      // values per 16-byte chunk
    static constexpr int kRows = ROWS;
    static constexpr int kLdw = WTN + kPerChunk;        // staged row stride (values)
    static constexpr int kBytes = kRows * kLdw * (kF32 ? 4 : 2);
    static constexpr int kCpr = WTN / kPerChunk;        // chunks per row
    static constexpr int kPerLane = kRows * kCpr / 64;  // chunks per lane per block
    static constexpr int kPasses = ST == Store::kBiasGelu ? 2 : 1;
    static constexpr int kSubs = 32 / kRows;            // staged blocks per 32 rows
};

template <int BM, int BN>
constexpr size_t pp_stage_bytes() {
    return size_t(2) * (BM + BN) * kPpBK * 2;
}

// Rows staged at a time: the most of 32, 16, 8 and 4 whose staging for 8
// waves fits beside the two stages and fills whole store instructions.
template <int BM, int BN, Store ST>
constexpr int pp_rows() {
    constexpr int wtn = BN / 2;
    constexpr bool f32 = ST == Store::kBiasResidual;
    constexpr int per = f32 ? 4 : 8;
    for (int rows = 32; rows >= 4; rows /= 2) {
        const size_t bytes = size_t(rows) * (wtn + per) * (f32 ? 4 : 2);
        if (pp_stage_bytes<BM, BN>() + 8 * bytes <= kPpLds && rows * (wtn / per) % 64 == 0)
            return rows;
    }
    return 0;
}

template <int BM, int BN, Store ST>
__global__ void __launch_bounds__(kPpThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemm_pp(Operands op, TileArgs ta) {
#if defined(__HIP_DEVICE_COMPILE__)
    constexpr int BK = kPpBK;
    constexpr int WTM = BM / 4, WTN = BN / 2;
    constexpr int FM = WTM / 32, FN = WTN / 32;
    constexpr int LOADS = (BM + BN) / 8;          // 1 KB loads per k-step
    constexpr int PER = LOADS / 8;                // per wave
    constexpr int STAGE = (BM + BN) * BK;         // halves per stage
    constexpr int ROWS = pp_rows<BM, BN, ST>();
    static_assert(ROWS > 0, "epilogue staging does not fit");
    using E = PpEpi<WTN, ST, ROWS>;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0 && LOADS % 8 == 0, "tile shape");
    constexpr bool kBias =
        ST == Store::kBias || ST == Store::kBiasGelu || ST == Store::kBiasResidual;
    constexpr int kStores = FM * E::kSubs * E::kPerLane * E::kPasses;
    static_assert(kStores < 64 && 2 * PER < 64, "vmcnt range");
    __shared__ __attribute__((aligned(16))) _Float16 lds[2 * STAGE + 8 * E::kBytes / 2];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2, pos = wave & 3;
    const int fr = lane & 31, fc = lane >> 5;
    const int m = op.m, n = op.n, K = op.k;
    _Float16* const cst = lds + 2 * STAGE + wave * (E::kBytes / 2);

    const unsigned total = unsigned(ta.tiles_per_slice) * unsigned(ta.slices);
    const int n_tiles = int((total - 1 - blockIdx.x) / gridDim.x) + 1;
    const int steps = K / BK;                     // per tile
    const int s_total = n_tiles * steps;
    const int upt = 2 * steps;                    // k32 units per tile
    const int u_total = n_tiles * upt;

    struct Tile {
        int m0, n0;
    };
    auto tile = [&](int i) {
        int slice, tm, tn;
        map_tile(ta, blockIdx.x + unsigned(i) * gridDim.x, &slice, &tm, &tn);
        return Tile{tm * BM, tn * BN};
    };

    // This wave's loads of a step: instruction u = q * 8 + wave (q < PER)
    // fills LDS bytes [u KB, u KB + 1 KB) of the stage: 8 rows of 128 bytes,
    // x rows for u < BM / 8, then w rows. Lane l writes row l / 8, chunk
    // position l % 8, which holds global chunk (l % 8) ^ key(row).
    unsigned voff[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        const int u = q * 8 + wave;
        const int row = (u < BM / 8 ? u : u - BM / 8) * 8 + (lane >> 3);
        voff[q] = unsigned((row * K + (((lane & 7) ^ pp_key(row)) * 8)) * 2);
    }
    // The issue cursor: the next step to load and its tile's resources.
    struct Cursor {
        int step, tile, k0;
        __amdgpu_buffer_rsrc_t ra, rb;
    };
    auto set_tile = [&](Cursor& c, int i) {
        const Tile t = tile(i);
        c.tile = i;
        c.ra = __builtin_amdgcn_make_buffer_rsrc(
            uniform_ptr(op.x + size_t(t.m0) * K), 0,
            unsigned(min(BM, m - t.m0)) * unsigned(K) * 2u, 0x00020000);
        c.rb = __builtin_amdgcn_make_buffer_rsrc(
            uniform_ptr(op.w + size_t(t.n0) * K), 0,
            unsigned(min(BN, n - t.n0)) * unsigned(K) * 2u, 0x00020000);
    };
    // Past the stream's last step the cursor reloads that step into the stage
    // it frees (nobody reads it again), so every wave issues the same loads in
    // every slot and each wait below counts the same operations.
    auto issue_step = [&](Cursor& c) {
        _Float16* const stage = lds + (c.step & 1) * STAGE;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int u = q * 8 + wave;
            lds_half* dst = (lds_half*)(stage + u * 512);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(u < BM / 8 ? c.ra : c.rb,
                                                     (__attribute__((address_space(3))) void*)dst,
                                                     16, voff[q], unsigned(c.k0) * 2u, 0, 0);
        }
        ++c.step;
        if (c.step < s_total) {
            c.k0 += BK;
            if (c.k0 == K) {
                c.k0 = 0;
                set_tile(c, c.tile + 1);
            }
        }
    };

    f32x16 acc[FN][FM];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = f32x16{};
    f16x8 xf[2][FM], wf[2][FN];

    // Fragments of unit u (k16 sub-steps 2 (u % 2) and + 1 of its step):
    // lane l gets row r0 + l % 32, halves 8 (l / 32) .. + 8 of the sub-step.
    auto read_unit = [&](int u) {
        const int s = u >> 1;
        const _Float16* st = lds + (s & 1) * STAGE;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int kk = (u & 1) * 2 + h;
#pragma unroll
            for (int j = 0; j < FM; ++j) {
                const int row = pos * WTM + j * 32 + fr;
                xf[h][j] = *reinterpret_cast<const f16x8*>(
                    st + row * BK + (((kk * 2 + fc) ^ pp_key(row)) * 8));
            }
#pragma unroll
            for (int i = 0; i < FN; ++i) {
                const int row = grp * WTN + i * 32 + fr;
                wf[h][i] = *reinterpret_cast<const f16x8*>(
                    st + BM * BK + row * BK + (((kk * 2 + fc) ^ pp_key(row)) * 8));
            }
        }
    };
    auto compute_unit = [&]() {
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[h][i], xf[h][j],
                                                                       acc[i][j], 0, 0, 0);
        __builtin_amdgcn_s_setprio(0);
    };

    // Bias of this lane's columns: lane l holds columns 32 i + 8 g4 + 4 (l / 32)
    // .. + 4 of its wave's block i (columns past n read 0).
    f32x4 bias[kBias ? FN : 1][4];
    auto load_bias = [&](const Tile& t) {
        if constexpr (kBias) {
            const auto rbias = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(op.bias), 0,
                                                                 unsigned(n) * 4u, 0x00020000);
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const int c = t.n0 + grp * WTN + i * 32 + g4 * 8 + fc * 4;
                    bias[i][g4] = __builtin_bit_cast(
                        f32x4, __builtin_amdgcn_raw_buffer_load_b128(rbias, unsigned(c) * 4u, 0, 0));
                }
        }
    };

    // The epilogue of tile t for this wave: per staged block of ROWS rows,
    // registers -> staging (the lanes holding those rows) -> whole 16-byte
    // chunks to HBM (every lane), kStores buffer stores in all.
    auto epilogue = [&](const Tile& t) {
        const int row_base = t.m0 + pos * WTM;
        const int col_base = t.n0 + grp * WTN;
        const unsigned out_bytes = unsigned(size_t(m) * n * E::kOutElem);
        auto chunk_at = [&](int j, int hb, int q, int elem, int* r, int* cc) {
            const int c = q * 64 + lane;
            *r = c / E::kCpr;
            *cc = c % E::kCpr;
            const int gr = row_base + j * 32 + hb * E::kRows + *r;
            const int gc = col_base + *cc * E::kPerChunk;
            return gr < m && gc < n ? (unsigned(gr) * unsigned(n) + unsigned(gc)) * unsigned(elem)
                                    : 0xfffffff0u;
        };
#pragma unroll
        for (int j = 0; j < FM; ++j) {
#pragma unroll
            for (int hb = 0; hb < E::kSubs; ++hb) {
                f32x4 rd[ST == Store::kBiasResidual ? E::kPerLane : 1];
                if constexpr (ST == Store::kBiasResidual) {
                    const auto rs = __builtin_amdgcn_make_buffer_rsrc(
                        const_cast<void*>(static_cast<const void*>(op.aux)), 0, out_bytes,
                        0x00020000);
#pragma unroll
                    for (int q = 0; q < E::kPerLane; ++q) {
                        int r, cc;
                        rd[q] = __builtin_bit_cast(
                            f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                       rs, chunk_at(j, hb, q, 4, &r, &cc), 0, 0));
                    }
                }
#pragma unroll
                for (int pass = 0; pass < E::kPasses; ++pass) {
                    const bool gelu_pass = ST == Store::kBiasGelu && pass == 1;
                    if (E::kRows == 32 || fr / E::kRows == hb) {
                        const int srow = fr % E::kRows;
#pragma unroll
                        for (int i = 0; i < FN; ++i) {
#pragma unroll
                            for (int g4 = 0; g4 < 4; ++g4) {
                                f32x4 v = {acc[i][j][g4 * 4 + 0], acc[i][j][g4 * 4 + 1],
                                           acc[i][j][g4 * 4 + 2], acc[i][j][g4 * 4 + 3]};
                                if constexpr (kBias) v += bias[i][g4];
                                const int at = srow * E::kLdw + i * 32 + g4 * 8 + fc * 4;
                                if constexpr (E::kF32) {
                                    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(cst) + at) = v;
                                } else {
                                    if (gelu_pass) {
#pragma unroll
                                        for (int e = 0; e < 4; ++e) v[e] = gelu(v[e]);
                                    }
                                    const f16x4 hv = {_Float16(v[0]), _Float16(v[1]),
                                                      _Float16(v[2]), _Float16(v[3])};
                                    *reinterpret_cast<f16x4*>(cst + at) = hv;
                                }
                            }
                        }
                    }
                    // Every lane reads what the row-holding lanes wrote.
                    __builtin_amdgcn_wave_barrier();
                    asm volatile("" ::: "memory");
                    void* out = ST == Store::kBiasGelu && pass == 0 ? op.aux : op.y;
                    const auto rout = __builtin_amdgcn_make_buffer_rsrc(out, 0, out_bytes, 0x00020000);
#pragma unroll
                    for (int q = 0; q < E::kPerLane; ++q) {
                        int r, cc;
                        if constexpr (E::kF32) {
                            const unsigned off = chunk_at(j, hb, q, 4, &r, &cc);
                            const f32x4 sv = *reinterpret_cast<const f32x4*>(
                                reinterpret_cast<const float*>(cst) + r * E::kLdw + cc * 4);
                            const f32x4 o = rd[q] + sv;
                            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, o),
                                                                   rout, off, 0, kPpStoreAux);
                        } else {
                            const unsigned off = chunk_at(j, hb, q, 2, &r, &cc);
                            const f16x8 v = *reinterpret_cast<const f16x8*>(cst + r * E::kLdw + cc * 8);
                            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v),
                                                                   rout, off, 0, kPpStoreAux);
                        }
                    }
                    // The next block's writes come after these reads.
                    __builtin_amdgcn_wave_barrier();
                    asm volatile("" ::: "memory");
                }
            }
        }
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FM; ++j) acc[i][j] = f32x16{};
    };

    // ---- prologue: steps 0 and 1 go out; step 0 lands; unit 0's fragments.
    Cursor cur;
    cur.step = 0;
    cur.k0 = 0;
    set_tile(cur, 0);
    issue_step(cur);
    issue_step(cur);
    pp_wait_vm_lgkm0<PER>();
    block_sync();
    read_unit(0);
    if (grp == 1) block_sync();     // group 1 runs one slot behind

    for (int u = 0; u < u_total; ++u) {
        // ---- compute slot: unit u's MFMAs.
        compute_unit();
        // Group 0 waits here for its share of step (u + 1) / 2 (issued in the
        // memory slot of unit u - 1), which group 0 reads after the barrier
        // that ends group 1's next memory slot. The stores of an epilogue in
        // that memory slot came after the loads and may stay in flight.
        if (grp == 0 && (u & 1)) {
            if ((u - 1) % upt == 0 && u > 1) pp_wait_vm_lgkm0<kStores>();
            else pp_wait_vm_lgkm0<0>();
        }
        block_sync();
        // ---- memory slot of unit v = u + 1.
        const int v = u + 1;
        const bool tile_end = v % upt == 0;
        if (tile_end) load_bias(tile(v / upt - 1));
        __builtin_amdgcn_sched_barrier(0);
        // The first unit of a step issues the loads of the step after it.
        if (!(v & 1)) issue_step(cur);
        __builtin_amdgcn_sched_barrier(0);
        if (tile_end) epilogue(tile(v / upt - 1));
        if (v < u_total) read_unit(v);
        if (grp == 1 && (v & 1)) {
            if ((v - 1) % upt == 0 && v > 1) pp_wait_vm_lgkm0<kStores>();
            else pp_wait_vm_lgkm0<0>();
        }
        block_sync();
    }
    if (grp == 0) block_sync();
    wait_vmcnt<0>();
#endif
}

struct PpConfig {
    int bm, bn;
};
constexpr PpConfig kPpConfigs[] = {{256, 256}, {256, 192}, {256, 128}};

// 256 x 256 holds 128 accumulators per wave, which leaves too few registers
// for a bias epilogue (it spills); it serves the plain product only.
bool pp_serves(const PpConfig& c, Epilogue e) { return c.bn != 256 || e == Epilogue::kNone; }

// FLINT_GEMM_PP: "0" turns the ping-pong kernel off; "bm,bn" forces one of
// kPpConfigs (tests and tuning sweeps; read per call).
bool pp_env(PpConfig* forced, bool* disabled, Epilogue e) {
    *disabled = false;
    const char* env = std::getenv("FLINT_GEMM_PP");
    if (env == nullptr) return false;
    if (env[0] == '0' && env[1] == '\0') {
        *disabled = true;
        return false;
    }
    PpConfig c{};
    if (std::sscanf(env, "%d,%d", &c.bm, &c.bn) != 2) return false;
    for (const PpConfig& k : kPpConfigs) {
        if (k.bm == c.bm && k.bn == c.bn && pp_serves(k, e)) {
            *forced = c;
            return true;
        }
    }
    return false;
}

// Whole rounds of tiles over the CUs weigh most; then tile area (larger tiles
// load fewer bytes per FLOP).
PpConfig pick_pp(size_t m, size_t n, int cus, Epilogue e) {
    PpConfig best = kPpConfigs[1];
    double best_cost = 1e300;
    for (const PpConfig& c : kPpConfigs) {
        if (!pp_serves(c, e)) continue;
        const double tiles = double((m + c.bm - 1) / c.bm) * double((n + c.bn - 1) / c.bn);
        const double rounds = std::ceil(tiles / cus);
        const double eff = c.bn == 256 ? 1.0 : (c.bn == 192 ? 0.97 : 0.9);
        const double cost = rounds * double(c.bm) * double(c.bn) / eff;
        if (cost < best_cost * 0.999) {
            best_cost = cost;
            best = c;
        }
    }
    return best;
}

template <Store ST>
hipError_t launch_pp(const PpConfig& c, const Operands& op, int cus, hipStream_t stream) {
    TileArgs ta{};
    ta.tiles_m = (op.m + c.bm - 1) / c.bm;
    ta.tiles_n = (op.n + c.bn - 1) / c.bn;
    ta.tiles_per_slice = ta.tiles_m * ta.tiles_n;
    ta.slices = 1;
    ta.group_m = 8;
    const size_t total = size_t(ta.tiles_per_slice);
    size_t gx = std::min(total, size_t(cus));
    if (gx >= 8) gx -= gx % 8;
#define FLINT_PP_CASE(BM_, BN_)                                                                 \
    if (c.bm == BM_ && c.bn == BN_) {                                                           \
        hipLaunchKernelGGL((gemm_pp<BM_, BN_, ST>), dim3(unsigned(gx)), dim3(kPpThreads), 0,   \
                           stream, op, ta);                                                     \
        return hipGetLastError();                                                               \
    }
    if constexpr (ST == Store::kNone) FLINT_PP_CASE(256, 256)
    FLINT_PP_CASE(256, 192)
    FLINT_PP_CASE(256, 128)
#undef FLINT_PP_CASE
    return hipErrorInvalidValue;
}

}  // namespace

bool gemm_pp_eligible(Epilogue e, size_t m, size_t n, size_t k) {
    PpConfig forced;
    bool disabled = false;
    const bool force = pp_env(&forced, &disabled, e);
    if (disabled || m == 0 || n == 0 || n % 8 != 0 || k % kPpBK != 0 || k == 0) return false;
    if (e != Epilogue::kNone && e != Epilogue::kBias && e != Epilogue::kBiasGelu &&
        e != Epilogue::kBiasResidual)
        return false;
    // Buffer offsets are 32-bit: the output and each operand.
    const size_t out_elem = e == Epilogue::kBiasResidual ? 4 : 2;
    if (m * n * out_elem >= (size_t{1} << 31) || m * k * 2 >= (size_t{1} << 31) ||
        n * k * 2 >= (size_t{1} << 31))
        return false;
    // Only when a tile is forced: measured against the one-wave-per-SIMD
    // pipeline (gemm_pipe.hip) this kernel is slower at every GPT-2 shape (MLP
    // up 65 against 55 us, logits 805 against 747 us): its 64-row wave tiles
    // read 43% more LDS per MFMA, and its memory slots (fragment reads, the
    // TA-bound load issue, the epilogue) run about three times as long as a
    // compute slot, so the computing waves wait at the barriers.
    return force;
}

hipError_t launch_gemm_pp(Epilogue e, void* y, const void* x, const void* w, const void* bias,
                          void* aux, size_t m, size_t n, size_t k, hipStream_t stream) {
    int cus = 256;
    if (hipError_t err = device_cus(&cus); err != hipSuccess) return err;
    Operands op{};
    op.y = y;
    op.x = static_cast<const _Float16*>(x);
    op.w = static_cast<const _Float16*>(w);
    op.bias = static_cast<const float*>(bias);
    op.aux = aux;
    op.scale = 1.0f;
    op.m = int(m);
    op.n = int(n);
    op.k = int(k);
    PpConfig c;
    bool disabled = false;
    if (!pp_env(&c, &disabled, e)) c = pick_pp(m, n, cus, e);
    switch (e) {
    case Epilogue::kNone: return launch_pp<Store::kNone>(c, op, cus, stream);
    case Epilogue::kBias: return launch_pp<Store::kBias>(c, op, cus, stream);
    case Epilogue::kBiasGelu: return launch_pp<Store::kBiasGelu>(c, op, cus, stream);
    case Epilogue::kBiasResidual: return launch_pp<Store::kBiasResidual>(c, op, cus, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace flint
