// Fused causal attention for gfx950, head width 64: the forward pass
// O = softmax(scale Q K^T, causal) V with its per-query log-sum-exp, and the
// backward pass to dQ, dK and dV, without materialising the length x length
// scores or probabilities in HBM.
//
// Layout: q, k, v, o, dO, dQ, dK, dV hold 64-half rows of FP16 at a row
// stride of their own (AttnLayout: [batches][length][64] for the C ABI, the
// heads' slices of [tokens][width] rows inside the model); lse and D (the
// backward's row sums of dO * O) are [batches][length] FP32.
//
// How the work maps to the hardware:
//  * Scores come from v_mfma_f32_32x32x16_f16 computing S^T = K Q^T (keys as
//    the MFMA's rows, queries as its columns): each lane then holds one query
//    (lane % 32) and 16 keys per 32-key block (8a + 4h + b for register
//    4a + b, h = lane / 32), so a query's running max, sum and rescale are
//    per-lane values and the row reductions are in-register plus one exchange
//    with lane ^ 32.
//  * The probabilities feed the next MFMA straight from those registers as
//    its B operand (queries as columns, keys as k): within a 16-key step a
//    lane holds keys 4h .. 4h + 3 and 8 + 4h .. 8 + 4h + 3, and the k order of
//    an MFMA is free as long as both operands agree, so the A operand (V^T or
//    K^T, d as rows) is read with the same key order by two ds_read_b64_tr_b16,
//    each giving a lane 4 consecutive rows (keys) of one column (d) of the
//    row-major LDS tile.
//  * K and V tiles of 64 keys (8 KB each) stream into LDS with direct-to-LDS
//    buffer loads, double-buffered, one barrier per block; rows are 128 bytes
//    with 16-byte chunks XOR-swizzled by (row >> 1) & 7. Loads past the
//    sequence read zeros.
//  * exp is exp2 of scores pre-scaled by scale * log2(e); lse is kept in log2
//    units inside the kernels and stored as a natural log.
//  * The backward is deterministic (no atomics): one kernel owns a block of
//    queries and accumulates dQ over the keys (it also writes D), a second
//    owns a block of keys and accumulates dK and dV over the queries; both
//    recompute P from Q, K and lse (FlashAttention-2's scheme).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdlib>
#include <type_traits>

#include "common/common.h"
#include "common/tuning.h"
#include "kernels/gemm_common.h"
#include "kernels/kernels.h"

namespace flint {
namespace {

constexpr int kHd = 64;                  // head width
constexpr int kTile = 64 * kHd;          // halves in a 64-row tile (8 KB)
constexpr int kAttnThreads = 256;        // 4 waves
constexpr float kLn2 = 0.69314718055994531f;
constexpr float kLog2e = 1.4426950408889634f;
// How far (log2 units) a query's scores may rise above the forward's running
// max before O and l are rescaled: P = 2^(c s - m) <= 2^8 until then.
constexpr float kRescale = 8.0f;

typedef int i32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int akey(int row) { return (row >> 1) & 7; }

struct TrPair {
    i32x2 lo, hi;
};
__device__ __forceinline__ f16x8 join(const TrPair& f) {
    return __builtin_shufflevector(__builtin_bit_cast(f16x4, f.lo), __builtin_bit_cast(f16x4, f.hi),
                                   0, 1, 2, 3, 4, 5, 6, 7);
}
// lgkmcnt(0): the transposing reads are inline asm, invisible to the
// compiler's wait insertion.
__device__ __forceinline__ void wait_lds() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_sched_barrier(0);
}

// The work item (in longest-first order) that workgroup `bid` takes. The
// kernels' grids are about what the GPU holds at once, so dispatch does little
// balancing, and workgroups bid, bid + CUs, bid + 2 CUs, ... tend to share a
// CU. With round > 0 (the CU count) every other run of `round` workgroups
// takes its items in reverse, so that a CU's workgroups pair long items with
// short ones.
__device__ __forceinline__ int work_rank(int bid, int round, int total) {
    if (round <= 0) return bid;
    const int r = bid / round, pos = bid - r * round;
    if ((r & 1) == 0) return bid;
    const int n = min(round, total - r * round);
    return r * round + (n - 1 - pos);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const void* base, unsigned bytes) {
    const uint64_t v = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(v >> 32));
    void* p = reinterpret_cast<void*>((uint64_t(hi) << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(p, 0, bytes, 0x00020000);
}

// Rows r0 .. r0 + 63 of a matrix of 64-half rows `stride` halves apart into a
// tile: 8 loads of 1 KB (8 rows each), two per wave. Lane l writes row l / 8
// at chunk position l % 8, which holds global chunk (l % 8) ^ key(row).
__device__ __forceinline__ void load_tile(_Float16* tile, __amdgpu_buffer_rsrc_t rs, int r0,
                                          int stride, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int u = wave + 4 * i;
        const int row = u * 8 + (lane >> 3);
        const unsigned voff = unsigned(((r0 + row) * stride + (((lane & 7) ^ akey(row)) * 8)) * 2);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (__attribute__((address_space(3))) void*)(lds_half*)(tile + u * 512), 16, voff, 0, 0, 0);
    }
}

// Per-lane byte offsets of the fragment reads inside a 64-row tile, computed
// once per kernel and kept in registers (an empty asm makes them opaque, so
// they are not recomputed per read): the row-major read of (32 hb, kk) is
// rows[kk] + 4096 hb, the transposing reads of (16 cs, db) are tr[db][0 | 1]
// + 2048 cs. The key (row >> 1) & 7 of the XOR swizzle is the same for rows
// 32 or 16 apart, which is what lets hb and cs become immediate offsets.
struct FragOff {
    unsigned rows[4];
    unsigned tr[2][2];
};
__device__ __forceinline__ FragOff frag_offsets(int lane) {
    FragOff f;
    const int fr = lane & 31, h = lane >> 5, j = lane & 15;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        f.rows[kk] = unsigned((fr * kHd + (((2 * kk + h) ^ akey(fr)) * 8)) * 2);
        asm volatile("" : "+v"(f.rows[kk]));
    }
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int row = 4 * h + (j >> 2) + 8 * t;
            const int col = 32 * db + 16 * ((lane >> 4) & 1) + 4 * (j & 3);
            f.tr[db][t] = unsigned((row * kHd + (((col >> 3) ^ akey(row)) * 8) + (col & 7)) * 2);
            asm volatile("" : "+v"(f.tr[db][t]));
        }
    return f;
}

// An MFMA operand with tile rows as its rows and d as k: lane l gets row
// 32 hb + l % 32, halves 16 kk + 8 (l / 32) .. + 8.
__device__ __forceinline__ f16x8 frag_rows(const _Float16* tile, const FragOff& fo, int hb, int kk) {
    return *reinterpret_cast<const f16x8*>(reinterpret_cast<const char*>(tile) + fo.rows[kk] +
                                           4096 * hb);
}

// An MFMA operand with d as its rows and tile rows as k, in the permuted k
// order of the register-held probabilities: lane l (d = 32 db + l % 32,
// h = l / 32) gets tile rows 16 cs + 4h .. + 3 (k 0..3) and 16 cs + 8 + 4h ..
// + 3 (k 4..7) of column d. Within 16 lanes, lane j addresses 4 halves of row
// 16 cs + 4h + j / 4 (+ 8) at column 32 db + 16 ((l / 16) % 2) + 4 (j % 4);
// lane i receives column 32 db + 16 ((l / 16) % 2) + i.
template <int CS>
__device__ __forceinline__ TrPair frag_tr(const _Float16* tile, const FragOff& fo, int db) {
    const unsigned base = unsigned(reinterpret_cast<uintptr_t>((lds_half*)tile));
    TrPair f;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                 : "=v"(f.lo) : "v"(base + fo.tr[db][0]), "i"(2048 * CS));
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                 : "=v"(f.hi) : "v"(base + fo.tr[db][1]), "i"(2048 * CS));
    return f;
}
// frag_tr for a slice index known once the loops are unrolled.
__device__ __forceinline__ TrPair frag_tr(const _Float16* tile, const FragOff& fo, int cs, int db) {
    switch (cs) {
    case 0: return frag_tr<0>(tile, fo, db);
    case 1: return frag_tr<1>(tile, fo, db);
    case 2: return frag_tr<2>(tile, fo, db);
    default: return frag_tr<3>(tile, fo, db);
    }
}

// Batch b's rows in a tensor of row stride `stride`: its first row, and the
// bytes up to the end of its last one (the buffer resource's length, so that
// rows at or past `length` read zeros).
struct Rows {
    int heads, length;
    __device__ size_t first(int b, int stride) const {
        return (size_t(b / heads) * length) * size_t(stride) + size_t(b % heads) * kHd;
    }
    __device__ unsigned bytes(int stride) const {
        return unsigned((size_t(length - 1) * stride + kHd) * 2);
    }
};

// The value of lane ^ 32 (the other half of the wave holds the same query).
__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32); }

// ---------------------------------------------------------------- forward

template <bool NEG>
__global__ void __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(3, 3)))
attn_forward(_Float16* __restrict__ out, float* __restrict__ lse, const _Float16* q,
             const _Float16* k, const _Float16* v, int batches, int length, float c, int heads,
             int in_stride, int o_stride, int round) {
    __shared__ __attribute__((aligned(16))) _Float16 lds[2 * 2 * kTile];   // [buf][K, V]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int fr = lane & 31, h = lane >> 5;
    const FragOff fo = frag_offsets(lane);
    const int nqb = (length + 127) / 128;
    const int rank = work_rank(int(blockIdx.x), round, int(gridDim.x));
    const int qb = nqb - 1 - rank / batches;      // longest blocks first
    const int b = rank % batches;
    const Rows rows{heads, length};
    const size_t in_first = rows.first(b, in_stride);
    const unsigned in_bytes = rows.bytes(in_stride);
    const auto rq = rsrc_of(q + in_first, in_bytes);
    const auto rk = rsrc_of(k + in_first, in_bytes);
    const auto rv = rsrc_of(v + in_first, in_bytes);
    const int q0 = qb * 128 + wave * 32;
    const int qi = q0 + fr;

    f16x8 qf[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
        qf[kk] = __builtin_bit_cast(
            f16x8, __builtin_amdgcn_raw_buffer_load_b128(
                       rq, unsigned((qi * in_stride + 16 * kk + 8 * h) * 2), 0, 0));

    float m = -INFINITY, l = 0.0f;
    f32x16 oacc[2] = {f32x16{}, f32x16{}};
    const int q_last = min(qb * 128 + 127, length - 1);
    const int nkb = q_last / 64 + 1;
    load_tile(lds, rk, 0, in_stride, wave, lane);
    load_tile(lds + kTile, rv, 0, in_stride, wave, lane);
    for (int j = 0; j < nkb; ++j) {
        wait_vmcnt<0>();
        block_sync();
        const _Float16* kt = lds + (j & 1) * 2 * kTile;
        const _Float16* vt = kt + kTile;
        if (j + 1 < nkb) {
            _Float16* nt = lds + ((j + 1) & 1) * 2 * kTile;
            load_tile(nt, rk, 64 * (j + 1), in_stride, wave, lane);
            load_tile(nt + kTile, rv, 64 * (j + 1), in_stride, wave, lane);
        }
        const int kbase = 64 * j;
        if (kbase > q0 + 31) continue;          // every key above every query of the wave
        f32x16 s[2] = {f32x16{}, f32x16{}};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int hb = 0; hb < 2; ++hb)
                s[hb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(frag_rows(kt, fo, hb, kk), qf[kk],
                                                               s[hb], 0, 0, 0);
        // The block's largest scaled score c s. The diagonal block scales
        // first and masks keys above the query (a uniform branch: the other
        // blocks skip the compares); the others take c max(s) (c min(s) for
        // c < 0: the max of -s, the negation a free source modifier), the
        // same value since rounding is monotonic, and scale inside the
        // exponent's FMA below.
        float mx = -INFINITY;
        float ce = c;   // what the exponent multiplies s by
        auto max_scores = [&](auto masked) {
#pragma unroll
            for (int hb = 0; hb < 2; ++hb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    if constexpr (masked) {
                        float t = s[hb][r] * c;
                        if (kbase + 32 * hb + 8 * (r >> 2) + 4 * h + (r & 3) > qi) t = -INFINITY;
                        s[hb][r] = t;
                        mx = fmaxf(mx, t);
                    } else {
                        mx = fmaxf(mx, NEG ? -s[hb][r] : s[hb][r]);
                    }
                }
        };
        if (kbase + 63 > q0) {
            max_scores(std::true_type{});
            ce = 1.0f;
        } else {
            max_scores(std::false_type{});
            mx *= NEG ? -c : c;
        }
        mx = fmaxf(mx, xor32(mx));
        // The running max m moves only when some lane's block max passes it
        // by more than kRescale (log2 units). Until then P = 2^(c s - m)
        // stays below 2^kRescale, well inside FP16, and O and l keep their
        // scale (the final O / l and lse = m + log2 l are the same quotient
        // and sum); the rescale of O and l is skipped.
        const float m_cand = fmaxf(m, mx);
        if (__any(m_cand > m + kRescale)) {
            const float alpha = __builtin_amdgcn_exp2f(m - m_cand);
            l *= alpha;
#pragma unroll
            for (int db = 0; db < 2; ++db) oacc[db] *= alpha;
            m = m_cand;
        }
        // P goes to FP16 as it is formed: 16-key slice cs is pf[cs].
        float sum = 0.0f;
        f16x8 pf[4];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[hb][r], ce, -m));
                pf[2 * hb + (r >> 3)][r & 7] = _Float16(p);
                sum += p;
            }
        sum += xor32(sum);
        l += sum;
        // O^T += V^T P^T, two 16-key slices at a time.
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            TrPair vf[2][2];
#pragma unroll
            for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
                for (int db = 0; db < 2; ++db) vf[c2][db] = frag_tr(vt, fo, 2 * half + c2, db);
            wait_lds();
#pragma unroll
            for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
                for (int db = 0; db < 2; ++db)
                    oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(join(vf[c2][db]),
                                                                      pf[2 * half + c2], oacc[db], 0,
                                                                      0, 0);
        }
    }
    wait_vmcnt<0>();
    if (qi < length) {
        const float inv = 1.0f / l;
        _Float16* orow = out + rows.first(b, o_stride) + size_t(qi) * o_stride;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const f16x4 o4 = {_Float16(oacc[db][4 * a] * inv), _Float16(oacc[db][4 * a + 1] * inv),
                                  _Float16(oacc[db][4 * a + 2] * inv), _Float16(oacc[db][4 * a + 3] * inv)};
                *reinterpret_cast<f16x4*>(orow + 32 * db + 8 * a + 4 * h) = o4;
            }
        if (h == 0) lse[size_t(b) * length + qi] = (m + __builtin_amdgcn_logf(l)) * kLn2;
    }
}

// ---------------------------------------------------------------- backward: dQ (and D)

__global__ void __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(3, 3)))
attn_backward_dq(_Float16* __restrict__ dq, float* __restrict__ dsum, const _Float16* q,
                 const _Float16* k, const _Float16* v, const _Float16* o, const _Float16* dout,
                 const float* lse, int batches, int length, float c, float scale, int heads,
                 int in_stride, int o_stride, int g_stride, int round) {
    __shared__ __attribute__((aligned(16))) _Float16 lds[2 * 2 * kTile];   // [buf][K, V]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int fr = lane & 31, h = lane >> 5;
    const FragOff fo = frag_offsets(lane);
    const int nqb = (length + 127) / 128;
    const int rank = work_rank(int(blockIdx.x), round, int(gridDim.x));
    const int qb = nqb - 1 - rank / batches;
    const int b = rank % batches;
    const Rows rows{heads, length};
    const size_t in_first = rows.first(b, in_stride), o_first = rows.first(b, o_stride);
    const unsigned in_bytes = rows.bytes(in_stride), o_bytes = rows.bytes(o_stride);
    const auto rq = rsrc_of(q + in_first, in_bytes);
    const auto rk = rsrc_of(k + in_first, in_bytes);
    const auto rv = rsrc_of(v + in_first, in_bytes);
    const auto ro = rsrc_of(o + o_first, o_bytes);
    const auto rdo = rsrc_of(dout + o_first, o_bytes);
    const int q0 = qb * 128 + wave * 32;
    const int qi = q0 + fr;

    f16x8 qf[4], df[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const unsigned in_off = unsigned((qi * in_stride + 16 * kk + 8 * h) * 2);
        const unsigned o_off = unsigned((qi * o_stride + 16 * kk + 8 * h) * 2);
        qf[kk] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rq, in_off, 0, 0));
        df[kk] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rdo, o_off, 0, 0));
    }
    // D = sum_d dO * O for this lane's query: halves 32 h .. 32 h + 31 here,
    // the rest from lane ^ 32.
    float dd = 0.0f;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const unsigned off = unsigned((qi * o_stride + 32 * h + 8 * kk) * 2);
        const f16x8 ov = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(ro, off, 0, 0));
        const f16x8 gv = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rdo, off, 0, 0));
#pragma unroll
        for (int e = 0; e < 8; ++e) dd = __builtin_fmaf(float(gv[e]), float(ov[e]), dd);
    }
    dd += xor32(dd);
    const float lse2 = qi < length ? lse[size_t(b) * length + qi] * kLog2e : 0.0f;
    if (qi < length && h == 0) dsum[size_t(b) * length + qi] = dd;

    f32x16 acc[2] = {f32x16{}, f32x16{}};   // dQ^T[d][q]
    const int q_last = min(qb * 128 + 127, length - 1);
    const int nkb = q_last / 64 + 1;
    load_tile(lds, rk, 0, in_stride, wave, lane);
    load_tile(lds + kTile, rv, 0, in_stride, wave, lane);
    for (int j = 0; j < nkb; ++j) {
        wait_vmcnt<0>();
        block_sync();
        const _Float16* kt = lds + (j & 1) * 2 * kTile;
        const _Float16* vt = kt + kTile;
        if (j + 1 < nkb) {
            _Float16* nt = lds + ((j + 1) & 1) * 2 * kTile;
            load_tile(nt, rk, 64 * (j + 1), in_stride, wave, lane);
            load_tile(nt + kTile, rv, 64 * (j + 1), in_stride, wave, lane);
        }
        const int kbase = 64 * j;
        if (kbase > q0 + 31) continue;
        // The block in two halves of 32 keys, each through all of its
        // products before the next (fewer registers live at once).
        const bool masked = kbase + 63 > q0;
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            f32x16 s = {}, dp = {};
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                s = __builtin_amdgcn_mfma_f32_32x32x16_f16(frag_rows(kt, fo, hb, kk), qf[kk], s, 0,
                                                           0, 0);
                dp = __builtin_amdgcn_mfma_f32_32x32x16_f16(frag_rows(vt, fo, hb, kk), df[kk], dp,
                                                            0, 0, 0);
            }
            // dS^T = P (dP - D) goes to FP16 as it is formed: 16-key slice c2
            // of the half is sf[c2]. Keys above the query are masked in the
            // diagonal block only.
            f16x8 sf[2];
            auto form_ds = [&](auto mask) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float p = __builtin_amdgcn_exp2f(s[r] * c - lse2);
                    if constexpr (mask)
                        if (kbase + 32 * hb + 8 * (r >> 2) + 4 * h + (r & 3) > qi) p = 0.0f;
                    sf[r >> 3][r & 7] = _Float16(p * (dp[r] - dd));
                }
            };
            if (masked) form_ds(std::true_type{});
            else form_ds(std::false_type{});
            // dQ^T += K^T dS^T over the half's 32 keys.
            TrPair kf[2][2];
#pragma unroll
            for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
                for (int db = 0; db < 2; ++db) kf[c2][db] = frag_tr(kt, fo, 2 * hb + c2, db);
            wait_lds();
#pragma unroll
            for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
                for (int db = 0; db < 2; ++db)
                    acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(join(kf[c2][db]), sf[c2],
                                                                     acc[db], 0, 0, 0);
        }
    }
    wait_vmcnt<0>();
    if (qi < length) {
        _Float16* row = dq + rows.first(b, g_stride) + size_t(qi) * g_stride;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const f16x4 o4 = {_Float16(acc[db][4 * a] * scale), _Float16(acc[db][4 * a + 1] * scale),
                                  _Float16(acc[db][4 * a + 2] * scale), _Float16(acc[db][4 * a + 3] * scale)};
                *reinterpret_cast<f16x4*>(row + 32 * db + 8 * a + 4 * h) = o4;
            }
    }
}

// ---------------------------------------------------------------- backward: dK, dV

// A workgroup owns 128 keys (32 per wave) and walks the query blocks of 64 at
// or after its first key. S[q][key] = Q K^T with queries as the MFMA's rows:
// a lane holds one key (lane % 32) and 16 queries per 32-query block, whose
// lse and D come from the block's LDS copy.
__global__ void __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
attn_backward_dkdv(_Float16* __restrict__ dk, _Float16* __restrict__ dv, const _Float16* q,
                   const _Float16* k, const _Float16* v, const _Float16* dout, const float* lse,
                   const float* dsum, int batches, int length, float c, float scale, int heads,
                   int in_stride, int o_stride, int g_stride, int round) {
    // [buf][Q tile, dO tile] then [buf][lse2 64, D 64].
    __shared__ __attribute__((aligned(16))) _Float16 lds[2 * 2 * kTile];
    __shared__ __attribute__((aligned(16))) float rowstat[2][2][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int fr = lane & 31, h = lane >> 5;
    const FragOff fo = frag_offsets(lane);
    const int nkb = (length + 127) / 128;
    const int rank = work_rank(int(blockIdx.x), round, int(gridDim.x));
    const int kb = rank / batches;                // earliest keys have the most queries
    const int b = rank % batches;
    const Rows rows{heads, length};
    const size_t in_first = rows.first(b, in_stride);
    const unsigned in_bytes = rows.bytes(in_stride);
    const auto rq = rsrc_of(q + in_first, in_bytes);
    const auto rk = rsrc_of(k + in_first, in_bytes);
    const auto rv = rsrc_of(v + in_first, in_bytes);
    const auto rdo = rsrc_of(dout + rows.first(b, o_stride), rows.bytes(o_stride));
    const float* lse_b = lse + size_t(b) * length;
    const float* d_b = dsum + size_t(b) * length;
    (void)nkb;
    const int k0 = kb * 128 + wave * 32;      // this wave's first key
    const int ki = k0 + fr;                   // this lane's key

    f16x8 kf[4], vf[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const unsigned off = unsigned((ki * in_stride + 16 * kk + 8 * h) * 2);
        kf[kk] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
        vf[kk] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
    }
    f32x16 dka[2] = {f32x16{}, f32x16{}}, dva[2] = {f32x16{}, f32x16{}};   // dK^T, dV^T [d][key]
    const int qs0 = (kb * 128) / 64;          // first query block
    const int nqb = (length + 63) / 64;
    // The block's tiles, and (wave 0, one query a lane) its lse in log2 units
    // and D. The two register loads go out first, so that waiting for them
    // before their LDS writes does not wait for the tiles.
    auto stage_rows = [&](int buf, int qblk) {
        _Float16* t = lds + buf * 2 * kTile;
        const int qq = 64 * qblk + lane;
        float lv = 0.0f, dv0 = 0.0f;
        if (wave == 0 && qq < length) {
            lv = lse_b[qq];
            dv0 = d_b[qq];
        }
        load_tile(t, rq, 64 * qblk, in_stride, wave, lane);
        load_tile(t + kTile, rdo, 64 * qblk, o_stride, wave, lane);
        if (wave == 0) {
            rowstat[buf][0][lane] = lv * kLog2e;
            rowstat[buf][1][lane] = dv0;
        }
    };
    stage_rows(0, qs0);
    for (int qblk = qs0; qblk < nqb; ++qblk) {
        const int buf = (qblk - qs0) & 1;
        wait_vmcnt<0>();
        __syncthreads();
        const _Float16* qt = lds + buf * 2 * kTile;
        const _Float16* gt = qt + kTile;
        const float* l2 = rowstat[buf][0];
        const float* dd = rowstat[buf][1];
        if (qblk + 1 < nqb) stage_rows(buf ^ 1, qblk + 1);
        const int qbase = 64 * qblk;
        if (qbase + 63 < k0) continue;        // every query of the block precedes every key of the wave
        // The block in two halves of 32 queries, each through all of its
        // products before the next (fewer registers live at once).
        const bool masked = qbase < k0 + 31 || qbase + 63 >= length;
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) {
            f32x16 s = {}, dp = {};
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                s = __builtin_amdgcn_mfma_f32_32x32x16_f16(frag_rows(qt, fo, qh, kk), kf[kk],
                                                           s, 0, 0, 0);
                dp = __builtin_amdgcn_mfma_f32_32x32x16_f16(frag_rows(gt, fo, qh, kk), vf[kk],
                                                            dp, 0, 0, 0);
            }
            // P and dS = P (dP - D) go to FP16 as they are formed: 16-query
            // slice c2 of the half is MFMA operand pf[c2] / sf[c2]. Queries
            // before the key, and past the sequence, are masked only in the
            // blocks that hold any (a uniform branch).
            f16x8 pf[2], sf[2];
            auto form_p_ds = [&](auto mask) {
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    const int qr = 32 * qh + 8 * a + 4 * h;   // query row in the block, + e
                    const f32x4 l4 = *reinterpret_cast<const f32x4*>(l2 + qr);
                    const f32x4 d4 = *reinterpret_cast<const f32x4*>(dd + qr);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int r = 4 * a + e;
                        float p = __builtin_amdgcn_exp2f(s[r] * c - l4[e]);
                        if constexpr (mask) {
                            if (ki > qbase + qr + e) p = 0.0f;
                            if (qbase + qr + e >= length) p = 0.0f;
                        }
                        const int c2 = a >> 1, at = 4 * (a & 1) + e;
                        pf[c2][at] = _Float16(p);
                        sf[c2][at] = _Float16(p * (dp[r] - d4[e]));
                    }
                }
            };
            if (masked) form_p_ds(std::true_type{});
            else form_p_ds(std::false_type{});
            // dV^T += dO^T P^T and dK^T += Q^T dS^T over the half's 32 queries.
            TrPair gtr[2][2], qtr[2][2];
#pragma unroll
            for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
                for (int db = 0; db < 2; ++db) {
                    gtr[c2][db] = frag_tr(gt, fo, 2 * qh + c2, db);
                    qtr[c2][db] = frag_tr(qt, fo, 2 * qh + c2, db);
                }
            wait_lds();
#pragma unroll
            for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
                for (int db = 0; db < 2; ++db) {
                    dva[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(join(gtr[c2][db]), pf[c2],
                                                                     dva[db], 0, 0, 0);
                    dka[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(join(qtr[c2][db]), sf[c2],
                                                                     dka[db], 0, 0, 0);
                }
        }
    }
    wait_vmcnt<0>();
    if (ki < length) {
        const size_t g_first = rows.first(b, g_stride);
        _Float16* krow = dk + g_first + size_t(ki) * g_stride;
        _Float16* vrow = dv + g_first + size_t(ki) * g_stride;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const f16x4 k4 = {_Float16(dka[db][4 * a] * scale), _Float16(dka[db][4 * a + 1] * scale),
                                  _Float16(dka[db][4 * a + 2] * scale), _Float16(dka[db][4 * a + 3] * scale)};
                const f16x4 v4 = {_Float16(dva[db][4 * a]), _Float16(dva[db][4 * a + 1]),
                                  _Float16(dva[db][4 * a + 2]), _Float16(dva[db][4 * a + 3])};
                *reinterpret_cast<f16x4*>(krow + 32 * db + 8 * a + 4 * h) = k4;
                *reinterpret_cast<f16x4*>(vrow + 32 * db + 8 * a + 4 * h) = v4;
            }
    }
}

// Heads divide the batches, every stride holds a 64-half row, and buffer
// offsets (32-bit bytes) reach every row.
// work_rank's run: the CU count; the "attn_order" override "0" keeps plain
// longest-first order (A/B runs).
int order_round() {
    if (tuning_off(Tune::kAttnOrder)) return 0;
    int cus = 0;
    if (device_cus(&cus) != hipSuccess || cus <= 0) return 0;
    return cus;
}

bool layout_fits(const AttnLayout& l, size_t batches, size_t length) {
    if (l.heads < 1 || batches % size_t(l.heads) != 0 || length == 0) return false;
    for (int s : {l.qkv_stride, l.o_stride, l.grad_stride})
        if (s < kHd || length * size_t(s) >= (size_t{1} << 30)) return false;
    return true;
}

}  // namespace

hipError_t launch_attention_forward(void* out, void* lse, const void* q, const void* k,
                                    const void* v, size_t batches, size_t length, float scale,
                                    hipStream_t stream, AttnLayout layout) {
    if (!layout_fits(layout, batches, length)) return hipErrorInvalidValue;
    const unsigned blocks = unsigned(batches * ((length + 127) / 128));
    auto* const kernel = scale < 0.0f ? attn_forward<true> : attn_forward<false>;
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kAttnThreads), 0, stream,
                       static_cast<_Float16*>(out), static_cast<float*>(lse),
                       static_cast<const _Float16*>(q), static_cast<const _Float16*>(k),
                       static_cast<const _Float16*>(v), int(batches), int(length), scale * kLog2e,
                       layout.heads, layout.qkv_stride, layout.o_stride, order_round());
    return hipGetLastError();
}

hipError_t launch_attention_backward(void* dq, void* dk, void* dv, const void* dout, const void* q,
                                     const void* k, const void* v, const void* o, const void* lse,
                                     void* dsum, size_t batches, size_t length, float scale,
                                     hipStream_t stream, AttnLayout layout) {
    if (!layout_fits(layout, batches, length)) return hipErrorInvalidValue;
    const unsigned blocks = unsigned(batches * ((length + 127) / 128));
    hipLaunchKernelGGL(attn_backward_dq, dim3(blocks), dim3(kAttnThreads), 0, stream,
                       static_cast<_Float16*>(dq), static_cast<float*>(dsum),
                       static_cast<const _Float16*>(q), static_cast<const _Float16*>(k),
                       static_cast<const _Float16*>(v), static_cast<const _Float16*>(o),
                       static_cast<const _Float16*>(dout), static_cast<const float*>(lse),
                       int(batches), int(length), scale * kLog2e, scale, layout.heads,
                       layout.qkv_stride, layout.o_stride, layout.grad_stride, order_round());
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    hipLaunchKernelGGL(attn_backward_dkdv, dim3(blocks), dim3(kAttnThreads), 0, stream,
                       static_cast<_Float16*>(dk), static_cast<_Float16*>(dv),
                       static_cast<const _Float16*>(q), static_cast<const _Float16*>(k),
                       static_cast<const _Float16*>(v), static_cast<const _Float16*>(dout),
                       static_cast<const float*>(lse), static_cast<const float*>(dsum),
                       int(batches), int(length), scale * kLog2e, scale, layout.heads,
                       layout.qkv_stride, layout.o_stride, layout.grad_stride, order_round());
    return hipGetLastError();
}

}  // namespace flint
