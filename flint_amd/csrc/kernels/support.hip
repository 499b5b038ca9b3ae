// Data-movement kernels around the hot path: byte copy, FP32 -> FP16, the
// attention heads' split / merge, and the embedding's forward and backward
// passes. All are HBM-bound; every one moves 16-byte vectors where the
// alignment the ABI promises allows it.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>

#include "common/common.h"
#include "common/tuning.h"
#include "kernels/kernels.h"
#include "kernels/reduce_common.h"

#pragma clang fp contract(off)

namespace flint {
namespace {

constexpr unsigned kMaxGrid = 1u << 20;

unsigned grid_for(size_t items, unsigned threads) {
    return unsigned(std::clamp<size_t>((items + threads - 1) / threads, 1, kMaxGrid));
}

// ------------------------------------------------------------------- copy

__global__ void __launch_bounds__(256)
copy_vec(u4* __restrict__ dst, const u4* __restrict__ src, size_t vecs) {
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < vecs; i += size_t(gridDim.x) * 256)
        dst[i] = src[i];
}

__global__ void __launch_bounds__(256)
copy_bytes(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, size_t bytes) {
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < bytes;
         i += size_t(gridDim.x) * 256)
        dst[i] = src[i];
}

__global__ void __launch_bounds__(256)
fill_zero_vec(u4* __restrict__ dst, size_t vecs) {
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < vecs; i += size_t(gridDim.x) * 256)
        dst[i] = u4{0u, 0u, 0u, 0u};
}

__global__ void __launch_bounds__(256)
fill_zero_bytes(uint8_t* __restrict__ dst, size_t bytes) {
    for (size_t i = threadIdx.x; i < bytes; i += 256) dst[i] = 0;
}

// ------------------------------------------------------------ FP32 -> FP16

__global__ void __launch_bounds__(256)
fp32_to_fp16(_Float16* __restrict__ y, const float* __restrict__ x, size_t count) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const size_t quads = count / 4;
    const size_t stride = size_t(gridDim.x) * 256;
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < quads; i += stride) {
        const f4 v = reinterpret_cast<const f4*>(x)[i];
        reinterpret_cast<h4*>(y)[i] = h4{_Float16(v[0]), _Float16(v[1]), _Float16(v[2]),
                                         _Float16(v[3])};
    }
    // The last count % 4 values, one thread each.
    if (blockIdx.x == 0 && threadIdx.x < count - quads * 4) {
        const size_t i = quads * 4 + threadIdx.x;
        y[i] = _Float16(x[i]);
    }
}

// ------------------------------------------------------------ heads

// One thread per 16-byte chunk of the heads layout [b][h][t][c].
__global__ void __launch_bounds__(256)
heads_move(h8* __restrict__ y, const h8* __restrict__ x, size_t rows, size_t length, int heads,
           int head_chunks, int row_chunks, int first_chunk, int merge) {
    const size_t total = rows * size_t(heads) * head_chunks;
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < total;
         i += size_t(gridDim.x) * 256) {
        const int c = int(i % head_chunks);
        size_t rest = i / head_chunks;
        const size_t t = rest % length;
        rest /= length;
        const int h = int(rest % heads);
        const size_t b = rest / heads;
        const size_t row_at = (b * length + t) * row_chunks + first_chunk + h * head_chunks + c;
        if (merge) y[row_at] = x[i];
        else y[i] = x[row_at];
    }
}

// The model's attention: the three parts (q, k, v) of a [rows][3 * width]
// matrix to (split) or from (merge) three heads layouts in one pass, the same
// moves as three heads_move calls with first = 0, width, 2 * width. Index
// arithmetic is 32-bit (the caller checks that the element count fits).
__global__ void __launch_bounds__(256)
heads_move3(h8* wide, h8* p0, h8* p1, h8* p2, unsigned rows, unsigned length, unsigned heads,
            unsigned head_chunks, int merge) {
    const unsigned per_part = rows * heads * head_chunks;
    const unsigned row_chunks = 3 * heads * head_chunks;
    for (unsigned i = blockIdx.x * 256 + threadIdx.x; i < 3 * per_part; i += gridDim.x * 256) {
        const unsigned part = i / per_part;
        const unsigned j = i - part * per_part;
        const unsigned c = j % head_chunks;
        unsigned rest = j / head_chunks;
        const unsigned t = rest % length;
        rest /= length;
        const unsigned h = rest % heads;
        const unsigned b = rest / heads;
        const size_t at = size_t(b * length + t) * row_chunks + part * heads * head_chunks +
                          h * head_chunks + c;
        h8* const p = part == 0 ? p0 : (part == 1 ? p1 : p2);
        if (merge) wide[at] = p[j];
        else p[j] = wide[at];
    }
}

// ------------------------------------------------------------ embedding fwd

// One wave per row: x[r] = wte[tokens[r]] + wpe[r % length], one FP32 add each.
__global__ void __launch_bounds__(256)
embedding_forward(float* __restrict__ x, const uint16_t* __restrict__ tokens,
                  const float* __restrict__ wte, const float* __restrict__ wpe, size_t rows,
                  size_t length, size_t width) {
    const size_t quads = width / 4;
    for (size_t row = size_t(blockIdx.x) * 4 + (threadIdx.x >> 6); row < rows;
         row += size_t(gridDim.x) * 4) {
        const size_t tok = tokens[row];
        const f4* a = reinterpret_cast<const f4*>(wte + tok * width);
        const f4* b = reinterpret_cast<const f4*>(wpe + (row % length) * width);
        f4* o = reinterpret_cast<f4*>(x + row * width);
        for (size_t q = threadIdx.x & 63; q < quads; q += 64) o[q] = a[q] + b[q];
    }
}

// ------------------------------------------------------------ embedding bwd

constexpr int kSortTile = 2048;   // rows per sort workgroup
constexpr int kDigits = 256;      // 8-bit digits, two passes over 16-bit tokens

// Per tile, per digit counts, stored digit-major (counts[d * tiles + tile]) so
// one exclusive scan over the array gives every (tile, digit) its output base.
__global__ void __launch_bounds__(256)
sort_count(unsigned* __restrict__ counts, const uint16_t* __restrict__ tokens, size_t rows,
           int shift, unsigned tiles) {
    __shared__ unsigned hist[kDigits];
    hist[threadIdx.x] = 0;
    __syncthreads();
    const size_t base = size_t(blockIdx.x) * kSortTile;
    for (int i = threadIdx.x; i < kSortTile; i += 256) {
        const size_t r = base + i;
        if (r < rows) atomicAdd(&hist[(tokens[r] >> shift) & 255], 1u);
    }
    __syncthreads();
    counts[size_t(threadIdx.x) * tiles + blockIdx.x] = hist[threadIdx.x];
}

// Exclusive scan of n values in place, one workgroup of 1024 threads, each
// owning a contiguous segment.
__global__ void __launch_bounds__(1024)
scan_exclusive(unsigned* __restrict__ v, size_t n) {
    __shared__ unsigned part[1024];
    const size_t per = (n + 1023) / 1024;
    const size_t lo = std::min(n, size_t(threadIdx.x) * per);
    const size_t hi = std::min(n, lo + per);
    unsigned s = 0;
    for (size_t i = lo; i < hi; ++i) s += v[i];
    part[threadIdx.x] = s;
    __syncthreads();
    for (int off = 1; off < 1024; off *= 2) {
        const unsigned add = threadIdx.x >= unsigned(off) ? part[threadIdx.x - off] : 0u;
        __syncthreads();
        part[threadIdx.x] += add;
        __syncthreads();
    }
    unsigned run = part[threadIdx.x] - s;
    for (size_t i = lo; i < hi; ++i) {
        const unsigned c = v[i];
        v[i] = run;
        run += c;
    }
}

// Stable scatter of one 8-bit pass. Wave w of a tile owns rows
// [tile*2048 + 512 w, +512) and walks them 64 at a time in order; a row's rank
// among same-digit rows of its round comes from 8 ballots.
__global__ void __launch_bounds__(256)
sort_scatter(uint16_t* __restrict__ out_tokens, unsigned* __restrict__ out_rows,
             const uint16_t* __restrict__ in_tokens, const unsigned* __restrict__ in_rows,
             const unsigned* __restrict__ scanned, size_t rows, int shift, unsigned tiles) {
    __shared__ unsigned wcount[4][kDigits];
    __shared__ unsigned run[4][kDigits];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    for (int w = 0; w < 4; ++w) wcount[w][threadIdx.x] = 0;
    __syncthreads();
    const size_t wave_base = size_t(blockIdx.x) * kSortTile + size_t(wave) * 512;
    for (int i = lane; i < 512; i += 64) {
        const size_t r = wave_base + i;
        if (r < rows) atomicAdd(&wcount[wave][(in_tokens[r] >> shift) & 255], 1u);
    }
    __syncthreads();
    {
        const int d = threadIdx.x;
        unsigned b = scanned[size_t(d) * tiles + blockIdx.x];
        for (int w = 0; w < 4; ++w) {
            run[w][d] = b;
            b += wcount[w][d];
        }
    }
    __syncthreads();
    for (int round = 0; round < 8; ++round) {
        const size_t r = wave_base + size_t(round) * 64 + lane;
        const bool valid = r < rows;
        const uint16_t tok = valid ? in_tokens[r] : 0;
        const unsigned row_id = valid ? (in_rows ? in_rows[r] : unsigned(r)) : 0u;
        const int digit = (tok >> shift) & 255;
        unsigned long long match = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 8; ++bit) {
            const bool set = (digit >> bit) & 1;
            const unsigned long long b = __ballot(set);
            match &= set ? b : ~b;
        }
        const unsigned long long below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
        const unsigned rank = unsigned(__popcll(match & below));
        if (valid) {
            const unsigned pos = run[wave][digit] + rank;
            out_tokens[pos] = tok;
            out_rows[pos] = row_id;
        }
        // The group's last lane advances the digit's running base.
        const bool last = valid && (match >> lane) == 1ull;
        __builtin_amdgcn_wave_barrier();
        if (last) run[wave][digit] += unsigned(__popcll(match));
        __builtin_amdgcn_wave_barrier();
    }
}

// Both 8-bit passes of the stable token sort in one workgroup, in LDS, for up
// to kBlockSortRows rows: the order sort_count / scan_exclusive /
// sort_scatter give (stable by token, rows ascending within a token), in one
// launch instead of six. Wave w owns rows [w p, (w + 1) p), p a multiple of
// 64; per pass it counts its digits, one scan over (digit, wave) in
// digit-major order gives each its base, and the wave scatters its rows in
// order, 64 at a time, ranked among equal digits by ballots.
constexpr int kBlockSortRows = 8192;

__device__ __forceinline__ void sort_block_body(uint16_t* __restrict__ out_tokens,
                                                unsigned* __restrict__ out_rows,
                                                const uint16_t* __restrict__ tokens, int rows) {
    __shared__ uint16_t key[2][kBlockSortRows];
    __shared__ unsigned idx[2][kBlockSortRows];
    __shared__ unsigned cnt[16][kDigits];
    __shared__ unsigned wsum[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int per_wave = ((rows + 15) / 16 + 63) / 64 * 64;
    const int lo = wave * per_wave, hi = min(rows, lo + per_wave);
    for (int i = tid; i < rows; i += 1024) {
        key[0][i] = tokens[i];
        idx[0][i] = unsigned(i);
    }
    for (int pass = 0; pass < 2; ++pass) {
        const int src = pass, dst = pass ^ 1, shift = 8 * pass;
        for (int i = tid; i < 16 * kDigits; i += 1024) cnt[i / kDigits][i % kDigits] = 0;
        __syncthreads();
        for (int r = lo + lane; r < hi; r += 64) atomicAdd(&cnt[wave][(key[src][r] >> shift) & 255], 1u);
        __syncthreads();
        {
            // Thread t holds entries 4t .. 4t + 3 of the digit-major order:
            // digit t / 4, waves 4 (t % 4) .. + 3.
            const int d = tid >> 2, w0 = (tid & 3) * 4;
            unsigned c[4], own = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                c[k] = cnt[w0 + k][d];
                own += c[k];
            }
            unsigned v = own;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const unsigned t = __shfl_up(v, o, 64);
                if (lane >= o) v += t;
            }
            if (lane == 63) wsum[wave] = v;
            __syncthreads();
            unsigned run = v - own;
            for (int w = 0; w < wave; ++w) run += wsum[w];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                cnt[w0 + k][d] = run;
                run += c[k];
            }
        }
        __syncthreads();
        for (int base = lo; base < lo + per_wave; base += 64) {
            const int r = base + lane;
            const bool valid = r < hi;
            const uint16_t tok = valid ? key[src][r] : 0;
            const unsigned row_id = valid ? idx[src][r] : 0u;
            const int digit = (tok >> shift) & 255;
            unsigned long long match = __ballot(valid);
#pragma unroll
            for (int bit = 0; bit < 8; ++bit) {
                const bool set = (digit >> bit) & 1;
                const unsigned long long b = __ballot(set);
                match &= set ? b : ~b;
            }
            const unsigned long long below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
            const unsigned rank = unsigned(__popcll(match & below));
            if (valid) {
                const unsigned pos = cnt[wave][digit] + rank;
                key[dst][pos] = tok;
                idx[dst][pos] = row_id;
            }
            // The group's last lane advances the digit's base.
            const bool last = valid && (match >> lane) == 1ull;
            __builtin_amdgcn_wave_barrier();
            if (last) cnt[wave][digit] += unsigned(__popcll(match));
            __builtin_amdgcn_wave_barrier();
        }
        __syncthreads();
    }
    for (int i = tid; i < rows; i += 1024) {
        out_tokens[i] = key[0][i];
        out_rows[i] = idx[0][i];
    }
}

__global__ void __launch_bounds__(1024)
sort_tokens_block(uint16_t* __restrict__ out_tokens, unsigned* __restrict__ out_rows,
                  const uint16_t* __restrict__ tokens, int rows) {
    sort_block_body(out_tokens, out_rows, tokens, rows);
}


// offsets[v] = number of sorted tokens below v, v = 0..vocab (binary search).
__global__ void __launch_bounds__(256)
token_offsets(unsigned* __restrict__ offsets, const uint16_t* __restrict__ sorted, size_t rows,
              unsigned vocab) {
    const unsigned v = blockIdx.x * 256 + threadIdx.x;
    if (v > vocab) return;
    size_t lo = 0, hi = rows;
    while (lo < hi) {
        const size_t mid = (lo + hi) / 2;
        if (sorted[mid] < v) lo = mid + 1;
        else hi = mid;
    }
    offsets[v] = unsigned(lo);
}

// dwte[v][c..c+3]: compensated sum of dx rows with token v in ascending row
// order. Grid (vocab, column tiles of 256); a thread owns 4 columns.
__global__ void __launch_bounds__(64)
embedding_words(float* __restrict__ dwte, const float* __restrict__ dx,
                const unsigned* __restrict__ sorted_rows, const unsigned* __restrict__ offsets,
                size_t width, int accumulate) {
    const size_t v = blockIdx.x;
    const size_t col = (size_t(blockIdx.y) * 64 + threadIdx.x) * 4;
    if (col >= width) return;
    const unsigned lo = offsets[v];
    const unsigned hi = offsets[v + 1];
    f4* out = reinterpret_cast<f4*>(dwte + v * width + col);
    if (lo == hi) {
        if (!accumulate) *out = f4{0.0f, 0.0f, 0.0f, 0.0f};
        return;
    }
    Comp s[4];
    for (unsigned i = lo; i < hi; ++i) {
        const f4 d = *reinterpret_cast<const f4*>(dx + size_t(sorted_rows[i]) * width + col);
#pragma unroll
        for (int j = 0; j < 4; ++j) comp_add(s[j], d[j]);
    }
    f4 r;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        r[j] = __builtin_isfinite(s[j].sum) ? add_rn(s[j].sum, s[j].error) : s[j].sum;
    if (accumulate) {
        const f4 old = *out;
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = add_rn(old[j], r[j]);
    }
    *out = r;
}

// The same sums when they add into dwte: only the rows of tokens that occur
// are touched, so a workgroup per sorted position (256 columns of it) works
// if the position starts a run of equal tokens and leaves at once otherwise;
// the run's rows come in ascending order (the sort is stable).
__global__ void __launch_bounds__(64)
embedding_runs(float* __restrict__ dwte, const float* __restrict__ dx,
               const uint16_t* __restrict__ sorted_tokens, const unsigned* __restrict__ sorted_rows,
               size_t rows, size_t width) {
    const size_t i = blockIdx.x;
    const uint16_t v = sorted_tokens[i];
    if (i > 0 && sorted_tokens[i - 1] == v) return;
    const size_t col = (size_t(blockIdx.y) * 64 + threadIdx.x) * 4;
    if (col >= width) return;
    Comp s[4];
    for (size_t k = i; k < rows && sorted_tokens[k] == v; ++k) {
        const f4 d = *reinterpret_cast<const f4*>(dx + size_t(sorted_rows[k]) * width + col);
#pragma unroll
        for (int j = 0; j < 4; ++j) comp_add(s[j], d[j]);
    }
    f4* out = reinterpret_cast<f4*>(dwte + size_t(v) * width + col);
    const f4 old = *out;
    f4 r;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        r[j] = add_rn(old[j], __builtin_isfinite(s[j].sum) ? add_rn(s[j].sum, s[j].error) : s[j].sum);
    *out = r;
}

struct EmbLayout {
    size_t partials, sorted_tokens, sorted_rows, offsets, pass_tokens, pass_rows, counts, bytes;
};

size_t align16(size_t b) { return (b + 15) / 16 * 16; }

// Workspace layout, region by region (sizes as ref src/kernels/embedding_backward.cuh:44-88
// fixes them, since the workspace size is part of the ABI): position partials,
// sorted tokens, sorted rows, token offsets, first-pass tokens and rows,
// per-tile digit counts.
EmbLayout emb_layout(size_t sequences, size_t length, size_t vocab, size_t width) {
    const size_t rows = sequences * length;
    const size_t tiles = (rows + kSortTile - 1) / kSortTile;
    EmbLayout l{};
    size_t at = align16(bias_gradient_workspace(sequences, length * width));
    l.partials = 0;
    l.sorted_tokens = at;
    at += align16(rows * 2);
    l.sorted_rows = at;
    at += align16(rows * 4);
    l.offsets = at;
    at += align16((vocab + 1) * 4);
    l.pass_tokens = at;
    at += align16(rows * 2);
    l.pass_rows = at;
    at += align16(rows * 4);
    l.counts = at;
    at += align16(tiles * kDigits * 4);
    l.bytes = at;
    return l;
}

constexpr int kPhasesF32 = 8;   // row phases of the column-sum order

// Column partials of an FP32 matrix (bias-gradient order), for dwpe.
__global__ void __launch_bounds__(64)
column_partials_f32(float* __restrict__ partial, const float* __restrict__ dy, size_t rows,
                    size_t cols) {
    __shared__ float sums[8][8][8];
    __shared__ float errs[8][8][8];
    const int px = threadIdx.x & 7;
    const int ph = threadIdx.x >> 3;
    const size_t pieces = cols / 8;
    const size_t piece = size_t(blockIdx.x) * 8 + px;
    const size_t first = size_t(blockIdx.y) * 256;
    const size_t end = rows - first < 256 ? rows : first + 256;
    Comp acc[8];
    if (piece < pieces) {
        for (size_t r = first + ph; r < end; r += 8) {
            const f4* p = reinterpret_cast<const f4*>(dy + r * cols + piece * 8);
            const f4 a = p[0], b = p[1];
#pragma unroll
            for (int j = 0; j < 4; ++j) comp_add(acc[j], a[j]);
#pragma unroll
            for (int j = 0; j < 4; ++j) comp_add(acc[j + 4], b[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        sums[ph][px][j] = acc[j].sum;
        errs[ph][px][j] = acc[j].error;
    }
    __syncthreads();
    if (ph != 0 || piece >= pieces) return;
    for (int o = 1; o < 8; ++o) {
#pragma unroll
        for (int j = 0; j < 8; ++j) comp_merge(acc[j], sums[o][px][j], errs[o][px][j]);
    }
    float* srow = partial + size_t(blockIdx.y) * 2 * cols + piece * 8;
    f4* s4 = reinterpret_cast<f4*>(srow);
    f4* e4 = reinterpret_cast<f4*>(srow + cols);
    s4[0] = f4{acc[0].sum, acc[1].sum, acc[2].sum, acc[3].sum};
    s4[1] = f4{acc[4].sum, acc[5].sum, acc[6].sum, acc[7].sum};
    e4[0] = f4{acc[0].error, acc[1].error, acc[2].error, acc[3].error};
    e4[1] = f4{acc[4].error, acc[5].error, acc[6].error, acc[7].error};
}

// The same column sums for at most one chunk of rows (rows <= 256), merged and
// finished in one launch: a thread owns 4 columns, runs the 8 row phases as
// independent chains (row 8k + p to phase p), lets phase 0 merge phases 1..7
// in order, and then applies what column_finish does to a single chunk -- lane
// 0 merges it into an empty sum and the 32-lane butterfly merges five empty
// lanes' sums into it.
__device__ __forceinline__ void column_sums_quad(float* __restrict__ out,
                                                 const float* __restrict__ dy, int rows,
                                                 size_t cols, int accumulate, size_t quad) {
    if (quad >= cols / 4) return;
    Comp acc[kPhasesF32][4];
    for (int k = 0; k < rows; k += kPhasesF32) {
        f4 v[kPhasesF32];
#pragma unroll
        for (int p = 0; p < kPhasesF32; ++p)
            if (k + p < rows) v[p] = reinterpret_cast<const f4*>(dy + size_t(k + p) * cols)[quad];
#pragma unroll
        for (int p = 0; p < kPhasesF32; ++p) {
            if (k + p < rows) {
#pragma unroll
                for (int j = 0; j < 4; ++j) comp_add(acc[p][j], v[p][j]);
            }
        }
    }
    f4 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        for (int p = 1; p < kPhasesF32; ++p) comp_merge(acc[0][j], acc[p][j].sum, acc[p][j].error);
        Comp t;
        comp_merge(t, acc[0][j].sum, acc[0][j].error);
        for (int step = 0; step < 5; ++step) comp_merge(t, 0.0f, 0.0f);
        r[j] = __builtin_isfinite(t.sum) ? add_rn(t.sum, t.error) : t.sum;
    }
    f4* o = reinterpret_cast<f4*>(out) + quad;
    if (accumulate) {
        const f4 old = *o;
        r = f4{add_rn(old[0], r[0]), add_rn(old[1], r[1]), add_rn(old[2], r[2]),
               add_rn(old[3], r[3])};
    }
    *o = r;
}

__global__ void __launch_bounds__(256)
column_sums_one_chunk(float* __restrict__ out, const float* __restrict__ dy, int rows,
                      size_t cols, int accumulate) {
    column_sums_quad(out, dy, rows, cols, accumulate, size_t(blockIdx.x) * 256 + threadIdx.x);
}

// ------------------------------------------------ token rows without a sort

constexpr int kScanRows = 8192;   // tokens embedding_scan_runs holds in LDS
constexpr int kScanWaves = 4;     // positions (one a wave) per workgroup
constexpr int kScanThreads = kScanWaves * 64;
constexpr int kScanBatch = 4;     // rows of a run whose loads go out together

// The positions of one 512-position block of the scan that hold a token:
// bit l of m[k] says whether lane l's position 8 l + k does. next() returns
// them in ascending order (base + 8 l + k), then -1. Every member holds the
// same value on all lanes.
struct BlockMatches {
    uint64_t m[8];
    uint64_t lanes;   // lanes with a position not yet returned, but `at`
    unsigned cur;     // positions k of lane `at` not yet returned
    int at;
    int base;
    __device__ int next() {
        if (cur == 0) {
            if (lanes == 0) return -1;
            at = __builtin_ctzll(lanes);
            lanes &= lanes - 1;
#pragma unroll
            for (int k = 0; k < 8; ++k) cur |= unsigned((m[k] >> at) & 1) << k;
        }
        const int k = __builtin_ctz(cur);
        cur &= cur - 1;
        return base + 8 * at + k;
    }
};

// dwte += the token rows of dx without sorting them (up to kScanRows rows,
// widths up to 256 G). The tokens sit in LDS, and wave w of workgroup b takes
// position i = kScanWaves b + w. The wave scans the tokens in ascending
// blocks of 512, lane l reading positions 8 l .. 8 l + 7 of a block as one
// 16-byte word, so that lane order is position order. If the first block
// holding the wave's token holds it before i, an earlier position's wave owns
// the token and this one leaves. Otherwise i is the token's first position:
// the wave adds the dx rows of i and of every later position with the same
// token, in ascending order, kScanBatch rows' loads in flight at a time. That
// is the run a stable sort puts together, summed as embedding_runs sums it
// (compensated, in the same order), so the bits are the sorted path's. Lane l
// holds columns 256 g + 4 l (g < G). Workgroups from run_blocks on take
// column quads of the position gradient (column_sums_quad, as in
// sort_tokens_and_positions).
template <int G>
__global__ void __launch_bounds__(kScanThreads)
embedding_scan_runs(float* __restrict__ dwte, const float* __restrict__ dx,
                    const uint16_t* __restrict__ tokens, int rows, size_t width,
                    unsigned run_blocks, float* __restrict__ dwpe, int sequences, size_t cols,
                    int accumulate_wpe) {
    typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
    __shared__ __attribute__((aligned(16))) uint16_t tok[kScanRows];
    if (blockIdx.x >= run_blocks) {
        column_sums_quad(dwpe, dx, sequences, cols, accumulate_wpe,
                         size_t(blockIdx.x - run_blocks) * kScanThreads + threadIdx.x);
        return;
    }
    // The ABI's tokens are 16-byte aligned: whole words, then the last few.
    const int words = rows / 8;
    for (int q = int(threadIdx.x); q < words; q += kScanThreads)
        reinterpret_cast<u4*>(tok)[q] = reinterpret_cast<const u4*>(tokens)[q];
    for (int p = words * 8 + int(threadIdx.x); p < rows; p += kScanThreads) tok[p] = tokens[p];
    __syncthreads();
    const int lane = int(threadIdx.x & 63);
    const size_t col0 = size_t(lane) * 4;
    const int i = int(blockIdx.x) * kScanWaves + int(threadIdx.x >> 6);
    if (i >= rows) return;
    const uint16_t v = tok[i];
    Comp s[G][4];
    f4 old[G];
    bool owner = false;
    // Each block's word is read while the one before is tested. base + 8 lane
    // + 7 < base + 512 <= kScanRows: the word stays inside tok; positions at
    // or past rows are masked off.
    u16x8 next = *reinterpret_cast<const u16x8*>(tok + 8 * lane);
    for (int base = 0; base < rows; base += 512) {
        const u16x8 t = next;
        if (base + 512 < rows) next = *reinterpret_cast<const u16x8*>(tok + base + 512 + 8 * lane);
        const int left = rows - base - 8 * lane;
        BlockMatches bm;
        bm.lanes = 0;
        bm.cur = 0;
        bm.at = 0;
        bm.base = base;
#pragma unroll
        for (int k = 0; k < 8; ++k) bm.m[k] = __builtin_amdgcn_ballot_w64(t[k] == v);
        if (base + 512 > rows) {   // the last block: no match at or past rows
#pragma unroll
            for (int k = 0; k < 8; ++k) bm.m[k] &= __builtin_amdgcn_ballot_w64(k < left);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) bm.lanes |= bm.m[k];
        if (bm.lanes == 0) continue;
        if (!owner) {
            BlockMatches first = bm;
            if (first.next() < i) return;   // an earlier position holds the token
            owner = true;
            // The row the sums add into, loaded beside the first dx rows.
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const size_t col = col0 + size_t(g) * 256;
                old[g] = col < width ? *reinterpret_cast<const f4*>(dwte + size_t(v) * width + col)
                                     : f4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
        for (;;) {
            int j[kScanBatch];
#pragma unroll
            for (int u = 0; u < kScanBatch; ++u) j[u] = bm.next();
            f4 d[kScanBatch][G];
#pragma unroll
            for (int u = 0; u < kScanBatch; ++u)
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const size_t col = col0 + size_t(g) * 256;
                    d[u][g] = j[u] >= 0 && col < width
                                  ? *reinterpret_cast<const f4*>(dx + size_t(j[u]) * width + col)
                                  : f4{0.0f, 0.0f, 0.0f, 0.0f};
                }
#pragma unroll
            for (int u = 0; u < kScanBatch; ++u) {
                if (j[u] < 0) break;
#pragma unroll
                for (int g = 0; g < G; ++g)
#pragma unroll
                    for (int c = 0; c < 4; ++c) comp_add(s[g][c], d[u][g][c]);
            }
            if (j[kScanBatch - 1] < 0) break;
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const size_t col = col0 + size_t(g) * 256;
        if (col >= width) continue;
        f4 r;
#pragma unroll
        for (int c = 0; c < 4; ++c)
            r[c] = add_rn(old[g][c], __builtin_isfinite(s[g][c].sum)
                                         ? add_rn(s[g][c].sum, s[g][c].error)
                                         : s[g][c].sum);
        *reinterpret_cast<f4*>(dwte + size_t(v) * width + col) = r;
    }
}

// The block sort and the position gradient in one launch: they are
// independent, and the sort's one workgroup leaves the other CUs idle.
// Workgroup 0 sorts; workgroup b > 0 takes column quads (b - 1) * 1024 + t of
// column_sums_one_chunk's sums (the same arithmetic; the sort's LDS makes
// these one workgroup per CU, 1,024 threads each).
__global__ void __launch_bounds__(1024)
sort_tokens_and_positions(uint16_t* __restrict__ out_tokens, unsigned* __restrict__ out_rows,
                          const uint16_t* __restrict__ tokens, int rows,
                          float* __restrict__ dwpe, const float* __restrict__ dx,
                          int sequences, size_t cols, int accumulate) {
    if (blockIdx.x == 0) {
        sort_block_body(out_tokens, out_rows, tokens, rows);
        return;
    }
    column_sums_quad(dwpe, dx, sequences, cols, accumulate,
                     size_t(blockIdx.x - 1) * 1024 + threadIdx.x);
}

}  // namespace

hipError_t launch_copy(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    if ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) % 16 == 0) {
        const size_t vecs = bytes / 16;
        if (vecs > 0) {
            hipLaunchKernelGGL(copy_vec, dim3(grid_for(vecs, 256)), dim3(256), 0, stream,
                               static_cast<u4*>(dst), static_cast<const u4*>(src), vecs);
        }
        const size_t tail = bytes - vecs * 16;
        if (tail > 0) {
            hipLaunchKernelGGL(copy_bytes, dim3(1), dim3(256), 0, stream,
                               static_cast<uint8_t*>(dst) + vecs * 16,
                               static_cast<const uint8_t*>(src) + vecs * 16, tail);
        }
    } else {
        hipLaunchKernelGGL(copy_bytes, dim3(grid_for(bytes, 256)), dim3(256), 0, stream,
                           static_cast<uint8_t*>(dst), static_cast<const uint8_t*>(src), bytes);
    }
    return hipGetLastError();
}

hipError_t launch_fill_zero(void* dst, size_t bytes, hipStream_t stream) {
    const size_t vecs = bytes / 16;
    if (vecs > 0) {
        hipLaunchKernelGGL(fill_zero_vec, dim3(grid_for(vecs, 256)), dim3(256), 0, stream,
                           static_cast<u4*>(dst), vecs);
    }
    const size_t tail = bytes - vecs * 16;
    if (tail > 0) {
        hipLaunchKernelGGL(fill_zero_bytes, dim3(1), dim3(256), 0, stream,
                           static_cast<uint8_t*>(dst) + vecs * 16, tail);
    }
    return hipGetLastError();
}

hipError_t launch_fp32_to_fp16(void* y, const void* x, size_t count, hipStream_t stream) {
    hipLaunchKernelGGL(fp32_to_fp16, dim3(grid_for(std::max<size_t>(count / 4, 1), 256)),
                       dim3(256), 0, stream, static_cast<_Float16*>(y),
                       static_cast<const float*>(x), count);
    return hipGetLastError();
}

hipError_t launch_heads(void* y, const void* x, size_t batches, size_t length, size_t heads,
                        size_t head_width, size_t row_width, size_t first, bool merge,
                        hipStream_t stream) {
    const size_t rows = batches * length;
    const size_t total = rows * heads * (head_width / 8);
    hipLaunchKernelGGL(heads_move, dim3(grid_for(total, 256)), dim3(256), 0, stream,
                       static_cast<h8*>(y), static_cast<const h8*>(x), rows, length, int(heads),
                       int(head_width / 8), int(row_width / 8), int(first / 8), merge ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_heads3(void* wide, void* const parts[3], size_t batches, size_t length,
                         size_t heads, size_t head_width, bool merge, hipStream_t stream) {
    const size_t rows = batches * length;
    const size_t total = 3 * rows * heads * (head_width / 8);
    if (head_width % 8 != 0 || total >= (size_t{1} << 32)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(heads_move3, dim3(grid_for(total, 256)), dim3(256), 0, stream,
                       static_cast<h8*>(wide), static_cast<h8*>(parts[0]),
                       static_cast<h8*>(parts[1]), static_cast<h8*>(parts[2]), unsigned(rows),
                       unsigned(length), unsigned(heads), unsigned(head_width / 8),
                       merge ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_embedding_forward(void* x, const void* tokens, const void* wte,
                                    const void* wpe, size_t rows, size_t length, size_t width,
                                    hipStream_t stream) {
    hipLaunchKernelGGL(embedding_forward, dim3(grid_for(rows, 4)), dim3(256), 0, stream,
                       static_cast<float*>(x), static_cast<const uint16_t*>(tokens),
                       static_cast<const float*>(wte), static_cast<const float*>(wpe), rows,
                       length, width);
    return hipGetLastError();
}

size_t embedding_backward_workspace(size_t sequences, size_t length, size_t vocab, size_t width) {
    return emb_layout(sequences, length, vocab, width).bytes;
}

namespace {

// dwpe: the column sums of dx viewed as sequences x cols (cols = length *
// width), in the bias gradient's order; partials is the workspace's region for
// more than one chunk of sequences.
hipError_t launch_position_sums(void* dwpe, const void* dx, void* partials, size_t sequences,
                                size_t cols, bool accumulate, hipStream_t stream) {
    if (sequences <= 256) {
        hipLaunchKernelGGL(column_sums_one_chunk, dim3(unsigned((cols / 4 + 255) / 256)),
                           dim3(256), 0, stream, static_cast<float*>(dwpe),
                           static_cast<const float*>(dx), int(sequences), cols,
                           accumulate ? 1 : 0);
        return hipGetLastError();
    }
    const dim3 pgrid(unsigned((cols / 8 + 7) / 8), unsigned((sequences + 255) / 256));
    hipLaunchKernelGGL(column_partials_f32, pgrid, dim3(64), 0, stream,
                       static_cast<float*>(partials), static_cast<const float*>(dx), sequences,
                       cols);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    return launch_bias_gradient_finish(dwpe, partials, sequences, cols, accumulate, stream);
}

}  // namespace

hipError_t launch_embedding_backward(void* dwte, void* dwpe, const void* dx, const void* tokens,
                                     size_t sequences, size_t length, size_t vocab, size_t width,
                                     bool accumulate_wte, bool accumulate_wpe, void* workspace,
                                     hipStream_t stream) {
    const EmbLayout l = emb_layout(sequences, length, vocab, width);
    auto* ws = static_cast<uint8_t*>(workspace);
    const size_t rows = sequences * length;
    const unsigned tiles = unsigned((rows + kSortTile - 1) / kSortTile);
    auto* counts = reinterpret_cast<unsigned*>(ws + l.counts);
    auto* pass_tokens = reinterpret_cast<uint16_t*>(ws + l.pass_tokens);
    auto* pass_rows = reinterpret_cast<unsigned*>(ws + l.pass_rows);
    auto* sorted_tokens = reinterpret_cast<uint16_t*>(ws + l.sorted_tokens);
    auto* sorted_rows = reinterpret_cast<unsigned*>(ws + l.sorted_rows);
    auto* offsets = reinterpret_cast<unsigned*>(ws + l.offsets);
    const auto* tok = static_cast<const uint16_t*>(tokens);

    const size_t cols = length * width;   // dwpe: column sums of dx as sequences x cols
    // With one chunk of sequences the position gradient rides in the token
    // rows' launch ("emb_together" = "0": its own launch after them).
    const bool together = rows <= size_t(kBlockSortRows) && sequences <= 256 &&
                          (cols / 4 + 1023) / 1024 < (size_t{1} << 30) &&
                          !tuning_off(Tune::kEmbTogether);
    const unsigned pos_blocks = together ? unsigned((cols / 4 + 1023) / 1024) : 0u;
    const size_t scan_pos_blocks = together ? (cols / 4 + kScanThreads - 1) / kScanThreads : 0;
    // Accumulating into dwte, with the tokens in one workgroup's LDS: the
    // token rows without a sort ("emb_scan" = "0": the sorted path).
    const size_t groups = (width + 255) / 256;
    const size_t run_blocks = (rows + kScanWaves - 1) / kScanWaves;
    if (accumulate_wte && rows <= size_t(kScanRows) && groups <= 4 &&
        run_blocks + scan_pos_blocks < (size_t{1} << 31) && !tuning_off(Tune::kEmbScan)) {
        const dim3 grid(unsigned(run_blocks + scan_pos_blocks));
        auto scan = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, grid, dim3(kScanThreads), 0, stream, static_cast<float*>(dwte),
                               static_cast<const float*>(dx), tok, int(rows), width,
                               unsigned(run_blocks),
                               static_cast<float*>(dwpe), int(sequences), cols,
                               accumulate_wpe ? 1 : 0);
        };
        switch (groups) {
        case 1: scan(embedding_scan_runs<1>); break;
        case 2: scan(embedding_scan_runs<2>); break;
        case 3: scan(embedding_scan_runs<3>); break;
        default: scan(embedding_scan_runs<4>); break;
        }
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
        if (together) return hipSuccess;
        return launch_position_sums(dwpe, dx, ws + l.partials, sequences, cols, accumulate_wpe,
                                    stream);
    }
    // Two stable passes of 8 bits: low byte into the pass buffers, high byte
    // into the sorted buffers; in one workgroup's LDS when the rows fit.
    if (together) {
        hipLaunchKernelGGL(sort_tokens_and_positions, dim3(1 + pos_blocks), dim3(1024), 0, stream,
                           sorted_tokens, sorted_rows, tok, int(rows), static_cast<float*>(dwpe),
                           static_cast<const float*>(dx), int(sequences), cols,
                           accumulate_wpe ? 1 : 0);
    } else if (rows <= size_t(kBlockSortRows)) {
        hipLaunchKernelGGL(sort_tokens_block, dim3(1), dim3(1024), 0, stream, sorted_tokens,
                           sorted_rows, tok, int(rows));
    }
    for (int pass = 0; pass < (rows <= size_t(kBlockSortRows) ? 0 : 2); ++pass) {
        const int shift = pass * 8;
        const uint16_t* in_t = pass == 0 ? tok : pass_tokens;
        const unsigned* in_r = pass == 0 ? nullptr : pass_rows;
        uint16_t* out_t = pass == 0 ? pass_tokens : sorted_tokens;
        unsigned* out_r = pass == 0 ? pass_rows : sorted_rows;
        hipLaunchKernelGGL(sort_count, dim3(tiles), dim3(256), 0, stream, counts, in_t, rows,
                           shift, tiles);
        hipLaunchKernelGGL(scan_exclusive, dim3(1), dim3(1024), 0, stream, counts,
                           size_t(tiles) * kDigits);
        hipLaunchKernelGGL(sort_scatter, dim3(tiles), dim3(256), 0, stream, out_t, out_r, in_t,
                           in_r, counts, rows, shift, tiles);
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    }
    // A grid dimension holds fewer than 2^32 work-items.
    if (accumulate_wte && rows < (size_t{1} << 26)) {
        hipLaunchKernelGGL(embedding_runs, dim3(unsigned(rows), unsigned((width / 4 + 63) / 64)),
                           dim3(64), 0, stream, static_cast<float*>(dwte),
                           static_cast<const float*>(dx), sorted_tokens, sorted_rows, rows,
                           width);
    } else {
        hipLaunchKernelGGL(token_offsets, dim3(unsigned((vocab + 1 + 255) / 256)), dim3(256), 0,
                           stream, offsets, sorted_tokens, rows, unsigned(vocab));
        hipLaunchKernelGGL(embedding_words, dim3(unsigned(vocab), unsigned((width / 4 + 63) / 64)),
                           dim3(64), 0, stream, static_cast<float*>(dwte),
                           static_cast<const float*>(dx), sorted_rows, offsets, width,
                           accumulate_wte ? 1 : 0);
    }
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    if (together) return hipSuccess;
    return launch_position_sums(dwpe, dx, ws + l.partials, sequences, cols, accumulate_wpe,
                                stream);
}

}  // namespace flint
