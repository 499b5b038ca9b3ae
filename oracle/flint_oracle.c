/* CPU oracle for libflint's hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatement, in IEEE FP32 (built with -ffp-contract=off so no
 * multiply-add is fused unless written as fmaf), of the arithmetic the
 * reference (bayareahomelander/Flint) specifies for its reduction kernels,
 * including the summation orders its headers promise are shape-only:
 *
 *   layernorm_forward   ref src/kernels/layernorm.cu:33-155
 *   bias_gradient       ref src/kernels/bias_gradient.cu:1-25, :82-179
 *   layernorm_backward  ref src/kernels/layernorm_backward.cu:1-30, :120-271
 *   softmax_forward     ref src/kernels/softmax.cu:1-19, :68-122
 *   softmax_backward    ref src/kernels/softmax_backward.cu:1-27, :111-154
 *   cross_entropy       ref src/kernels/cross_entropy.cu:1-25, :106-172
 *   embedding_backward  ref include/flint/flint.h:270-303 (order of the sums)
 *
 * The reference's "warp" is 32 lanes; lane l of a row takes chunks l, l + 32,
 * ... and a butterfly with xor offsets 16, 8, 4, 2, 1 merges the lanes. The
 * emulation below keeps 32 lane accumulators and merges them the same way.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg load
 * this library, and only as the checker. Outputs are FP32; the caller rounds
 * to FP16 where the kernel does (numpy's float32 -> float16 cast is RNE). */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define LANES 32

typedef struct {
    float sum;
    float error;
} comp;

/* TwoSum (Knuth): t + e == sum + v exactly. */
static void comp_add(comp* a, float v) {
    const float t = a->sum + v;
    const float v_part = t - a->sum;
    a->error += (a->sum - (t - v_part)) + (v - v_part);
    a->sum = t;
}

static void comp_merge(comp* a, float b_sum, float b_error) {
    const float errors = a->error + b_error;
    a->error = 0.0f;
    comp_add(a, b_sum);
    a->error += errors;
}

static void comp_add_square(comp* a, float d) {
    const float p = d * d;
    a->error += fmaf(d, d, -p);
    comp_add(a, p);
}

static void comp_add_product(comp* a, float u, float v) {
    const float p = u * v;
    a->error += fmaf(u, v, -p);
    comp_add(a, p);
}

/* Butterfly over 32 lanes; returns lane 0's pair (all lanes agree). */
static comp comp_butterfly(comp* lanes) {
    comp next[LANES];
    for (int off = LANES / 2; off > 0; off /= 2) {
        for (int l = 0; l < LANES; ++l) {
            next[l] = lanes[l];
            comp_merge(&next[l], lanes[l ^ off].sum, lanes[l ^ off].error);
        }
        memcpy(lanes, next, sizeof next);
    }
    return lanes[0];
}

static float float_butterfly(float* lanes) {
    float next[LANES];
    for (int off = LANES / 2; off > 0; off /= 2) {
        for (int l = 0; l < LANES; ++l) next[l] = lanes[l] + lanes[l ^ off];
        memcpy(lanes, next, sizeof next);
    }
    return lanes[0];
}

static float comp_value(comp a) { return isfinite(a.sum) ? a.sum + a.error : a.sum; }

/* ---------------------------------------------------------------- LayerNorm */

void or_layernorm_forward(float* y, float* mean, float* rstd, const float* x, const float* gamma,
                          const float* beta, size_t rows, size_t cols, float eps) {
    const int vec = cols % 4 == 0 ? 4 : 1;
    const size_t groups = cols / vec;
    for (size_t r = 0; r < rows; ++r) {
        const float* xr = x + r * cols;
        comp lanes[LANES];
        memset(lanes, 0, sizeof lanes);
        for (size_t g = 0; g < groups; ++g)
            for (int j = 0; j < vec; ++j) comp_add(&lanes[g % LANES], xr[g * vec + j]);
        comp s = comp_butterfly(lanes);
        const float n = (float)cols;
        const float mu = (s.sum + s.error) / n;
        memset(lanes, 0, sizeof lanes);
        for (size_t g = 0; g < groups; ++g)
            for (int j = 0; j < vec; ++j) comp_add_square(&lanes[g % LANES], xr[g * vec + j] - mu);
        comp q = comp_butterfly(lanes);
        const float rs = 1.0f / sqrtf((q.sum + q.error) / n + eps);
        for (size_t c = 0; c < cols; ++c) y[r * cols + c] = fmaf((xr[c] - mu) * rs, gamma[c], beta[c]);
        mean[r] = mu;
        rstd[r] = rs;
    }
}

/* ---------------------------------------------------------- column sums
 * Chunks of 256 rows; within a chunk, phase p (0..7) adds rows p, p + 8, ...
 * in order, then phase 0 merges phases 1..7 in order. The chunks' pairs then
 * merge per column over 32 lanes (lane l takes chunks l, l + 32, ...) and a
 * butterfly. value(v, r, c) gives the addend. */

typedef void (*addend_fn)(comp* a, size_t r, size_t c, const void* ctx);

static void column_sums(float* out, size_t rows, size_t cols, int accumulate, addend_fn add,
                        const void* ctx) {
    const size_t chunks = (rows + 255) / 256;
    for (size_t c = 0; c < cols; ++c) {
        comp lanes[LANES];
        memset(lanes, 0, sizeof lanes);
        for (size_t ch = 0; ch < chunks; ++ch) {
            const size_t first = ch * 256;
            const size_t end = rows - first < 256 ? rows : first + 256;
            comp phase[8];
            memset(phase, 0, sizeof phase);
            for (int p = 0; p < 8; ++p)
                for (size_t r = first + p; r < end; r += 8) add(&phase[p], r, c, ctx);
            for (int p = 1; p < 8; ++p) comp_merge(&phase[0], phase[p].sum, phase[p].error);
            comp_merge(&lanes[ch % LANES], phase[0].sum, phase[0].error);
        }
        const comp t = comp_butterfly(lanes);
        const float v = comp_value(t);
        out[c] = accumulate ? out[c] + v : v;
    }
}

typedef struct {
    const float* dy;
    size_t cols;
} plain_ctx;

static void add_plain(comp* a, size_t r, size_t c, const void* ctx) {
    const plain_ctx* p = (const plain_ctx*)ctx;
    comp_add(a, p->dy[r * p->cols + c]);
}

/* dy holds the FP16 gradient's values widened to FP32. */
void or_bias_gradient(float* dbias, const float* dy, size_t rows, size_t cols, int accumulate) {
    const plain_ctx ctx = {dy, cols};
    column_sums(dbias, rows, cols, accumulate, add_plain, &ctx);
}

typedef struct {
    const float* dy;
    const float* x;
    const float* mean;
    const float* rstd;
    size_t cols;
} dgamma_ctx;

static void add_dgamma(comp* a, size_t r, size_t c, const void* ctx) {
    const dgamma_ctx* p = (const dgamma_ctx*)ctx;
    const float xhat = (p->x[r * p->cols + c] - p->mean[r]) * p->rstd[r];
    comp_add_product(a, p->dy[r * p->cols + c], xhat);
}

void or_layernorm_backward(float* dx, float* dgamma, float* dbeta, const float* dy,
                           const float* x, const float* mean, const float* rstd,
                           const float* gamma, size_t rows, size_t cols, int accumulate_dx,
                           int accumulate_params) {
    or_bias_gradient(dbeta, dy, rows, cols, accumulate_params);
    const dgamma_ctx ctx = {dy, x, mean, rstd, cols};
    column_sums(dgamma, rows, cols, accumulate_params, add_dgamma, &ctx);
    const size_t pieces = cols / 8;
    const float n = (float)cols;
    for (size_t r = 0; r < rows; ++r) {
        float g_lanes[LANES] = {0}, gx_lanes[LANES] = {0};
        for (size_t p = 0; p < pieces; ++p) {
            for (int j = 0; j < 8; ++j) {
                const size_t c = p * 8 + j;
                const float g = dy[r * cols + c] * gamma[c];
                const float xhat = (x[r * cols + c] - mean[r]) * rstd[r];
                g_lanes[p % LANES] += g;
                gx_lanes[p % LANES] += g * xhat;
            }
        }
        const float g_mean = float_butterfly(g_lanes) / n;
        const float gx_mean = float_butterfly(gx_lanes) / n;
        for (size_t c = 0; c < cols; ++c) {
            const float g = dy[r * cols + c] * gamma[c];
            const float xhat = (x[r * cols + c] - mean[r]) * rstd[r];
            const float v = rstd[r] * ((g - g_mean) - xhat * gx_mean);
            dx[r * cols + c] = accumulate_dx ? dx[r * cols + c] + v : v;
        }
    }
}

/* ------------------------------------------------------------ causal softmax */

void or_softmax_forward(float* p, const float* s, size_t rows, size_t length) {
    for (size_t row = 0; row < rows; ++row) {
        const size_t t = row % length;
        const float* sr = s + row * length;
        float* pr = p + row * length;
        float mx = -INFINITY;
        for (size_t c = 0; c <= t; ++c) mx = fmaxf(mx, sr[c]);
        float lanes[LANES] = {0};
        for (size_t c = 0; c <= t; ++c) lanes[(c / 8) % LANES] += expf(sr[c] - mx);
        /* A NaN max (fmaxf skips NaN only when the other operand is a number). */
        const float sum = float_butterfly(lanes);
        const float scale = 1.0f / sum;
        for (size_t c = 0; c < length; ++c) pr[c] = c <= t ? expf(sr[c] - mx) * scale : 0.0f;
    }
}

void or_softmax_backward(float* ds, const float* p, const float* dp, size_t rows, size_t length,
                         float scale) {
    for (size_t row = 0; row < rows; ++row) {
        const size_t t = row % length;
        const float* pr = p + row * length;
        const float* dr = dp + row * length;
        comp lanes[LANES];
        memset(lanes, 0, sizeof lanes);
        for (size_t c = 0; c <= t; ++c) comp_add(&lanes[(c / 8) % LANES], pr[c] * dr[c]);
        comp d = comp_butterfly(lanes);
        if (!isfinite(d.sum)) d.error = 0.0f;
        for (size_t c = 0; c < length; ++c)
            ds[row * length + c] = c <= t ? (pr[c] * ((dr[c] - d.sum) - d.error)) * scale : 0.0f;
    }
}

/* ----------------------------------------------------- softmax + cross-entropy */

void or_cross_entropy(float* dlogits, float* row_loss, const float* logits,
                      const uint16_t* targets, float scale, size_t rows, size_t vocab,
                      size_t cols) {
    for (size_t r = 0; r < rows; ++r) {
        const float* lr = logits + r * cols;
        float mx = -INFINITY;
        for (size_t c = 0; c < vocab; ++c) mx = fmaxf(mx, lr[c]);
        comp lanes[LANES];
        memset(lanes, 0, sizeof lanes);
        for (size_t c = 0; c < vocab; ++c) comp_add(&lanes[(c / 8) % LANES], expf(lr[c] - mx));
        const comp t = comp_butterfly(lanes);
        const float sum = t.sum + t.error;
        const float inverse = 1.0f / sum;
        const size_t target = targets[r];
        for (size_t c = 0; c < cols; ++c) {
            if (c >= vocab) {
                dlogits[r * cols + c] = 0.0f;
                continue;
            }
            const float gap = lr[c] - mx;
            float pc = expf(gap) * inverse;
            if (c == target) {
                row_loss[r] = logf(sum) - gap;
                pc -= 1.0f;
            }
            dlogits[r * cols + c] = pc * scale;
        }
    }
}

/* ------------------------------------------------------------ embedding bwd */

void or_embedding_backward(float* dwte, float* dwpe, const float* dx, const uint16_t* tokens,
                           size_t sequences, size_t length, size_t vocab, size_t width,
                           int accumulate_wte, int accumulate_wpe) {
    const size_t rows = sequences * length;
    for (size_t v = 0; v < vocab; ++v) {
        for (size_t c = 0; c < width; ++c) {
            comp s = {0.0f, 0.0f};
            int any = 0;
            for (size_t r = 0; r < rows; ++r) {
                if (tokens[r] != v) continue;
                any = 1;
                comp_add(&s, dx[r * width + c]);
            }
            float* o = &dwte[v * width + c];
            if (!any) {
                if (!accumulate_wte) *o = 0.0f;
            } else {
                const float val = comp_value(s);
                *o = accumulate_wte ? *o + val : val;
            }
        }
    }
    const plain_ctx ctx = {dx, length * width};
    column_sums(dwpe, sequences, length * width, accumulate_wpe, add_plain, &ctx);
}
