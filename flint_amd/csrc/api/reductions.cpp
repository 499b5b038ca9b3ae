// C-ABI entry points of the row reductions: LayerNorm, bias gradient, causal
// softmax and softmax + cross-entropy. Each is a Checker chain (sizes, then
// its buffers) and one launcher call; the limits, the order of the checks and
// the message texts are the reference's interface (ref src/api/layernorm.cpp:11-119,
// bias_gradient.cpp:11-68, softmax.cpp:11-76, cross_entropy.cpp:9-49).
#include <cmath>

#include "common/args.h"
#include "flint/flint_noalloc.h"
#include "kernels/kernels.h"

namespace {

using flint::Checker;
using flint::Span;

// Column sums in 256-row chunks: LayerNorm backward needs at least one column
// chunk of 8 and one row; the bias gradient takes cols = 0 (a no-op).
Checker& ln_backward_sizes(Checker& c, size_t rows, size_t cols) {
    return c
        .require(cols != 0 && cols % 8 == 0 && cols <= flint::kBiasGradientMaxCols,
                 "cols (%zu) must be a multiple of 8 from 8 to %zu", cols,
                 flint::kBiasGradientMaxCols)
        .require(rows != 0 && rows <= flint::kLayerNormMaxRows, "rows (%zu) must be from 1 to %zu",
                 rows, flint::kLayerNormMaxRows);
}

Checker& bias_sizes(Checker& c, size_t rows, size_t cols) {
    return c
        .require(cols % 8 == 0 && cols <= flint::kBiasGradientMaxCols,
                 "cols (%zu) must be a multiple of 8 up to %zu", cols, flint::kBiasGradientMaxCols)
        .require(rows != 0 && rows <= flint::kBiasGradientMaxRows, "rows (%zu) must be from 1 to %zu",
                 rows, flint::kBiasGradientMaxRows);
}

Checker& softmax_sizes(Checker& c, size_t batches, size_t length) {
    return c
        .require(length % 8 == 0 && length <= flint::kSoftmaxMaxLength,
                 "length (%zu) must be a multiple of 8 up to %zu", length, flint::kSoftmaxMaxLength)
        .require(batches <= flint::kSoftmaxMaxBatches, "batches (%zu) can be up to %zu", batches,
                 flint::kSoftmaxMaxBatches);
}

Checker& finite_scale(Checker& c, float scale) {
    return c.require(std::isfinite(scale), "scale (%g) must be finite", double(scale));
}

}  // namespace

extern "C" {

FLINT_API flint_status flint_layernorm_forward(void* y, void* mean, void* rstd, const void* x,
                                               const void* gamma, const void* beta, size_t rows,
                                               size_t cols, float eps, flint_stream stream) {
    Checker c("flint_layernorm_forward");
    c.require(cols != 0 && cols <= flint::kLayerNormMaxCols, "cols (%zu) must be from 1 to %zu", cols,
              flint::kLayerNormMaxCols)
        .require(rows <= flint::kLayerNormMaxRows, "rows (%zu) can be up to %zu", rows,
                 flint::kLayerNormMaxRows)
        .require(std::isfinite(eps) && eps >= 0.0f, "eps (%g) must be finite and non-negative",
                 double(eps));
    if (!c.ok() || rows == 0) return c.status();
    // Outputs first: y, mean and rstd may not touch each other or an input.
    c.buffers({{"y", y, rows * cols * 2},
               {"mean", mean, rows * 4},
               {"rstd", rstd, rows * 4},
               {"x", x, rows * cols * 4},
               {"gamma", gamma, cols * 4},
               {"beta", beta, cols * 4}},
              3);
    if (!c.ok()) return c.status();
    FLINT_HIP_CHECK(flint::launch_layernorm_forward(y, mean, rstd, x, gamma, beta, rows, cols, eps,
                                                    flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_layernorm_backward(void* dx, void* dgamma, void* dbeta,
                                                const void* dy, const void* x, const void* mean,
                                                const void* rstd, const void* gamma, size_t rows,
                                                size_t cols, int accumulate_dx,
                                                int accumulate_params, void* workspace,
                                                size_t workspace_bytes, flint_stream stream) {
    Checker c("flint_layernorm_backward");
    if (!ln_backward_sizes(c, rows, cols).ok()) return c.status();
    const size_t needed = flint::layernorm_backward_workspace(rows, cols);
    c.require(workspace_bytes >= needed, "needs %zu bytes of workspace, given %zu", needed,
              workspace_bytes)
        .buffers({{"dx", dx, rows * cols * 4},
                  {"dgamma", dgamma, cols * 4},
                  {"dbeta", dbeta, cols * 4},
                  {"workspace", workspace, needed},
                  {"dy", dy, rows * cols * 2},
                  {"x", x, rows * cols * 4},
                  {"mean", mean, rows * 4},
                  {"rstd", rstd, rows * 4},
                  {"gamma", gamma, cols * 4}},
                 4);
    if (!c.ok()) return c.status();
    FLINT_HIP_CHECK(flint::launch_layernorm_backward(dx, dgamma, dbeta, dy, x, mean, rstd, gamma,
                                                     rows, cols, accumulate_dx != 0,
                                                     accumulate_params != 0, workspace,
                                                     flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_layernorm_backward_workspace(size_t rows, size_t cols,
                                                          size_t* bytes) {
    Checker c("flint_layernorm_backward_workspace");
    if (!ln_backward_sizes(c.require(bytes != nullptr, "bytes is null"), rows, cols).ok())
        return c.status();
    *bytes = flint::layernorm_backward_workspace(rows, cols);
    return FLINT_OK;
}

FLINT_API flint_status flint_bias_gradient_workspace(size_t rows, size_t cols, size_t* bytes) {
    Checker c("flint_bias_gradient_workspace");
    if (!bias_sizes(c.require(bytes != nullptr, "bytes is null"), rows, cols).ok())
        return c.status();
    *bytes = flint::bias_gradient_workspace(rows, cols);
    return FLINT_OK;
}

FLINT_API flint_status flint_bias_gradient(void* dbias, const void* dy, size_t rows, size_t cols,
                                           int accumulate, void* workspace,
                                           size_t workspace_bytes, flint_stream stream) {
    Checker c("flint_bias_gradient");
    if (!bias_sizes(c, rows, cols).ok() || cols == 0) return c.status();
    const size_t needed = flint::bias_gradient_workspace(rows, cols);
    c.require(workspace_bytes >= needed, "needs %zu bytes of workspace, given %zu", needed,
              workspace_bytes)
        .buffers({{"dbias", dbias, cols * 4},
                  {"workspace", workspace, needed},
                  {"dy", dy, rows * cols * 2}},
                 2);
    if (!c.ok()) return c.status();
    FLINT_HIP_CHECK(flint::launch_bias_gradient(dbias, dy, rows, cols, accumulate != 0, workspace,
                                                flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_bias_gradient_noalloc(void* dbias, const void* dy, size_t rows,
                                                   size_t cols, int accumulate,
                                                   flint_stream stream) {
    Checker c("flint_bias_gradient_noalloc");
    if (!bias_sizes(c, rows, cols).ok() || cols == 0) return c.status();
    const size_t needed = flint::bias_gradient_workspace(rows, cols);
    c.require(needed <= flint::kBiasGradientScratchBytes,
              "%zu x %zu needs %zu bytes of scratch, more than the %zu the library holds", rows,
              cols, needed, flint::kBiasGradientScratchBytes)
        .buffers({{"dbias", dbias, cols * 4}, {"dy", dy, rows * cols * 2}}, 1);
    if (!c.ok()) return c.status();
    FLINT_HIP_CHECK(flint::launch_bias_gradient_noalloc(dbias, dy, rows, cols, accumulate != 0,
                                                        flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_causal_softmax_forward(void* p, const void* s, size_t batches,
                                                    size_t length, flint_stream stream) {
    Checker c("flint_causal_softmax_forward");
    if (!softmax_sizes(c, batches, length).ok() || batches == 0 || length == 0) return c.status();
    const size_t bytes = batches * length * length * 2;
    if (!c.buffers({{"p", p, bytes}, {"s", s, bytes}}, 1).ok()) return c.status();
    FLINT_HIP_CHECK(flint::launch_causal_softmax_forward(p, s, batches * length, length,
                                                         flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_causal_softmax_backward(void* ds, const void* p, const void* dp,
                                                     size_t batches, size_t length, float scale,
                                                     flint_stream stream) {
    Checker c("flint_causal_softmax_backward");
    if (!finite_scale(softmax_sizes(c, batches, length), scale).ok() || batches == 0 ||
        length == 0)
        return c.status();
    const size_t bytes = batches * length * length * 2;
    // In place (ds == dp) is allowed: dp then drops out of the overlap test.
    const Span list[] = {{"ds", ds, bytes}, {"p", p, bytes}, {"dp", dp, bytes}};
    if (!c.buffers(list, ds == dp ? 2 : 3, 1).ok()) return c.status();
    FLINT_HIP_CHECK(flint::launch_causal_softmax_backward(ds, p, dp, batches * length, length,
                                                          scale, flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_softmax_cross_entropy(void* dlogits, void* row_loss,
                                                   const void* logits, const void* targets,
                                                   float scale, size_t rows, size_t vocab,
                                                   size_t cols, flint_stream stream) {
    Checker c("flint_softmax_cross_entropy");
    c.require(cols != 0 && cols % 8 == 0 && cols <= flint::kCrossEntropyMaxCols,
              "cols (%zu) must be a multiple of 8 from 8 to %zu", cols, flint::kCrossEntropyMaxCols)
        .require(vocab != 0 && vocab <= cols, "vocab (%zu) must be from 1 to cols (%zu)", vocab,
                 cols)
        .require(rows <= flint::kCrossEntropyMaxRows, "rows (%zu) can be up to %zu", rows,
                 flint::kCrossEntropyMaxRows);
    if (!finite_scale(c, scale).ok() || rows == 0) return c.status();
    c.buffers({{"dlogits", dlogits, rows * cols * 2},
               {"row_loss", row_loss, rows * 4},
               {"logits", logits, rows * cols * 2},
               {"targets", targets, rows * 2}},
              2);
    if (!c.ok()) return c.status();
    FLINT_HIP_CHECK(flint::launch_softmax_cross_entropy(dlogits, row_loss, logits, targets, scale,
                                                        rows, vocab, cols, flint::to_hip(stream)));
    return FLINT_OK;
}

}  // extern "C"
