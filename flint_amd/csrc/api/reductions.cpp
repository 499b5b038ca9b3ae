// C-ABI entry points of the row reductions: LayerNorm, bias gradient, causal
// softmax and softmax + cross-entropy. Checks and message text follow the
// reference's src/api/layernorm.cpp:11-119, bias_gradient.cpp:11-68,
// softmax.cpp:11-76 and cross_entropy.cpp:9-49.
#include <cmath>
#include <iterator>

#include "common/common.h"
#include "kernels/kernels.h"

using flint::fail;

namespace {

flint_status check_ln_backward_dims(const char* name, size_t rows, size_t cols) {
    if (cols == 0 || cols % 8 != 0 || cols > flint::kBiasGradientMaxCols) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT,
                    "%s: cols (%zu) must be a multiple of 8 from 8 to %zu", name, cols,
                    flint::kBiasGradientMaxCols);
    }
    if (rows == 0 || rows > flint::kLayerNormMaxRows) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: rows (%zu) must be from 1 to %zu", name,
                    rows, flint::kLayerNormMaxRows);
    }
    return FLINT_OK;
}

flint_status check_bias_dims(const char* name, size_t rows, size_t cols) {
    if (cols % 8 != 0 || cols > flint::kBiasGradientMaxCols) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: cols (%zu) must be a multiple of 8 up to %zu",
                    name, cols, flint::kBiasGradientMaxCols);
    }
    if (rows == 0 || rows > flint::kBiasGradientMaxRows) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: rows (%zu) must be from 1 to %zu", name,
                    rows, flint::kBiasGradientMaxRows);
    }
    return FLINT_OK;
}

flint_status check_softmax_dims(const char* name, size_t batches, size_t length) {
    if (length % 8 != 0 || length > flint::kSoftmaxMaxLength) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: length (%zu) must be a multiple of 8 up to %zu",
                    name, length, flint::kSoftmaxMaxLength);
    }
    if (batches > flint::kSoftmaxMaxBatches) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: batches (%zu) can be up to %zu", name,
                    batches, flint::kSoftmaxMaxBatches);
    }
    return FLINT_OK;
}

}  // namespace

extern "C" {

FLINT_API flint_status flint_layernorm_forward(void* y, void* mean, void* rstd, const void* x,
                                               const void* gamma, const void* beta, size_t rows,
                                               size_t cols, float eps, flint_stream stream) {
    constexpr const char* name = "flint_layernorm_forward";
    if (cols == 0 || cols > flint::kLayerNormMaxCols) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: cols (%zu) must be from 1 to %zu", name,
                    cols, flint::kLayerNormMaxCols);
    }
    if (rows > flint::kLayerNormMaxRows) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: rows (%zu) can be up to %zu", name, rows,
                    flint::kLayerNormMaxRows);
    }
    if (!std::isfinite(eps) || eps < 0.0f) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: eps (%g) must be finite and non-negative",
                    name, static_cast<double>(eps));
    }
    if (rows == 0) return FLINT_OK;
    const flint::Buffer buffers[] = {
        {"y", y, rows * cols * 2},  {"mean", mean, rows * 4}, {"rstd", rstd, rows * 4},
        {"x", x, rows * cols * 4},  {"gamma", gamma, cols * 4}, {"beta", beta, cols * 4},
    };
    if (flint_status s = flint::check_buffers(name, buffers, std::size(buffers), 3); s != FLINT_OK) {
        return s;
    }
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
    constexpr const char* name = "flint_layernorm_backward";
    if (flint_status s = check_ln_backward_dims(name, rows, cols); s != FLINT_OK) return s;
    const size_t needed = flint::bias_gradient_workspace(rows, cols);
    if (workspace_bytes < needed) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: needs %zu bytes of workspace, given %zu",
                    name, needed, workspace_bytes);
    }
    const flint::Buffer buffers[] = {
        {"dx", dx, rows * cols * 4},       {"dgamma", dgamma, cols * 4},
        {"dbeta", dbeta, cols * 4},        {"workspace", workspace, needed},
        {"dy", dy, rows * cols * 2},       {"x", x, rows * cols * 4},
        {"mean", mean, rows * 4},          {"rstd", rstd, rows * 4},
        {"gamma", gamma, cols * 4},
    };
    if (flint_status s = flint::check_buffers(name, buffers, std::size(buffers), 4); s != FLINT_OK) {
        return s;
    }
    FLINT_HIP_CHECK(flint::launch_layernorm_backward(dx, dgamma, dbeta, dy, x, mean, rstd, gamma,
                                                     rows, cols, accumulate_dx != 0,
                                                     accumulate_params != 0, workspace,
                                                     flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_layernorm_backward_workspace(size_t rows, size_t cols,
                                                          size_t* bytes) {
    constexpr const char* name = "flint_layernorm_backward_workspace";
    if (bytes == nullptr) return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: bytes is null", name);
    if (flint_status s = check_ln_backward_dims(name, rows, cols); s != FLINT_OK) return s;
    *bytes = flint::bias_gradient_workspace(rows, cols);
    return FLINT_OK;
}

FLINT_API flint_status flint_bias_gradient_workspace(size_t rows, size_t cols, size_t* bytes) {
    constexpr const char* name = "flint_bias_gradient_workspace";
    if (bytes == nullptr) return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: bytes is null", name);
    if (flint_status s = check_bias_dims(name, rows, cols); s != FLINT_OK) return s;
    *bytes = flint::bias_gradient_workspace(rows, cols);
    return FLINT_OK;
}

FLINT_API flint_status flint_bias_gradient(void* dbias, const void* dy, size_t rows, size_t cols,
                                           int accumulate, void* workspace,
                                           size_t workspace_bytes, flint_stream stream) {
    constexpr const char* name = "flint_bias_gradient";
    if (flint_status s = check_bias_dims(name, rows, cols); s != FLINT_OK) return s;
    if (cols == 0) return FLINT_OK;
    const size_t needed = flint::bias_gradient_workspace(rows, cols);
    if (workspace_bytes < needed) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: needs %zu bytes of workspace, given %zu",
                    name, needed, workspace_bytes);
    }
    const flint::Buffer buffers[] = {
        {"dbias", dbias, cols * 4},
        {"workspace", workspace, needed},
        {"dy", dy, rows * cols * 2},
    };
    if (flint_status s = flint::check_buffers(name, buffers, std::size(buffers), 2); s != FLINT_OK) {
        return s;
    }
    FLINT_HIP_CHECK(flint::launch_bias_gradient(dbias, dy, rows, cols, accumulate != 0, workspace,
                                                flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_causal_softmax_forward(void* p, const void* s, size_t batches,
                                                    size_t length, flint_stream stream) {
    constexpr const char* name = "flint_causal_softmax_forward";
    if (flint_status st = check_softmax_dims(name, batches, length); st != FLINT_OK) return st;
    if (batches == 0 || length == 0) return FLINT_OK;
    const size_t bytes = batches * length * length * 2;
    const flint::Buffer buffers[] = {{"p", p, bytes}, {"s", s, bytes}};
    if (flint_status st = flint::check_buffers(name, buffers, std::size(buffers), 1);
        st != FLINT_OK) {
        return st;
    }
    FLINT_HIP_CHECK(flint::launch_causal_softmax_forward(p, s, batches * length, length,
                                                         flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_causal_softmax_backward(void* ds, const void* p, const void* dp,
                                                     size_t batches, size_t length, float scale,
                                                     flint_stream stream) {
    constexpr const char* name = "flint_causal_softmax_backward";
    if (flint_status st = check_softmax_dims(name, batches, length); st != FLINT_OK) return st;
    if (!std::isfinite(scale)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: scale (%g) must be finite", name,
                    static_cast<double>(scale));
    }
    if (batches == 0 || length == 0) return FLINT_OK;
    const size_t bytes = batches * length * length * 2;
    // In place (ds == dp) leaves dp out of the list; otherwise ds overlaps neither.
    const flint::Buffer buffers[] = {{"ds", ds, bytes}, {"p", p, bytes}, {"dp", dp, bytes}};
    if (flint_status st = flint::check_buffers(name, buffers, ds == dp ? 2 : std::size(buffers), 1);
        st != FLINT_OK) {
        return st;
    }
    FLINT_HIP_CHECK(flint::launch_causal_softmax_backward(ds, p, dp, batches * length, length,
                                                          scale, flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_softmax_cross_entropy(void* dlogits, void* row_loss,
                                                   const void* logits, const void* targets,
                                                   float scale, size_t rows, size_t vocab,
                                                   size_t cols, flint_stream stream) {
    constexpr const char* name = "flint_softmax_cross_entropy";
    if (cols == 0 || cols % 8 != 0 || cols > flint::kCrossEntropyMaxCols) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT,
                    "%s: cols (%zu) must be a multiple of 8 from 8 to %zu", name, cols,
                    flint::kCrossEntropyMaxCols);
    }
    if (vocab == 0 || vocab > cols) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: vocab (%zu) must be from 1 to cols (%zu)",
                    name, vocab, cols);
    }
    if (rows > flint::kCrossEntropyMaxRows) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: rows (%zu) can be up to %zu", name, rows,
                    flint::kCrossEntropyMaxRows);
    }
    if (!std::isfinite(scale)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: scale (%g) must be finite", name,
                    static_cast<double>(scale));
    }
    if (rows == 0) return FLINT_OK;
    const flint::Buffer buffers[] = {
        {"dlogits", dlogits, rows * cols * 2},
        {"row_loss", row_loss, rows * 4},
        {"logits", logits, rows * cols * 2},
        {"targets", targets, rows * 2},
    };
    if (flint_status s = flint::check_buffers(name, buffers, std::size(buffers), 2); s != FLINT_OK) {
        return s;
    }
    FLINT_HIP_CHECK(flint::launch_softmax_cross_entropy(dlogits, row_loss, logits, targets, scale,
                                                        rows, vocab, cols, flint::to_hip(stream)));
    return FLINT_OK;
}

}  // extern "C"
