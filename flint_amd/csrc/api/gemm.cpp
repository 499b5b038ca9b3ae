// C-ABI entry points of the GEMM family: argument checks (order and message
// text as the reference's src/api/gemm.cpp:24-168 has them, which its tests
// match verbatim), then one launcher call.
#include <cmath>
#include <iterator>

#include "common/common.h"
#include "kernels/kernels.h"

namespace {

using flint::aligned16;
using flint::fail;
using flint::fits;
using flint::overlap;

// NT's and NN's checks for m, n > 0 (ref src/api/gemm.cpp:27-67). w holds n*k
// halves in both layouts; NN moves w's rows (n long) in 16-byte chunks, so n
// must be a multiple of 8 there. y has y_element bytes per value.
flint_status check_nt_nn(const char* name, bool n_in_chunks, void* y, const void* x,
                         const void* w, size_t m, size_t n, size_t k, size_t y_element = 2) {
    if (k == 0 || k % 8 != 0) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: k (%zu) must be a positive multiple of 8",
                    name, k);
    }
    if (n_in_chunks && n % 8 != 0) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: n (%zu) must be a multiple of 8", name, n);
    }
    if (m > flint::kGemmMaxMN || n > flint::kGemmMaxMN || k > flint::kGemmMaxK) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT,
                    "%s: %zu x %zu x %zu is too large: m and n can be up to %zu, and k up to %zu",
                    name, m, n, k, flint::kGemmMaxMN, flint::kGemmMaxK);
    }
    if (y == nullptr || x == nullptr || w == nullptr) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: %s is null", name,
                    y == nullptr ? "y" : x == nullptr ? "x" : "w");
    }
    if (!aligned16(y) || !aligned16(x) || !aligned16(w)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: %s is not 16-byte aligned", name,
                    !aligned16(y) ? "y" : !aligned16(x) ? "x" : "w");
    }
    const size_t y_bytes = m * n * y_element;
    const size_t x_bytes = m * k * 2;
    const size_t w_bytes = n * k * 2;
    if (!fits(y, y_bytes) || !fits(x, x_bytes) || !fits(w, w_bytes)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: %s runs past the end of the address space",
                    name, !fits(y, y_bytes) ? "y" : !fits(x, x_bytes) ? "x" : "w");
    }
    if (overlap(y, y_bytes, x, x_bytes)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: y and x overlap", name);
    }
    if (overlap(y, y_bytes, w, w_bytes)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: y and w overlap", name);
    }
    return FLINT_OK;
}

flint_status check_bias(const char* name, const void* y, const void* bias, size_t m, size_t n,
                        size_t y_element = 2) {
    if (bias == nullptr) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: bias is null", name);
    }
    if (!aligned16(bias)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: bias is not 16-byte aligned", name);
    }
    const size_t bias_bytes = n * 4;
    if (!fits(bias, bias_bytes)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: bias runs past the end of the address space",
                    name);
    }
    if (overlap(y, m * n * y_element, bias, bias_bytes)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: y and bias overlap", name);
    }
    return FLINT_OK;
}

flint_status check_pre(const char* name, const void* y, const void* pre, size_t m, size_t n) {
    if (pre == nullptr) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: pre is null", name);
    }
    if (!aligned16(pre)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: pre is not 16-byte aligned", name);
    }
    const size_t pre_bytes = m * n * 2;
    if (!fits(pre, pre_bytes)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: pre runs past the end of the address space",
                    name);
    }
    if (overlap(pre, pre_bytes, y, pre_bytes)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: y and pre overlap", name);
    }
    return FLINT_OK;
}

// TN: x (k x m) and w (k x n) move in 16-byte chunks along m and n; k, their
// row count, can be anything from 1 (ref src/api/gemm.cpp:114-129).
flint_status check_tn_dims(const char* name, size_t m, size_t n, size_t k) {
    if (k == 0) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: k must be positive", name);
    }
    if (m % 8 != 0 || n % 8 != 0) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: %s (%zu) must be a multiple of 8", name,
                    m % 8 != 0 ? "m" : "n", m % 8 != 0 ? m : n);
    }
    if (m > flint::kGemmMaxMN || n > flint::kGemmMaxMN || k > flint::kGemmMaxK) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT,
                    "%s: %zu x %zu x %zu is too large: m and n can be up to %zu, and k up to %zu",
                    name, m, n, k, flint::kGemmMaxMN, flint::kGemmMaxK);
    }
    return FLINT_OK;
}

flint_status check_batched(const char* name, void* y, const void* x, const void* w,
                           size_t batches, size_t m, size_t n, size_t k) {
    if (batches > flint::kGemmMaxBatches) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: batches (%zu) can be up to %zu", name,
                    batches, flint::kGemmMaxBatches);
    }
    if (m > flint::kGemmBatchedMaxM) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: m (%zu) can be up to %zu", name, m,
                    flint::kGemmBatchedMaxM);
    }
    const flint::Buffer buffers[] = {
        {"y", y, batches * m * n * 2},
        {"x", x, batches * m * k * 2},
        {"w", w, batches * n * k * 2},
    };
    return flint::check_buffers(name, buffers, std::size(buffers), 1);
}

flint_status check_batched_nt_nn(const char* name, bool n_in_chunks, size_t n, size_t k) {
    if (k == 0 || k % 8 != 0) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: k (%zu) must be a positive multiple of 8",
                    name, k);
    }
    if (n_in_chunks && n % 8 != 0) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: n (%zu) must be a multiple of 8", name, n);
    }
    if (n > flint::kGemmMaxMN || k > flint::kGemmMaxK) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: n (%zu) can be up to %zu, and k (%zu) up to %zu",
                    name, n, flint::kGemmMaxMN, k, flint::kGemmMaxK);
    }
    return FLINT_OK;
}

}  // namespace

extern "C" {

FLINT_API flint_status flint_gemm_nt(void* y, const void* x, const void* w, size_t m, size_t n,
                                     size_t k, flint_stream stream) {
    if (m == 0 || n == 0) return FLINT_OK;
    if (flint_status s = check_nt_nn("flint_gemm_nt", false, y, x, w, m, n, k); s != FLINT_OK) {
        return s;
    }
    FLINT_HIP_CHECK(flint::launch_gemm_nt(y, x, w, nullptr, nullptr, flint::Epilogue::kNone, m, n,
                                          k, flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_nt_bias(void* y, const void* x, const void* w, const void* bias,
                                          size_t m, size_t n, size_t k, flint_stream stream) {
    if (m == 0 || n == 0) return FLINT_OK;
    constexpr const char* name = "flint_gemm_nt_bias";
    if (flint_status s = check_nt_nn(name, false, y, x, w, m, n, k); s != FLINT_OK) return s;
    if (flint_status s = check_bias(name, y, bias, m, n); s != FLINT_OK) return s;
    FLINT_HIP_CHECK(flint::launch_gemm_nt(y, x, w, bias, nullptr, flint::Epilogue::kBias, m, n, k,
                                          flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_nt_bias_gelu(void* y, void* pre, const void* x, const void* w,
                                               const void* bias, size_t m, size_t n, size_t k,
                                               flint_stream stream) {
    if (m == 0 || n == 0) return FLINT_OK;
    constexpr const char* name = "flint_gemm_nt_bias_gelu";
    if (flint_status s = check_nt_nn(name, false, y, x, w, m, n, k); s != FLINT_OK) return s;
    if (flint_status s = check_bias(name, y, bias, m, n); s != FLINT_OK) return s;
    if (flint_status s = check_pre(name, y, pre, m, n); s != FLINT_OK) return s;
    const size_t pre_bytes = m * n * 2;
    if (overlap(pre, pre_bytes, x, m * k * 2)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: pre and x overlap", name);
    }
    if (overlap(pre, pre_bytes, w, n * k * 2)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: pre and w overlap", name);
    }
    if (overlap(pre, pre_bytes, bias, n * 4)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: pre and bias overlap", name);
    }
    FLINT_HIP_CHECK(flint::launch_gemm_nt(y, x, w, bias, pre, flint::Epilogue::kBiasGelu, m, n, k,
                                          flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_nt_bias_residual(void* y, const void* x, const void* w,
                                                   const void* bias, const void* residual,
                                                   size_t m, size_t n, size_t k,
                                                   flint_stream stream) {
    if (m == 0 || n == 0) return FLINT_OK;
    constexpr const char* name = "flint_gemm_nt_bias_residual";
    if (flint_status s = check_nt_nn(name, false, y, x, w, m, n, k, 4); s != FLINT_OK) return s;
    if (n % 2 != 0) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: n (%zu) must be even", name, n);
    }
    if (flint_status s = check_bias(name, y, bias, m, n, 4); s != FLINT_OK) return s;
    if (residual == nullptr) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: residual is null", name);
    }
    if (!aligned16(residual)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: residual is not 16-byte aligned", name);
    }
    const size_t residual_bytes = m * n * 4;
    if (!fits(residual, residual_bytes)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT,
                    "%s: residual runs past the end of the address space", name);
    }
    if (overlap(y, residual_bytes, residual, residual_bytes)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: y and residual overlap", name);
    }
    FLINT_HIP_CHECK(flint::launch_gemm_nt(y, x, w, bias, const_cast<void*>(residual),
                                          flint::Epilogue::kBiasResidual, m, n, k,
                                          flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_nn(void* y, const void* x, const void* w, size_t m, size_t n,
                                     size_t k, flint_stream stream) {
    if (m == 0 || n == 0) return FLINT_OK;
    if (flint_status s = check_nt_nn("flint_gemm_nn", true, y, x, w, m, n, k); s != FLINT_OK) {
        return s;
    }
    FLINT_HIP_CHECK(flint::launch_gemm_nn(y, x, w, nullptr, flint::Epilogue::kNone, m, n, k,
                                          flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_nn_dgelu(void* y, const void* x, const void* w,
                                           const void* pre, size_t m, size_t n, size_t k,
                                           flint_stream stream) {
    if (m == 0 || n == 0) return FLINT_OK;
    constexpr const char* name = "flint_gemm_nn_dgelu";
    if (flint_status s = check_nt_nn(name, true, y, x, w, m, n, k); s != FLINT_OK) return s;
    if (flint_status s = check_pre(name, y, pre, m, n); s != FLINT_OK) return s;
    FLINT_HIP_CHECK(flint::launch_gemm_nn(y, x, w, pre, flint::Epilogue::kDGelu, m, n, k,
                                          flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_tn_workspace(size_t m, size_t n, size_t k, size_t* bytes) {
    if (bytes == nullptr) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "flint_gemm_tn_workspace: bytes is null");
    }
    *bytes = 0;
    if (m == 0 || n == 0) return FLINT_OK;
    if (flint_status s = check_tn_dims("flint_gemm_tn_workspace", m, n, k); s != FLINT_OK) {
        return s;
    }
    FLINT_HIP_CHECK(flint::gemm_tn_workspace(m, n, k, bytes));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_tn(void* y, const void* x, const void* w, size_t m, size_t n,
                                     size_t k, int accumulate, void* workspace,
                                     size_t workspace_bytes, flint_stream stream) {
    if (m == 0 || n == 0) return FLINT_OK;
    constexpr const char* name = "flint_gemm_tn";
    if (flint_status s = check_tn_dims(name, m, n, k); s != FLINT_OK) return s;
    if (y == nullptr || x == nullptr || w == nullptr) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: %s is null", name,
                    y == nullptr ? "y" : x == nullptr ? "x" : "w");
    }
    if (!aligned16(y) || !aligned16(x) || !aligned16(w)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: %s is not 16-byte aligned", name,
                    !aligned16(y) ? "y" : !aligned16(x) ? "x" : "w");
    }
    const size_t y_bytes = m * n * 4;
    const size_t x_bytes = k * m * 2;
    const size_t w_bytes = k * n * 2;
    if (!fits(y, y_bytes) || !fits(x, x_bytes) || !fits(w, w_bytes)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: %s runs past the end of the address space",
                    name, !fits(y, y_bytes) ? "y" : !fits(x, x_bytes) ? "x" : "w");
    }
    if (overlap(y, y_bytes, x, x_bytes)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: y and x overlap", name);
    }
    if (overlap(y, y_bytes, w, w_bytes)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: y and w overlap", name);
    }
    size_t needed = 0;
    FLINT_HIP_CHECK(flint::gemm_tn_workspace(m, n, k, &needed));
    if (needed > 0) {
        if (workspace == nullptr || workspace_bytes < needed) {
            return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: needs %zu bytes of workspace, given %zu",
                        name, needed, workspace == nullptr ? size_t{0} : workspace_bytes);
        }
        if (!aligned16(workspace)) {
            return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: workspace is not 16-byte aligned", name);
        }
        if (!fits(workspace, needed)) {
            return fail(FLINT_ERROR_INVALID_ARGUMENT,
                        "%s: workspace runs past the end of the address space", name);
        }
        if (overlap(workspace, needed, y, y_bytes) || overlap(workspace, needed, x, x_bytes) ||
            overlap(workspace, needed, w, w_bytes)) {
            return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: workspace overlaps y, x or w", name);
        }
    }
    FLINT_HIP_CHECK(flint::launch_gemm_tn(y, x, w, m, n, k, accumulate != 0, workspace,
                                          flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_nt_batched(void* y, const void* x, const void* w, size_t batches,
                                             size_t m, size_t n, size_t k, float scale,
                                             flint_stream stream) {
    if (batches == 0 || m == 0 || n == 0) return FLINT_OK;
    constexpr const char* name = "flint_gemm_nt_batched";
    if (flint_status s = check_batched_nt_nn(name, false, n, k); s != FLINT_OK) return s;
    if (!std::isfinite(scale)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: scale (%g) must be finite", name,
                    static_cast<double>(scale));
    }
    if (flint_status s = check_batched(name, y, x, w, batches, m, n, k); s != FLINT_OK) return s;
    FLINT_HIP_CHECK(flint::launch_gemm_nt_batched(y, x, w, batches, m, n, k, scale,
                                                  flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_nn_batched(void* y, const void* x, const void* w, size_t batches,
                                             size_t m, size_t n, size_t k, flint_stream stream) {
    if (batches == 0 || m == 0 || n == 0) return FLINT_OK;
    constexpr const char* name = "flint_gemm_nn_batched";
    if (flint_status s = check_batched_nt_nn(name, true, n, k); s != FLINT_OK) return s;
    if (flint_status s = check_batched(name, y, x, w, batches, m, n, k); s != FLINT_OK) return s;
    FLINT_HIP_CHECK(flint::launch_gemm_nn_batched(y, x, w, batches, m, n, k,
                                                  flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_tn_batched(void* y, const void* x, const void* w, size_t batches,
                                             size_t m, size_t n, size_t k, flint_stream stream) {
    if (batches == 0 || m == 0 || n == 0) return FLINT_OK;
    constexpr const char* name = "flint_gemm_tn_batched";
    if (flint_status s = check_tn_dims(name, m, n, k); s != FLINT_OK) return s;
    if (flint_status s = check_batched(name, y, x, w, batches, m, n, k); s != FLINT_OK) return s;
    FLINT_HIP_CHECK(flint::launch_gemm_tn_batched(y, x, w, batches, m, n, k,
                                                  flint::to_hip(stream)));
    return FLINT_OK;
}

}  // extern "C"
