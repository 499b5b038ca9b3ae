// C-ABI entry points of the GEMM family.
//
// Each entry point is one row of a table (kEntries): its name, the operand
// layout, the element size of y and which extra buffers it takes. One
// validator walks a row's rules in the order the reference reports them
// (ref src/api/gemm.cpp:24-168; its tests match the order and the message
// texts), then the entry point makes one launcher call.
#include <cmath>

#include "common/args.h"
#include "kernels/kernels.h"

namespace {

using flint::Checker;
using flint::Span;

enum Shape { kNt, kNn, kTn, kNtBatched, kNnBatched, kTnBatched };
enum Extra : unsigned { kNoExtra = 0, kBias = 1, kPre = 2, kResidual = 4, kCrossPre = 8 };

struct Entry {
    const char* name;
    Shape shape;
    size_t y_elem;      // bytes per element of y
    unsigned extras;
};

constexpr Entry kGemmNt{"flint_gemm_nt", kNt, 2, kNoExtra};
constexpr Entry kGemmNtBias{"flint_gemm_nt_bias", kNt, 2, kBias};
constexpr Entry kGemmNtBiasGelu{"flint_gemm_nt_bias_gelu", kNt, 2, kBias | kPre | kCrossPre};
constexpr Entry kGemmNtBiasResidual{"flint_gemm_nt_bias_residual", kNt, 4, kBias | kResidual};
constexpr Entry kGemmNn{"flint_gemm_nn", kNn, 2, kNoExtra};
constexpr Entry kGemmNnDGelu{"flint_gemm_nn_dgelu", kNn, 2, kPre};
constexpr Entry kGemmTn{"flint_gemm_tn", kTn, 4, kNoExtra};
constexpr Entry kGemmNtBatched{"flint_gemm_nt_batched", kNtBatched, 2, kNoExtra};
constexpr Entry kGemmNnBatched{"flint_gemm_nn_batched", kNnBatched, 2, kNoExtra};
constexpr Entry kGemmTnBatched{"flint_gemm_tn_batched", kTnBatched, 2, kNoExtra};

// Everything one call hands over.
struct Call {
    void* y;
    const void* x;
    const void* w;
    const void* bias = nullptr;
    const void* pre = nullptr;        // GELU's stored sums (written or read)
    const void* residual = nullptr;
    size_t batches = 1, m = 0, n = 0, k = 0;
    float scale = 1.0f;
};

constexpr size_t kMaxMN = flint::kGemmMaxMN;
constexpr size_t kMaxK = flint::kGemmMaxK;

// TN's sizes: k is a row count (any positive value); m and n are the rows of
// x and w moved in 16-byte chunks.
void tn_sizes(Checker& c, const Call& a) {
    c.require(a.k != 0, "k must be positive")
        .require(a.m % 8 == 0, "m (%zu) must be a multiple of 8", a.m)
        .require(a.n % 8 == 0, "n (%zu) must be a multiple of 8", a.n)
        .require(a.m <= kMaxMN && a.n <= kMaxMN && a.k <= kMaxK,
                 "%zu x %zu x %zu is too large: m and n can be up to %zu, and k up to %zu", a.m,
                 a.n, a.k, kMaxMN, kMaxK);
}

// NT's and NN's k (a multiple of 8: rows of x and w move in 16-byte chunks),
// and NN's n (w's rows, n long, move in chunks too).
void chunked_k(Checker& c, const Call& a, bool n_in_chunks) {
    c.require(a.k != 0 && a.k % 8 == 0, "k (%zu) must be a positive multiple of 8", a.k)
        .require(!n_in_chunks || a.n % 8 == 0, "n (%zu) must be a multiple of 8", a.n);
}

flint_status validate(const Entry& e, const Call& a) {
    Checker c(e.name);
    const size_t per = a.batches;
    const Span y{"y", a.y, per * a.m * a.n * e.y_elem};
    const Span x{"x", a.x, per * a.m * a.k * 2};
    const Span w{"w", a.w, per * a.n * a.k * 2};
    switch (e.shape) {
    case kNt:
    case kNn:
        chunked_k(c, a, e.shape == kNn);
        c.require(a.m <= kMaxMN && a.n <= kMaxMN && a.k <= kMaxK,
                  "%zu x %zu x %zu is too large: m and n can be up to %zu, and k up to %zu", a.m,
                  a.n, a.k, kMaxMN, kMaxK);
        c.operands({y, x, w}).apart(y, {x, w});
        break;
    case kTn:
        tn_sizes(c, a);
        c.operands({y, x, w}).apart(y, {x, w});
        break;
    case kNtBatched:
    case kNnBatched:
    case kTnBatched:
        if (e.shape == kTnBatched) {
            tn_sizes(c, a);
        } else {
            chunked_k(c, a, e.shape == kNnBatched);
            c.require(a.n <= kMaxMN && a.k <= kMaxK, "n (%zu) can be up to %zu, and k (%zu) up to %zu",
                      a.n, kMaxMN, a.k, kMaxK);
        }
        if (e.shape == kNtBatched)
            c.require(std::isfinite(a.scale), "scale (%g) must be finite", double(a.scale));
        c.require(a.batches <= flint::kGemmMaxBatches, "batches (%zu) can be up to %zu", a.batches,
                  flint::kGemmMaxBatches)
            .require(a.m <= flint::kGemmBatchedMaxM, "m (%zu) can be up to %zu", a.m,
                     flint::kGemmBatchedMaxM)
            .buffers({y, x, w}, 1);
        break;
    }
    if (e.extras & kResidual) c.require(a.n % 2 == 0, "n (%zu) must be even", a.n);
    const Span bias{"bias", a.bias, a.n * 4};
    if (e.extras & kBias) c.operands({bias}).apart(y, {bias});
    if (e.extras & kPre) {
        const Span pre{"pre", a.pre, a.m * a.n * 2};
        c.operands({pre}).apart(y, {pre});
        // pre is an output of the forward epilogue: it must miss the inputs too.
        if (e.extras & kCrossPre) c.apart(pre, {x, w, bias});
    }
    if (e.extras & kResidual) {
        const Span residual{"residual", a.residual, a.m * a.n * 4};
        c.operands({residual}).apart(y, {residual});
    }
    return c.status();
}

}  // namespace

#define FLINT_VALIDATE(entry, call)                                        \
    do {                                                                   \
        if (const flint_status s_ = validate(entry, call); s_ != FLINT_OK) \
            return s_;                                                     \
    } while (0)

extern "C" {

// m or n of 0 is an empty product: OK before any check, null pointers
// included (ref src/api/gemm.cpp:174-176).

FLINT_API flint_status flint_gemm_nt(void* y, const void* x, const void* w, size_t m, size_t n,
                                     size_t k, flint_stream stream) {
    if (m == 0 || n == 0) return FLINT_OK;
    FLINT_VALIDATE(kGemmNt, (Call{y, x, w, nullptr, nullptr, nullptr, 1, m, n, k}));
    FLINT_HIP_CHECK(flint::launch_gemm_nt(y, x, w, nullptr, nullptr, flint::Epilogue::kNone, m, n,
                                          k, flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_nt_bias(void* y, const void* x, const void* w, const void* bias,
                                          size_t m, size_t n, size_t k, flint_stream stream) {
    if (m == 0 || n == 0) return FLINT_OK;
    FLINT_VALIDATE(kGemmNtBias, (Call{y, x, w, bias, nullptr, nullptr, 1, m, n, k}));
    FLINT_HIP_CHECK(flint::launch_gemm_nt(y, x, w, bias, nullptr, flint::Epilogue::kBias, m, n, k,
                                          flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_nt_bias_gelu(void* y, void* pre, const void* x, const void* w,
                                               const void* bias, size_t m, size_t n, size_t k,
                                               flint_stream stream) {
    if (m == 0 || n == 0) return FLINT_OK;
    FLINT_VALIDATE(kGemmNtBiasGelu, (Call{y, x, w, bias, pre, nullptr, 1, m, n, k}));
    FLINT_HIP_CHECK(flint::launch_gemm_nt(y, x, w, bias, pre, flint::Epilogue::kBiasGelu, m, n, k,
                                          flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_nt_bias_residual(void* y, const void* x, const void* w,
                                                   const void* bias, const void* residual,
                                                   size_t m, size_t n, size_t k,
                                                   flint_stream stream) {
    if (m == 0 || n == 0) return FLINT_OK;
    FLINT_VALIDATE(kGemmNtBiasResidual, (Call{y, x, w, bias, nullptr, residual, 1, m, n, k}));
    FLINT_HIP_CHECK(flint::launch_gemm_nt(y, x, w, bias, const_cast<void*>(residual),
                                          flint::Epilogue::kBiasResidual, m, n, k,
                                          flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_nn(void* y, const void* x, const void* w, size_t m, size_t n,
                                     size_t k, flint_stream stream) {
    if (m == 0 || n == 0) return FLINT_OK;
    FLINT_VALIDATE(kGemmNn, (Call{y, x, w, nullptr, nullptr, nullptr, 1, m, n, k}));
    FLINT_HIP_CHECK(flint::launch_gemm_nn(y, x, w, nullptr, flint::Epilogue::kNone, m, n, k,
                                          flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_nn_dgelu(void* y, const void* x, const void* w,
                                           const void* pre, size_t m, size_t n, size_t k,
                                           flint_stream stream) {
    if (m == 0 || n == 0) return FLINT_OK;
    FLINT_VALIDATE(kGemmNnDGelu, (Call{y, x, w, nullptr, pre, nullptr, 1, m, n, k}));
    FLINT_HIP_CHECK(flint::launch_gemm_nn(y, x, w, pre, flint::Epilogue::kDGelu, m, n, k,
                                          flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_tn_workspace(size_t m, size_t n, size_t k, size_t* bytes) {
    Checker c("flint_gemm_tn_workspace");
    if (!c.require(bytes != nullptr, "bytes is null").ok()) return c.status();
    *bytes = 0;
    if (m == 0 || n == 0) return FLINT_OK;
    tn_sizes(c, Call{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 1, m, n, k});
    if (!c.ok()) return c.status();
    FLINT_HIP_CHECK(flint::gemm_tn_workspace(m, n, k, bytes));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_tn(void* y, const void* x, const void* w, size_t m, size_t n,
                                     size_t k, int accumulate, void* workspace,
                                     size_t workspace_bytes, flint_stream stream) {
    if (m == 0 || n == 0) return FLINT_OK;
    const Call call{y, x, w, nullptr, nullptr, nullptr, 1, m, n, k};
    FLINT_VALIDATE(kGemmTn, call);
    size_t needed = 0;
    FLINT_HIP_CHECK(flint::gemm_tn_workspace(m, n, k, &needed));
    Checker c(kGemmTn.name);
    c.workspace(workspace, workspace_bytes, needed);
    if (needed > 0) {
        const Span ws{"workspace", workspace, needed};
        c.require(!ws.meets({"y", y, m * n * 4}) && !ws.meets({"x", x, k * m * 2}) &&
                      !ws.meets({"w", w, k * n * 2}),
                  "workspace overlaps y, x or w");
    }
    if (!c.ok()) return c.status();
    FLINT_HIP_CHECK(flint::launch_gemm_tn(y, x, w, m, n, k, accumulate != 0, workspace,
                                          flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_nt_batched(void* y, const void* x, const void* w, size_t batches,
                                             size_t m, size_t n, size_t k, float scale,
                                             flint_stream stream) {
    if (batches == 0 || m == 0 || n == 0) return FLINT_OK;
    FLINT_VALIDATE(kGemmNtBatched, (Call{y, x, w, nullptr, nullptr, nullptr, batches, m, n, k, scale}));
    FLINT_HIP_CHECK(flint::launch_gemm_nt_batched(y, x, w, batches, m, n, k, scale,
                                                  flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_nn_batched(void* y, const void* x, const void* w, size_t batches,
                                             size_t m, size_t n, size_t k, flint_stream stream) {
    if (batches == 0 || m == 0 || n == 0) return FLINT_OK;
    FLINT_VALIDATE(kGemmNnBatched, (Call{y, x, w, nullptr, nullptr, nullptr, batches, m, n, k}));
    FLINT_HIP_CHECK(flint::launch_gemm_nn_batched(y, x, w, batches, m, n, k,
                                                  flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_gemm_tn_batched(void* y, const void* x, const void* w, size_t batches,
                                             size_t m, size_t n, size_t k, flint_stream stream) {
    if (batches == 0 || m == 0 || n == 0) return FLINT_OK;
    FLINT_VALIDATE(kGemmTnBatched, (Call{y, x, w, nullptr, nullptr, nullptr, batches, m, n, k}));
    FLINT_HIP_CHECK(flint::launch_gemm_tn_batched(y, x, w, batches, m, n, k,
                                                  flint::to_hip(stream)));
    return FLINT_OK;
}

}  // extern "C"
