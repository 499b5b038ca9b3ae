// GPT-2 assembled from the public C ABI: the model's device memory, its master
// weights (PyTorch named_parameters order and names), the FP16 compute copies,
// the forward pass to logits / row_loss / dlogits, and the backward pass to
// every master weight's gradient.
//
// The call sequence is the model's definition and the numerical contract of
// the reference (ref src/api/gpt2.cpp:495-618 for a block's forward and
// backward, :721-813 for the passes), so the order of the calls and their
// precisions match it. Everything else is this library's own: one bump-pointer
// allocation sized once (HBM holds every layer's activations at GPT-2 124M
// sizes many times over), every launch through the checked entry points but
// the attention products (the batched GEMMs' causal variants, below), and
// the one zero-fill the backward pass needs done by a kernel rather than a
// memset, so the pass can be captured in a HIP graph.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <iterator>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "common/args.h"
#include "common/tuning.h"
#include "kernels/kernels.h"

using flint::fail;

namespace {

constexpr size_t kAlign = 256;
constexpr float kLnEps = 1e-5f;   // GPT-2's LayerNorm eps

// Limits (ref src/api/gpt2.cpp:24-43): the ABI's per-call limits seen from the model.
constexpr size_t kMaxLayers = 1024;
constexpr size_t kMaxWidth = 16384;
constexpr size_t kMaxLength = 1024;
constexpr size_t kMaxHeadBatches = 65535;
constexpr size_t kMaxPaddedVocab = 65536;
constexpr size_t kMaxRows = size_t{65535} * 128;
constexpr size_t kMaxBackwardRows = 65536;
constexpr size_t kMaxBackwardPositionValues = 16776960;

#define FLINT_TRY(call)                               \
    do {                                              \
        const flint_status flint_try_ = (call);       \
        if (flint_try_ != FLINT_OK) return flint_try_; \
    } while (0)

struct Param {
    std::string name;
    size_t rows, cols;
    void* data = nullptr;
    void* grad = nullptr;
};

struct Linear {
    Param* w;
    Param* b;
    void* half = nullptr;   // FP16 compute copy of w
};

struct Norm {
    Param* w;
    Param* b;
};

// What a block keeps for its backward pass (with backward one set per block;
// without, one shared set).
struct Saved {
    void *x_in = nullptr, *x_mid = nullptr, *x_out = nullptr;
    void *h1 = nullptr, *mean1 = nullptr, *rstd1 = nullptr;
    void *q = nullptr, *k = nullptr, *v = nullptr, *p = nullptr;
    // Fused attention: the qkv projection itself ([rows][3 width], whose
    // heads the kernels read in place) and the log-sum-exp.
    void *qkv = nullptr, *lse = nullptr;
    void* attn_out = nullptr;
    void *h2 = nullptr, *mean2 = nullptr, *rstd2 = nullptr;
    void *gelu = nullptr, *pre = nullptr;
};

struct Layer {
    Norm ln_1;
    Linear attn, attn_proj;
    Norm ln_2;
    Linear fc, fc_proj;
    Saved s;
};

struct Request {
    void** where;
    size_t bytes;
};

size_t round_up(size_t b) { return (b + kAlign - 1) / kAlign * kAlign; }

}  // namespace

// How the default model's attention holds its per-head operands: split and
// merged by copies (flint_heads_split / _merge, the reference's sequence), or
// as heads views of the token rows. The same bits either way.
enum class AttnPlan : int { kCopies, kViews };

struct flint_gpt2 {
    flint_gpt2_config cfg{};
    size_t rows = 0, head_width = 0, head_batches = 0;
    // Fused attention (attention.hip) in place of the stored scores and
    // probabilities: chosen at creation (flint_gpt2_create_fused), head width 64.
    bool flash = false;
    void* attn_work = nullptr;   // the fused backward's D
    std::deque<Param> params;   // stable addresses
    Param* wte = nullptr;
    Param* wpe = nullptr;
    void* wte_half = nullptr;
    std::vector<Layer> layers;
    Norm ln_f{};
    void *x_final = nullptr, *h_f = nullptr, *mean_f = nullptr, *rstd_f = nullptr;
    void *qkv = nullptr, *scores = nullptr, *heads_out = nullptr;
    void *logits = nullptr, *dlogits = nullptr, *row_loss = nullptr;
    void *dres = nullptr, *dres_half = nullptr, *dh = nullptr, *dpre = nullptr;
    void *dq = nullptr, *dk = nullptr, *dv = nullptr;
    void* work = nullptr;
    size_t work_bytes = 0;
    void* tn_work = nullptr;
    size_t tn_work_bytes = 0;
    // LayerNorm backward's chunk partials sit in `work` past the first
    // ln_offset bytes, where a linear layer's bias partials of up to
    // ln_offset bytes leave them alone: their merge is then deferred to the
    // next linear layer's gradient finish; `pending` describes it. ln_offset
    // is 0 when the two do not fit side by side in `work` (the merge then
    // runs at once).
    size_t ln_offset = 0;
    mutable flint::ParamsMerge pending{};
    // The attention plan of the last forward, which its backward follows
    // (plan overrides may change in between).
    AttnPlan attn_plan = AttnPlan::kCopies;
    std::vector<Request> requests;
    std::vector<void*> blocks;   // hipMalloc'd allocations
    std::vector<float> host_loss;

    flint_gpt2() = default;
    flint_gpt2(const flint_gpt2&) = delete;
    flint_gpt2& operator=(const flint_gpt2&) = delete;
    ~flint_gpt2() {
        for (void* b : blocks) (void)hipFree(b);
        (void)hipGetLastError();
    }
};

namespace {

// The configuration's limits, in the order and words the reference reports
// them (ref src/api/gpt2.cpp:187-243). A link's condition is evaluated even
// after an earlier one failed (only the first failure is reported), so each
// guards its own divisions.
flint_status check_config(const char* name, const flint_gpt2_config* config) {
    flint::Checker ck(name);
    if (!ck.require(config != nullptr, "config is null").ok()) return ck.status();
    const flint_gpt2_config& c = *config;
    ck.require(c.layers != 0 && c.layers <= kMaxLayers, "layers (%zu) must be from 1 to %zu",
               c.layers, kMaxLayers)
        .require(c.width != 0 && c.width % 8 == 0 && c.width <= kMaxWidth,
                 "width (%zu) must be a multiple of 8 from 8 to %zu", c.width, kMaxWidth)
        .require(c.heads != 0 && c.width % c.heads == 0 && (c.width / c.heads) % 8 == 0,
                 "heads (%zu) must split width (%zu) into multiples of 8", c.heads, c.width)
        .require(c.length != 0 && c.length % 8 == 0 && c.length <= kMaxLength,
                 "length (%zu) must be a multiple of 8 from 8 to %zu", c.length, kMaxLength)
        .require(c.block_size >= c.length && c.block_size <= kMaxLength,
                 "block_size (%zu) must be from length (%zu) to %zu", c.block_size, c.length,
                 kMaxLength)
        .require(c.padded_vocab != 0 && c.padded_vocab % 8 == 0 && c.padded_vocab <= kMaxPaddedVocab,
                 "padded_vocab (%zu) must be a multiple of 8 from 8 to %zu", c.padded_vocab,
                 kMaxPaddedVocab)
        .require(c.vocab != 0 && c.vocab <= c.padded_vocab,
                 "vocab (%zu) must be from 1 to padded_vocab (%zu)", c.vocab, c.padded_vocab)
        .require(c.sequences != 0 && c.heads != 0 && c.sequences <= kMaxHeadBatches / c.heads,
                 "sequences (%zu) x heads (%zu) must be from 1 to %zu", c.sequences, c.heads,
                 kMaxHeadBatches)
        .require(c.length != 0 && c.sequences <= kMaxRows / c.length,
                 "sequences (%zu) x length (%zu) can be up to %zu rows", c.sequences, c.length,
                 kMaxRows);
    if (c.backward != 0) {
        ck.require(c.length != 0 && c.sequences <= kMaxBackwardRows / c.length,
                   "sequences (%zu) x length (%zu) can be up to %zu rows with backward",
                   c.sequences, c.length, kMaxBackwardRows)
            .require(c.width != 0 && c.length <= kMaxBackwardPositionValues / c.width,
                     "length (%zu) x width (%zu) can be up to %zu with backward", c.length,
                     c.width, kMaxBackwardPositionValues);
    }
    return ck.status();
}

Param* param(flint_gpt2& m, std::string name, size_t rows, size_t cols) {
    m.params.push_back(Param{std::move(name), rows, cols});
    Param* p = &m.params.back();
    m.requests.push_back({&p->data, rows * cols * 4});
    return p;
}

// Sizes of the shared workspaces: the bias gradient / LayerNorm / embedding one,
// and flint_gemm_tn's over every weight-gradient shape (k = rows).
flint_status size_workspaces(flint_gpt2& m) {
    const flint_gpt2_config& c = m.cfg;
    const size_t w = c.width;
    size_t need = 0, b = 0;
    for (size_t cols : {w, 3 * w, 4 * w}) {
        FLINT_TRY(flint_bias_gradient_workspace(m.rows, cols, &b));
        need = std::max(need, b);
    }
    size_t ln = 0, bias_w = 0;
    FLINT_TRY(flint_layernorm_backward_workspace(m.rows, w, &ln));
    need = std::max(need, ln);
    FLINT_TRY(flint_embedding_backward_workspace(c.sequences, c.length, c.padded_vocab, w, &b));
    m.work_bytes = std::max(need, b);
    // The linear layer after a LayerNorm backward (attention projection, MLP
    // down) has width-wide bias partials.
    FLINT_TRY(flint_bias_gradient_workspace(m.rows, w, &bias_w));
    m.ln_offset = round_up(bias_w) + ln <= m.work_bytes ? round_up(bias_w) : 0;
    const size_t shapes[][2] = {{c.padded_vocab, w}, {3 * w, w}, {w, w}, {4 * w, w}, {w, 4 * w}};
    need = 0;
    for (const auto& s : shapes) {
        FLINT_TRY(flint_gemm_tn_workspace(s[0], s[1], m.rows, &b));
        need = std::max(need, b);
    }
    m.tn_work_bytes = need;
    return FLINT_OK;
}

// Declares every parameter (named_parameters order), gradient, compute copy,
// activation and scratch buffer as a request; allocation comes after. With
// m.flash set (by the caller) the attention keeps the qkv projection and the
// log-sum-exp instead of q, k, v and the probabilities.
flint_status plan(flint_gpt2& m) {
    const flint_gpt2_config& c = m.cfg;
    const bool bwd = c.backward != 0;
    const size_t w = c.width;
    m.rows = c.sequences * c.length;
    m.head_width = w / c.heads;
    m.head_batches = c.sequences * c.heads;

    m.wte = param(m, "wte.weight", c.padded_vocab, w);
    m.wpe = param(m, "wpe.weight", c.block_size, w);
    m.layers.resize(c.layers);
    for (size_t i = 0; i < c.layers; ++i) {
        const std::string pre = "blocks." + std::to_string(i) + ".";
        Layer& L = m.layers[i];
        L.ln_1 = {param(m, pre + "ln_1.weight", 1, w), param(m, pre + "ln_1.bias", 1, w)};
        L.attn = {param(m, pre + "attn.c_attn.weight", 3 * w, w),
                  param(m, pre + "attn.c_attn.bias", 1, 3 * w)};
        L.attn_proj = {param(m, pre + "attn.c_proj.weight", w, w),
                       param(m, pre + "attn.c_proj.bias", 1, w)};
        L.ln_2 = {param(m, pre + "ln_2.weight", 1, w), param(m, pre + "ln_2.bias", 1, w)};
        L.fc = {param(m, pre + "mlp.c_fc.weight", 4 * w, w),
                param(m, pre + "mlp.c_fc.bias", 1, 4 * w)};
        L.fc_proj = {param(m, pre + "mlp.c_proj.weight", w, 4 * w),
                     param(m, pre + "mlp.c_proj.bias", 1, w)};
    }
    m.ln_f = {param(m, "ln_f.weight", 1, w), param(m, "ln_f.bias", 1, w)};
    if (bwd) {
        for (Param& p : m.params) m.requests.push_back({&p.grad, p.rows * p.cols * 4});
    }
    m.requests.push_back({&m.wte_half, c.padded_vocab * w * 2});
    for (Layer& L : m.layers) {
        for (Linear* lin : {&L.attn, &L.attn_proj, &L.fc, &L.fc_proj})
            m.requests.push_back({&lin->half, lin->w->rows * lin->w->cols * 2});
    }

    const size_t rows = m.rows;
    const size_t resid = rows * w * 4;
    const size_t half_rows = rows * w * 2;
    const size_t heads = m.head_batches * c.length * m.head_width * 2;
    const size_t matrix = m.head_batches * c.length * c.length * 2;
    auto req = [&](void** p, size_t b) { m.requests.push_back({p, b}); };
    if (bwd) {
        for (Layer& L : m.layers) {
            req(&L.s.x_in, resid);
            req(&L.s.x_mid, resid);
        }
        req(&m.x_final, resid);
        for (Layer& L : m.layers) {
            Saved& s = L.s;
            req(&s.h1, half_rows);
            req(&s.mean1, rows * 4);
            req(&s.rstd1, rows * 4);
            if (m.flash) {
                req(&s.qkv, rows * 3 * w * 2);
                req(&s.lse, m.head_batches * c.length * 4);
            } else {
                req(&s.q, heads);
                req(&s.k, heads);
                req(&s.v, heads);
                req(&s.p, matrix);
            }
            req(&s.attn_out, half_rows);
            req(&s.h2, half_rows);
            req(&s.mean2, rows * 4);
            req(&s.rstd2, rows * 4);
            req(&s.gelu, rows * 4 * w * 2);
            req(&s.pre, rows * 4 * w * 2);
        }
        req(&m.h_f, half_rows);
        req(&m.mean_f, rows * 4);
        req(&m.rstd_f, rows * 4);
        req(&m.qkv, rows * 3 * w * 2);
        if (m.flash) {
            req(&m.attn_work, m.head_batches * c.length * 4);
        } else {
            req(&m.scores, matrix);
            req(&m.heads_out, heads);
            req(&m.dq, heads);
            req(&m.dk, heads);
            req(&m.dv, heads);
        }
        FLINT_TRY(size_workspaces(m));
        req(&m.dres, resid);
        req(&m.dres_half, half_rows);
        req(&m.dh, half_rows);
        req(&m.dpre, rows * 4 * w * 2);
        req(&m.work, m.work_bytes);
        req(&m.tn_work, m.tn_work_bytes);
    } else {
        Saved& s = m.layers[0].s;
        req(&s.x_in, resid);
        req(&s.x_mid, resid);
        req(&s.h1, half_rows);
        req(&s.mean1, rows * 4);
        req(&s.rstd1, rows * 4);
        req(&m.qkv, rows * 3 * w * 2);
        if (m.flash) {
            req(&s.lse, m.head_batches * c.length * 4);
        } else {
            req(&s.q, heads);
            req(&s.k, heads);
            req(&s.v, heads);
            req(&m.scores, matrix);
            req(&s.p, matrix);
            req(&m.heads_out, heads);
        }
        req(&s.attn_out, half_rows);
        req(&s.gelu, rows * 4 * w * 2);
        req(&s.pre, rows * 4 * w * 2);
    }
    req(&m.logits, rows * c.padded_vocab * 2);
    req(&m.dlogits, rows * c.padded_vocab * 2);
    req(&m.row_loss, rows * 4);
    return FLINT_OK;
}

// Pointers that alias other buffers: with backward a block's output is the
// next block's input; without, every block shares block 0's set.
void link(flint_gpt2& m) {
    if (m.cfg.backward != 0) {
        for (size_t i = 0; i < m.layers.size(); ++i)
            m.layers[i].s.x_out = i + 1 < m.layers.size() ? m.layers[i + 1].s.x_in : m.x_final;
        return;
    }
    Saved& s = m.layers[0].s;
    s.x_out = s.x_in;
    s.h2 = s.h1;
    s.mean2 = s.mean1;
    s.rstd2 = s.rstd1;
    for (Layer& L : m.layers) L.s = s;
    m.x_final = s.x_in;
    m.h_f = s.h1;
    m.mean_f = s.mean1;
    m.rstd_f = s.rstd1;
}

size_t total_bytes(const flint_gpt2& m) {
    size_t t = 0;
    for (const Request& r : m.requests) t += round_up(r.bytes);
    return t;
}

flint_status allocate(flint_gpt2& m) {
    m.blocks.reserve(m.requests.size());
    if (m.cfg.separate_buffers != 0) {
        for (const Request& r : m.requests) {
            void* p = nullptr;
            FLINT_HIP_CHECK(hipMalloc(&p, std::max<size_t>(r.bytes, 1)));
            m.blocks.push_back(p);
            *r.where = p;
        }
        return FLINT_OK;
    }
    void* base = nullptr;
    FLINT_HIP_CHECK(hipMalloc(&base, total_bytes(m)));
    m.blocks.push_back(base);
    char* at = static_cast<char*>(base);
    for (const Request& r : m.requests) {
        *r.where = at;
        at += round_up(r.bytes);
    }
    return FLINT_OK;
}

float score_scale(size_t head_width) { return 1.0f / std::sqrt(float(head_width)); }


// The six attention products go to the batched GEMMs' causal variants: the
// scores and their gradient are read only at or below the diagonal (the
// causal softmax passes read the visible chunks alone), and P and dS are zero
// above it, so the pipeline skips those tiles and k-ranges. The skipped
// products are exact zeros, so no value that is read changes.
// The "attn_causal" override "0" computes everything and writes every zero
// (the tests compare the two bit for bit).
bool attn_causal() { return !flint::tuning_off(flint::Tune::kAttnCausal); }

flint_status attn_nt(void* y, const void* x, const void* w, size_t batches, size_t m, size_t n,
                     size_t k, float scale, flint_stream st) {
    FLINT_HIP_CHECK(flint::launch_gemm_nt_batched(y, x, w, batches, m, n, k, scale,
                                                  flint::to_hip(st), attn_causal()));
    return FLINT_OK;
}

flint_status attn_nn(void* y, const void* x, const void* w, size_t batches, size_t m, size_t n,
                     size_t k, flint_stream st) {
    FLINT_HIP_CHECK(flint::launch_gemm_nn_batched(y, x, w, batches, m, n, k, flint::to_hip(st),
                                                  attn_causal()));
    return FLINT_OK;
}

flint_status attn_tn(void* y, const void* x, const void* w, size_t batches, size_t m, size_t n,
                     size_t k, flint_stream st) {
    FLINT_HIP_CHECK(flint::launch_gemm_tn_batched(y, x, w, batches, m, n, k, flint::to_hip(st),
                                                  attn_causal()));
    return FLINT_OK;
}

// q, k and v to (merge: from) their heads layouts in one launch: the moves of
// three flint_heads_split / flint_heads_merge calls at first = 0, w, 2w.
flint_status attn_heads3(void* qkv, void* const parts[3], size_t sequences, size_t length,
                         size_t heads, size_t head_width, bool merge, flint_stream st) {
    const size_t w = heads * head_width;
    if (3 * sequences * length * (w / 8) >= (size_t{1} << 32)) {   // past 32-bit indexing
        for (size_t i = 0; i < 3; ++i) {
            FLINT_TRY(merge ? flint_heads_merge(qkv, parts[i], sequences, length, heads,
                                                head_width, 3 * w, i * w, st)
                            : flint_heads_split(parts[i], qkv, sequences, length, heads,
                                                head_width, 3 * w, i * w, st));
        }
        return FLINT_OK;
    }
    FLINT_HIP_CHECK(flint::launch_heads3(qkv, parts, sequences, length, heads, head_width, merge,
                                         flint::to_hip(st)));
    return FLINT_OK;
}

// When the NN and TN products that read P and dS both take the causal path,
// the softmax passes write the masked zeros only up to the end of the
// 256-column block holding the diagonal: nothing reads past it.
int attn_zero_span(size_t length, size_t head_width) {
    using flint::GemmLayout;
    const bool taken =
        attn_causal() &&
        flint::gemm_batched_causal_taken(GemmLayout::kNN, length, head_width, length) &&
        flint::gemm_batched_causal_taken(GemmLayout::kTN, length, head_width, length);
    return taken ? flint::kCausalZeroSpan : 0;
}

// Scores and softmax (forward), dP and the softmax backward: one fused launch
// each where attention_stored.hip takes the shape and the batched product
// would run on the pipeline (whose MFMA chain and rounding the fused kernels
// reproduce); the "attn_scores" override "0" runs the two launches instead.
// The same bits either way.
bool attn_scores_fused(size_t length, size_t head_width) {
    return !flint::tuning_off(flint::Tune::kAttnScores) &&
           flint::attn_scores_fusable(length, head_width) &&
           flint::gemm_pipe_eligible(flint::GemmLayout::kNT, flint::Epilogue::kScale, length,
                                     length, head_width);
}

// The stored path without head copies: q, k and v are read as heads views of
// the qkv projection (written into the layer's q, k, v buffers, which then lie
// back to back as one [rows][3 width] block), O, dQ, dK and dV are written as
// heads views of their token rows, and dO is read as one. The split / merge
// launches of the sequence (flint_heads_split / _merge) go away; the products
// and their bits do not change. Taken where the fused scores take the shape,
// the pipeline takes both batched products, and every layer's q, k, v lie
// back to back (one allocation whose 256-byte grid the head buffers' size is
// on).
AttnPlan attn_plan_of(const flint_gpt2& m) {
    using flint::GemmLayout;
    if (m.flash) return AttnPlan::kCopies;
    const size_t len = m.cfg.length, hw = m.head_width;
    const size_t heads_bytes = m.head_batches * len * hw * 2;
    for (const Layer& L : m.layers) {
        const char* q = static_cast<const char*>(L.s.q);
        if (q == nullptr || L.s.k != q + heads_bytes || L.s.v != q + 2 * heads_bytes)
            return AttnPlan::kCopies;
    }
    const bool views = attn_scores_fused(len, hw) &&
                       flint::gemm_batched_causal_taken(GemmLayout::kNN, len, hw, len) &&
                       flint::gemm_batched_causal_taken(GemmLayout::kTN, len, hw, len);
    return views ? AttnPlan::kViews : AttnPlan::kCopies;
}

// Slices of [tokens][cols] rows as heads: slice b = sequence b / heads, head
// b % heads, at column (b % heads) * head_width.
flint::HeadView heads_view(const flint_gpt2& m, size_t cols) {
    flint::HeadView v;
    v.heads = int(m.cfg.heads);
    v.ld = int(cols);
    v.seq = (long long)(m.cfg.length * cols);
    v.head = (long long)(m.head_width);
    return v;
}

flint_status attn_softmax_forward(void* p, const void* s, size_t batches, size_t length,
                                  size_t head_width, flint_stream st) {
    FLINT_HIP_CHECK(flint::launch_causal_softmax_forward(p, s, batches * length, length,
                                                         flint::to_hip(st),
                                                         attn_zero_span(length, head_width)));
    return FLINT_OK;
}

flint_status attn_softmax_backward(void* ds, const void* p, const void* dp, size_t batches,
                                   size_t length, size_t head_width, flint_stream st) {
    FLINT_HIP_CHECK(flint::launch_causal_softmax_backward(
        ds, p, dp, batches * length, length, score_scale(head_width), flint::to_hip(st),
        attn_zero_span(length, head_width)));
    return FLINT_OK;
}

// The fused attention's rows inside the model: head h of sequence n is batch
// n * heads + h; q, k and v rows are the projection's ([rows][3 width]), o and
// dO rows the width-wide ones, dq, dk and dv the projection gradient's.
flint::AttnLayout attn_layout(const flint_gpt2& m) {
    flint::AttnLayout l;
    l.heads = int(m.cfg.heads);
    l.qkv_stride = int(3 * m.cfg.width);
    l.o_stride = int(m.cfg.width);
    l.grad_stride = int(3 * m.cfg.width);
    return l;
}

flint_status layer_norm(const flint_gpt2& m, const Norm& n, const void* x, void* y, void* mean,
                        void* rstd, flint_stream st) {
    return flint_layernorm_forward(y, mean, rstd, x, n.w->data, n.b->data, m.rows, m.cfg.width,
                                   kLnEps, st);
}

// x_out = x_mid + MLP(LN2(x_mid)), x_mid = x_in + Attn(LN1(x_in))
// (ref src/api/gpt2.cpp:495-530).
flint_status forward_layer(const flint_gpt2& m, const Layer& L, flint_stream st) {
    const flint_gpt2_config& c = m.cfg;
    const Saved& s = L.s;
    const size_t rows = m.rows, w = c.width, hw = m.head_width;
    FLINT_TRY(layer_norm(m, L.ln_1, s.x_in, s.h1, s.mean1, s.rstd1, st));
    if (m.flash) {
        // The kernel reads each head's q, k and v rows inside the projection
        // and writes its output rows straight into attn_out's columns.
        auto* qkv = static_cast<_Float16*>(c.backward ? s.qkv : m.qkv);
        FLINT_TRY(flint_gemm_nt_bias(qkv, s.h1, L.attn.half, L.attn.b->data, rows, 3 * w, w, st));
        FLINT_HIP_CHECK(flint::launch_attention_forward(
            s.attn_out, s.lse, qkv, qkv + w, qkv + 2 * w, m.head_batches, c.length,
            score_scale(hw), flint::to_hip(st), attn_layout(m)));
    } else if (m.attn_plan == AttnPlan::kViews) {
        auto* qkv = static_cast<_Float16*>(s.q);   // q, k, v back to back: [rows][3 width]
        FLINT_TRY(flint_gemm_nt_bias(qkv, s.h1, L.attn.half, L.attn.b->data, rows, 3 * w, w, st));
        const flint::HeadView qkv_v = heads_view(m, 3 * w), rows_v = heads_view(m, w);
        FLINT_HIP_CHECK(flint::launch_attn_scores_softmax(
            s.p, qkv, qkv + w, m.head_batches, c.length, hw, score_scale(hw), flint::to_hip(st),
            attn_zero_span(c.length, hw), &qkv_v, &qkv_v));
        FLINT_HIP_CHECK(flint::launch_gemm_nn_batched_views(
            s.attn_out, s.p, qkv + 2 * w, m.head_batches, c.length, hw, c.length, qkv_v, rows_v,
            flint::to_hip(st), attn_causal()));
    } else {
        FLINT_TRY(flint_gemm_nt_bias(m.qkv, s.h1, L.attn.half, L.attn.b->data, rows, 3 * w, w,
                                     st));
        void* const qkv_parts[] = {s.q, s.k, s.v};
        FLINT_TRY(attn_heads3(m.qkv, qkv_parts, c.sequences, c.length, c.heads, hw, false, st));
        if (attn_scores_fused(c.length, hw)) {
            FLINT_HIP_CHECK(flint::launch_attn_scores_softmax(
                s.p, s.q, s.k, m.head_batches, c.length, hw, score_scale(hw), flint::to_hip(st),
                attn_zero_span(c.length, hw)));
        } else {
            FLINT_TRY(attn_nt(m.scores, s.q, s.k, m.head_batches, c.length, c.length, hw,
                              score_scale(hw), st));
            FLINT_TRY(attn_softmax_forward(s.p, m.scores, m.head_batches, c.length, hw, st));
        }
        FLINT_TRY(attn_nn(m.heads_out, s.p, s.v, m.head_batches, c.length, hw, c.length, st));
        FLINT_TRY(flint_heads_merge(s.attn_out, m.heads_out, c.sequences, c.length, c.heads, hw,
                                    w, 0, st));
    }
    FLINT_TRY(flint_gemm_nt_bias_residual(s.x_mid, s.attn_out, L.attn_proj.half,
                                          L.attn_proj.b->data, s.x_in, rows, w, w, st));
    FLINT_TRY(layer_norm(m, L.ln_2, s.x_mid, s.h2, s.mean2, s.rstd2, st));
    FLINT_TRY(flint_gemm_nt_bias_gelu(s.gelu, s.pre, s.h2, L.fc.half, L.fc.b->data, rows, 4 * w,
                                      w, st));
    return flint_gemm_nt_bias_residual(s.x_out, s.gelu, L.fc_proj.half, L.fc_proj.b->data,
                                       s.x_mid, rows, w, 4 * w, st);
}

// Runs a deferred LayerNorm merge on its own (before its workspace is used
// again, or at the end of the backward).
flint_status flush_merge(const flint_gpt2& m, flint_stream st) {
    if (m.pending.cols > 0) {
        FLINT_HIP_CHECK(flint::launch_params_merge(m.pending, flint::to_hip(st)));
        m.pending = flint::ParamsMerge{};
    }
    return FLINT_OK;
}

flint_status weight_grad(const flint_gpt2& m, const Param& p, const void* x, const void* w,
                         int acc, flint_stream st) {
    return flint_gemm_tn(p.grad, x, w, p.rows, p.cols, m.rows, acc, m.tn_work, m.tn_work_bytes,
                         st);
}

flint_status bias_grad(const flint_gpt2& m, const Param& p, const void* dy, int acc,
                       flint_stream st) {
    return flint_bias_gradient(p.grad, dy, m.rows, p.cols, acc, m.work, m.work_bytes, st);
}

// A linear layer's weight and bias gradients from its output gradient dy
// (FP16, rows x w.rows) and input x: the TN product into its k-split
// partials, the bias's chunk partials, then one launch that sums the first
// and merges the second, in place of flint_gemm_tn's and
// flint_bias_gradient's two launches each (the same kernels' arithmetic, the
// same bits). The "fused_grads" override "0" calls the two entry points
// instead (the tests compare the two).
flint_status linear_grads(const flint_gpt2& m, const Param& w, const Param& b, const void* dy,
                          const void* x, int acc, flint_stream st) {
    const hipStream_t hs = flint::to_hip(st);
    if (flint::tuning_off(flint::Tune::kFusedGrads)) {
        FLINT_TRY(flush_merge(m, st));
        FLINT_TRY(weight_grad(m, w, dy, x, acc, st));
        return bias_grad(m, b, dy, acc, st);
    }
    // A deferred LayerNorm merge whose partials these bias partials would
    // overwrite runs first.
    size_t bias_bytes = 0;
    FLINT_TRY(flint_bias_gradient_workspace(m.rows, b.cols, &bias_bytes));
    if (bias_bytes > m.ln_offset) FLINT_TRY(flush_merge(m, st));
    int splits = 1;
    FLINT_HIP_CHECK(flint::launch_gemm_tn_split(w.grad, dy, x, w.rows, w.cols, m.rows, acc != 0,
                                                m.tn_work, &splits, hs));
    FLINT_HIP_CHECK(flint::launch_bias_partials(m.work, dy, m.rows, b.cols, hs));
    // The finish also carries a LayerNorm backward's deferred merge.
    FLINT_HIP_CHECK(flint::launch_linear_grads_finish(w.grad, m.tn_work, w.rows, w.cols, splits,
                                                      acc != 0, b.grad, m.work, m.rows, b.cols,
                                                      acc != 0, hs, &m.pending));
    m.pending = flint::ParamsMerge{};
    return FLINT_OK;
}

// LayerNorm backward: dx, with its FP16 copy written by the dx kernel, then
// dbeta and dgamma from one pass over dy and x. The "fused_sums" override
// "0" calls flint_layernorm_backward instead and converts dx to FP16 after it
// (the tests compare the two).
bool fused_sums() { return !flint::tuning_off(flint::Tune::kFusedSums); }

// On return dres holds the residual stream's gradient and dres_half its FP16
// copy (written by the dx kernel, or converted after the ABI path).
flint_status norm_backward(const flint_gpt2& m, const Norm& n, const void* x, const void* mean,
                           const void* rstd, int acc_dx, int acc, flint_stream st) {
    if (!fused_sums()) {
        FLINT_TRY(flint_layernorm_backward(m.dres, n.w->grad, n.b->grad, m.dh, x, mean, rstd,
                                           n.w->data, m.rows, m.cfg.width, acc_dx, acc, m.work,
                                           m.work_bytes, st));
        return flint_fp32_to_fp16(m.dres_half, m.dres, m.rows * m.cfg.width, st);
    }
    // Its dbeta / dgamma merge is left to the next linear layer's finish
    // where its partials fit beside that layer's bias partials ("ln_defer" =
    // "0": merged here).
    FLINT_TRY(flush_merge(m, st));
    const bool defer = m.ln_offset > 0 && !flint::tuning_off(flint::Tune::kLnDefer);
    void* const ws = static_cast<char*>(m.work) + (defer ? m.ln_offset : 0);
    FLINT_HIP_CHECK(flint::launch_layernorm_backward(m.dres, n.w->grad, n.b->grad, m.dh, x, mean,
                                                     rstd, n.w->data, m.rows, m.cfg.width,
                                                     acc_dx != 0, acc != 0, ws,
                                                     flint::to_hip(st), m.dres_half,
                                                     defer ? &m.pending : nullptr));
    return FLINT_OK;
}

// One layer backward, MLP then attention; dres holds the gradient of the
// residual stream leaving the layer on entry and entering it on return
// (ref src/api/gpt2.cpp:559-618).
flint_status backward_layer(const flint_gpt2& m, const Layer& L, int acc, flint_stream st) {
    const flint_gpt2_config& c = m.cfg;
    const Saved& s = L.s;
    const size_t rows = m.rows, w = c.width, hw = m.head_width;
    const size_t nb = m.head_batches, len = c.length;

    // dres_half = RN16(dres): written by the LayerNorm backward that produced
    // dres (norm_backward), in place of the reference's conversion here.
    FLINT_TRY(linear_grads(m, *L.fc_proj.w, *L.fc_proj.b, m.dres_half, s.gelu, acc, st));
    FLINT_TRY(flint_gemm_nn_dgelu(m.dpre, m.dres_half, L.fc_proj.half, s.pre, rows, 4 * w, w, st));
    FLINT_TRY(linear_grads(m, *L.fc.w, *L.fc.b, m.dpre, s.h2, acc, st));
    FLINT_TRY(flint_gemm_nn(m.dh, m.dpre, L.fc.half, rows, w, 4 * w, st));
    FLINT_TRY(norm_backward(m, L.ln_2, s.x_mid, s.mean2, s.rstd2, 1, acc, st));

    FLINT_TRY(linear_grads(m, *L.attn_proj.w, *L.attn_proj.b, m.dres_half, s.attn_out, acc, st));
    FLINT_TRY(flint_gemm_nn(m.dh, m.dres_half, L.attn_proj.half, rows, w, w, st));
    if (m.flash) {
        // dO rows in dh, O in attn_out, q, k, v in the saved projection; dq,
        // dk and dv go straight into the qkv gradient's columns.
        auto* g = static_cast<_Float16*>(m.qkv);
        const auto* qkv = static_cast<const _Float16*>(s.qkv);
        FLINT_HIP_CHECK(flint::launch_attention_backward(
            g, g + w, g + 2 * w, m.dh, qkv, qkv + w, qkv + 2 * w, s.attn_out, s.lse,
            m.attn_work, nb, len, score_scale(hw), flint::to_hip(st), attn_layout(m)));
    } else if (m.attn_plan == AttnPlan::kViews) {
        // dO rows in dh, q, k, v in the layer's projection block (where the
        // forward left them); dQ, dK, dV straight into the qkv gradient's
        // columns.
        auto* g = static_cast<_Float16*>(m.qkv);
        auto* qkv = static_cast<_Float16*>(s.q);
        const flint::HeadView qkv_v = heads_view(m, 3 * w), rows_v = heads_view(m, w);
        const hipStream_t hs = flint::to_hip(st);
        FLINT_HIP_CHECK(flint::launch_gemm_tn_batched_views(g + 2 * w, s.p, m.dh, nb, len, hw, len,
                                                            rows_v, qkv_v, hs, attn_causal()));
        FLINT_HIP_CHECK(flint::launch_attn_scores_softmax_backward(
            m.scores, s.p, m.dh, qkv + 2 * w, nb, len, hw, score_scale(hw), hs,
            attn_zero_span(len, hw), &rows_v, &qkv_v));
        FLINT_HIP_CHECK(flint::launch_gemm_nn_batched_views(g, m.scores, qkv + w, nb, len, hw, len,
                                                            qkv_v, qkv_v, hs, attn_causal()));
        FLINT_HIP_CHECK(flint::launch_gemm_tn_batched_views(g + w, m.scores, qkv, nb, len, hw, len,
                                                            qkv_v, qkv_v, hs, attn_causal()));
    } else {
        FLINT_TRY(flint_heads_split(m.heads_out, m.dh, c.sequences, len, c.heads, hw, w, 0, st));
        FLINT_TRY(attn_tn(m.dv, s.p, m.heads_out, nb, len, hw, len, st));
        if (attn_scores_fused(len, hw)) {
            FLINT_HIP_CHECK(flint::launch_attn_scores_softmax_backward(
                m.scores, s.p, m.heads_out, s.v, nb, len, hw, score_scale(hw), flint::to_hip(st),
                attn_zero_span(len, hw)));
        } else {
            FLINT_TRY(attn_nt(m.scores, m.heads_out, s.v, nb, len, len, hw, 1.0f, st));
            FLINT_TRY(attn_softmax_backward(m.scores, s.p, m.scores, nb, len, hw, st));
        }
        FLINT_TRY(attn_nn(m.dq, m.scores, s.k, nb, len, hw, len, st));
        FLINT_TRY(attn_tn(m.dk, m.scores, s.q, nb, len, hw, len, st));
        void* const parts[] = {m.dq, m.dk, m.dv};
        FLINT_TRY(attn_heads3(m.qkv, parts, c.sequences, len, c.heads, hw, true, st));
    }
    FLINT_TRY(linear_grads(m, *L.attn.w, *L.attn.b, m.qkv, s.h1, acc, st));
    FLINT_TRY(flint_gemm_nn(m.dh, m.qkv, L.attn.half, rows, w, 3 * w, st));
    return norm_backward(m, L.ln_1, s.x_in, s.mean1, s.rstd1, 1, acc, st);
}

flint_status param_info(const char* name, const flint_gpt2* m, size_t index,
                        flint_gpt2_parameter_info* info, bool grad) {
    if (m == nullptr || info == nullptr) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: model and info must not be null", name);
    }
    if (grad && m->cfg.backward == 0) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT,
                    "%s: the model was created without backward, so it has no gradients", name);
    }
    if (index >= m->params.size()) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: index (%zu) must be below %zu", name, index,
                    m->params.size());
    }
    const Param& p = m->params[index];
    info->name = p.name.c_str();
    info->data = grad ? p.grad : p.data;
    info->rows = p.rows;
    info->cols = p.cols;
    return FLINT_OK;
}

// The fused attention's kernels take head width 64 only.
flint_status check_fused(const char* name, const flint_gpt2_config& c) {
    return flint::Checker(name)
        .require(c.width / c.heads == 64, "the fused attention needs head width 64, not %zu",
                 c.width / c.heads)
        .status();
}

flint_status model_bytes(const char* name, const flint_gpt2_config* config, bool fused,
                         size_t* bytes) {
    FLINT_TRY(check_config(name, config));
    if (fused) FLINT_TRY(check_fused(name, *config));
    if (bytes == nullptr) return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: bytes is null", name);
    try {
        flint_gpt2 m;
        m.cfg = *config;
        m.flash = fused;
        FLINT_TRY(plan(m));
        *bytes = total_bytes(m);
    } catch (const std::bad_alloc&) {
        return fail(FLINT_ERROR_CUDA, "%s: out of host memory", name);
    }
    return FLINT_OK;
}

flint_status create_model(const char* name, const flint_gpt2_config* config, bool fused,
                          flint_gpt2** model) {
    if (model == nullptr) return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: model is null", name);
    *model = nullptr;
    FLINT_TRY(check_config(name, config));
    if (fused) FLINT_TRY(check_fused(name, *config));
    try {
        auto m = std::make_unique<flint_gpt2>();
        m->cfg = *config;
        m->flash = fused;
        FLINT_TRY(plan(*m));
        m->host_loss.resize(m->rows);
        FLINT_TRY(allocate(*m));
        link(*m);
        m->attn_plan = attn_plan_of(*m);
        *model = m.release();
    } catch (const std::bad_alloc&) {
        return fail(FLINT_ERROR_CUDA, "%s: out of host memory", name);
    }
    return FLINT_OK;
}

}  // namespace

extern "C" {

FLINT_API flint_status flint_gpt2_bytes(const flint_gpt2_config* config, size_t* bytes) {
    return model_bytes("flint_gpt2_bytes", config, false, bytes);
}

FLINT_API flint_status flint_gpt2_bytes_fused(const flint_gpt2_config* config, size_t* bytes) {
    return model_bytes("flint_gpt2_bytes_fused", config, true, bytes);
}

FLINT_API flint_status flint_gpt2_create(const flint_gpt2_config* config, flint_gpt2** model) {
    return create_model("flint_gpt2_create", config, false, model);
}

FLINT_API flint_status flint_gpt2_create_fused(const flint_gpt2_config* config,
                                               flint_gpt2** model) {
    return create_model("flint_gpt2_create_fused", config, true, model);
}

FLINT_API void flint_gpt2_destroy(flint_gpt2* model) { delete model; }

FLINT_API size_t flint_gpt2_parameter_count(const flint_gpt2* model) {
    return model == nullptr ? 0 : model->params.size();
}

FLINT_API flint_status flint_gpt2_parameter(const flint_gpt2* model, size_t index,
                                            flint_gpt2_parameter_info* info) {
    return param_info("flint_gpt2_parameter", model, index, info, false);
}

FLINT_API flint_status flint_gpt2_gradient(const flint_gpt2* model, size_t index,
                                           flint_gpt2_parameter_info* info) {
    return param_info("flint_gpt2_gradient", model, index, info, true);
}

FLINT_API flint_status flint_gpt2_sync_weights(flint_gpt2* model, flint_stream stream) {
    if (model == nullptr) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "flint_gpt2_sync_weights: model is null");
    }
    FLINT_TRY(flint_fp32_to_fp16(model->wte_half, model->wte->data,
                                 model->wte->rows * model->wte->cols, stream));
    for (const Layer& L : model->layers) {
        for (const Linear* lin : {&L.attn, &L.attn_proj, &L.fc, &L.fc_proj}) {
            FLINT_TRY(flint_fp32_to_fp16(lin->half, lin->w->data, lin->w->rows * lin->w->cols,
                                         stream));
        }
    }
    return FLINT_OK;
}

FLINT_API flint_status flint_gpt2_forward(flint_gpt2* model, const void* tokens,
                                          const void* targets, float scale, flint_stream stream) {
    constexpr const char* name = "flint_gpt2_forward";
    if (model == nullptr) return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: model is null", name);
    if (!std::isfinite(scale)) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: scale (%g) must be finite", name,
                    static_cast<double>(scale));
    }
    const flint_gpt2& m = *model;
    const flint_gpt2_config& c = m.cfg;
    const size_t rows = m.rows;
    FLINT_TRY(flint::Checker(name)
                  .buffers({{"logits", m.logits, rows * c.padded_vocab * 2},
                            {"dlogits", m.dlogits, rows * c.padded_vocab * 2},
                            {"row_loss", m.row_loss, rows * 4},
                            {"tokens", tokens, rows * 2},
                            {"targets", targets, rows * 2}},
                           3)
                  .status());
    FLINT_TRY(flint_embedding_forward(m.layers[0].s.x_in, tokens, m.wte->data, m.wpe->data,
                                      c.sequences, c.length, c.padded_vocab, c.width, stream));
    model->attn_plan = attn_plan_of(m);
    for (const Layer& L : m.layers) FLINT_TRY(forward_layer(m, L, stream));
    FLINT_TRY(layer_norm(m, m.ln_f, m.x_final, m.h_f, m.mean_f, m.rstd_f, stream));
    FLINT_TRY(flint_gemm_nt(m.logits, m.h_f, m.wte_half, rows, c.padded_vocab, c.width, stream));
    return flint_softmax_cross_entropy(m.dlogits, m.row_loss, m.logits, targets, scale, rows,
                                       c.vocab, c.padded_vocab, stream);
}

FLINT_API flint_status flint_gpt2_backward(flint_gpt2* model, const void* tokens, int accumulate,
                                           flint_stream stream) {
    constexpr const char* name = "flint_gpt2_backward";
    if (model == nullptr) return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: model is null", name);
    const flint_gpt2& m = *model;
    const flint_gpt2_config& c = m.cfg;
    if (c.backward == 0) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: the model was created without backward",
                    name);
    }
    const size_t rows = m.rows, w = c.width;
    flint::Checker check(name);
    check.buffers({{"logits", m.logits, rows * c.padded_vocab * 2},
                   {"dlogits", m.dlogits, rows * c.padded_vocab * 2},
                   {"row_loss", m.row_loss, rows * 4},
                   {"tokens", tokens, rows * 2}},
                  3);
    const flint::Span tok{"tokens", tokens, rows * 2};
    for (const Param& p : m.params)
        check.require(!tok.meets({"grad", p.grad, p.rows * p.cols * 4}),
                      "tokens and the gradient of %s overlap", p.name.c_str());
    FLINT_TRY(check.status());
    m.pending = flint::ParamsMerge{};   // nothing carries over from an earlier call
    // Output layer (tied to wte): dwte (+)= dlogits^T h_f; dh = dlogits wte.
    FLINT_TRY(weight_grad(m, *m.wte, m.dlogits, m.h_f, accumulate, stream));
    FLINT_TRY(flint_gemm_nn(m.dh, m.dlogits, m.wte_half, rows, w, c.padded_vocab, stream));
    FLINT_TRY(norm_backward(m, m.ln_f, m.x_final, m.mean_f, m.rstd_f, 0, accumulate, stream));
    for (auto L = m.layers.rbegin(); L != m.layers.rend(); ++L)
        FLINT_TRY(backward_layer(m, *L, accumulate, stream));
    FLINT_TRY(flush_merge(m, stream));
    // The embedding always adds into wte's gradient: (old + output layer) + embedding.
    FLINT_TRY(flint_embedding_backward(m.wte->grad, m.wpe->grad, m.dres, tokens, c.sequences,
                                       c.length, c.padded_vocab, w, 1, accumulate, m.work,
                                       m.work_bytes, stream));
    // Positions length..block_size never occur: their gradient is +0 (a fill
    // kernel, so a captured graph holds no memset node).
    if (accumulate == 0 && c.block_size > c.length) {
        char* unseen = static_cast<char*>(m.wpe->grad) + c.length * w * 4;
        FLINT_HIP_CHECK(flint::launch_fill_zero(unseen, (c.block_size - c.length) * w * 4,
                                                flint::to_hip(stream)));
    }
    return FLINT_OK;
}

FLINT_API flint_status flint_gpt2_outputs(const flint_gpt2* model, const void** logits,
                                          const void** dlogits, const void** row_loss) {
    if (model == nullptr) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "flint_gpt2_outputs: model is null");
    }
    if (logits) *logits = model->logits;
    if (dlogits) *dlogits = model->dlogits;
    if (row_loss) *row_loss = model->row_loss;
    return FLINT_OK;
}

FLINT_API flint_status flint_gpt2_mean_loss(flint_gpt2* model, flint_stream stream, double* loss) {
    constexpr const char* name = "flint_gpt2_mean_loss";
    if (model == nullptr || loss == nullptr) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: model and loss must not be null", name);
    }
    std::vector<float>& host = model->host_loss;
    FLINT_HIP_CHECK(hipMemcpyAsync(host.data(), model->row_loss, host.size() * sizeof(float),
                                   hipMemcpyDeviceToHost, flint::to_hip(stream)));
    FLINT_HIP_CHECK(hipStreamSynchronize(flint::to_hip(stream)));
    double sum = 0.0;
    for (float v : host) sum += double(v);
    *loss = sum / double(host.size());
    return FLINT_OK;
}

}  // extern "C"
