// Launchers for the gfx950 kernels. The C-ABI layer (csrc/api) validates the
// arguments, then calls exactly one of these; each queues its kernels on the
// stream and returns the launch error, if any.
#pragma once

#include <cstddef>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "flint/flint_train.h"

namespace flint {

// Size limits of the ABI (ref src/kernels/gemm.cuh:13-18, src/api/gemm.cpp:21).
constexpr size_t kGemmMaxMN = size_t{65535} * 128;
constexpr size_t kGemmMaxK = size_t{1} << 16;
constexpr size_t kGemmBatchedMaxM = 1024;
constexpr size_t kGemmMaxBatches = 65535;

// GEMM epilogues (what happens to the FP32 sums before the single rounding).
enum class Epilogue { kNone, kBias, kBiasGelu, kBiasResidual, kDGelu, kScale };

hipError_t launch_gemm_nt(void* y, const void* x, const void* w, const void* bias,
                          void* aux, Epilogue e, size_t m, size_t n, size_t k,
                          hipStream_t stream);
// The one-wave-per-SIMD GEMM pipeline (gemm_pipe.hip), for k % 32 == 0 and
// n % 8 == 0 (and m % 8 == 0 for TN). The launchers below route there when
// gemm_pipe_eligible says so (FLINT_GEMM_PIPE=0 turns it off).
enum class GemmLayout { kNT, kNN, kTN };
// kTnFloat: TN's FP32 output (y = sum, y += sum, or a split's partial);
// kNone with TN is the batched FP16 output.
constexpr Epilogue kTnFloat = Epilogue(100);
bool gemm_pipe_eligible(GemmLayout l, Epilogue e, size_t m, size_t n, size_t k);
// TN's FP32 output through the pipeline, choosing its own tile and split count
// up to max_splits (the ABI plan the workspace was sized for); the count used
// comes back in *splits (1: no partials, y written directly).
hipError_t launch_gemm_pipe_tn(void* y, const void* x, const void* w, size_t m, size_t n,
                               size_t k, bool accumulate, void* workspace, int max_splits,
                               int* splits, hipStream_t stream);
// causal: the per-slice m x m operand is zero above its diagonal (NT: only the
// output's tiles at or below it are computed; NN / TN: each tile's k-range is
// cut to where that operand can be nonzero). Requires m == n (NT) or m == k.
struct HeadView;
hipError_t launch_gemm_pipe(GemmLayout l, Epilogue e, void* y, const void* x, const void* w,
                            const void* bias, void* aux, float scale, size_t slices, size_t m,
                            size_t n, size_t k, bool accumulate, void* partials, int split_len,
                            hipStream_t stream, bool causal = false,
                            const HeadView* wv = nullptr, const HeadView* yv = nullptr);
hipError_t launch_gemm_nn(void* y, const void* x, const void* w, const void* aux, Epilogue e,
                          size_t m, size_t n, size_t k, hipStream_t stream);
// Number of k splits TN uses for m x n x k on this device (1 = none).
hipError_t gemm_tn_splits(size_t m, size_t n, size_t k, int* splits, int* split_len);
hipError_t gemm_tn_workspace(size_t m, size_t n, size_t k, size_t* bytes);
hipError_t launch_gemm_tn(void* y, const void* x, const void* w, size_t m, size_t n, size_t k,
                          bool accumulate, void* workspace, hipStream_t stream);
// launch_gemm_tn's two halves: the product, then (when *splits_used > 1, the
// partials being in workspace and y untouched) the sum of the partials.
hipError_t launch_gemm_tn_split(void* y, const void* x, const void* w, size_t m, size_t n,
                                size_t k, bool accumulate, void* workspace, int* splits_used,
                                hipStream_t stream);
hipError_t launch_tn_reduce(void* y, const void* partials, size_t m, size_t n, int splits,
                            bool accumulate, hipStream_t stream);
// A batched operand laid out as the heads of token rows (the GPT-2 model's
// attention): slice b is head b % heads of sequence b / heads, starting
// (b / heads) * seq + (b % heads) * head elements in, its rows ld elements
// apart. heads == 0: the plain [slices][rows][cols] layout.
struct HeadView {
    int heads = 0;
    int ld = 0;
    long long seq = 0, head = 0;
};

__host__ __device__ inline size_t head_view_offset(const HeadView& v, int slice) {
    return size_t(slice / v.heads) * size_t(v.seq) + size_t(slice % v.heads) * size_t(v.head);
}

// The batched GEMMs. causal (attention inside the GPT-2 model only): x (NN,
// TN) is zero above its diagonal per slice, or (NT) only y's entries at or
// below the diagonal are wanted; the pipeline then skips the rest, which
// changes no wanted value (the skipped products are exact zeros). Shapes the
// pipeline does not take compute everything.
hipError_t launch_gemm_nt_batched(void* y, const void* x, const void* w, size_t batches,
                                  size_t m, size_t n, size_t k, float scale, hipStream_t stream,
                                  bool causal = false);
hipError_t launch_gemm_nn_batched(void* y, const void* x, const void* w, size_t batches,
                                  size_t m, size_t n, size_t k, hipStream_t stream,
                                  bool causal = false);
hipError_t launch_gemm_tn_batched(void* y, const void* x, const void* w, size_t batches,
                                  size_t m, size_t n, size_t k, hipStream_t stream,
                                  bool causal = false);
// The same on the pipeline with w (k-major) and y as heads views, for the
// model's attention: only where gemm_batched_causal_taken says the pipeline
// takes the shape (otherwise hipErrorInvalidValue).
hipError_t launch_gemm_nn_batched_views(void* y, const void* x, const void* w, size_t batches,
                                        size_t m, size_t n, size_t k, const HeadView& wv,
                                        const HeadView& yv, hipStream_t stream, bool causal);
hipError_t launch_gemm_tn_batched_views(void* y, const void* x, const void* w, size_t batches,
                                        size_t m, size_t n, size_t k, const HeadView& wv,
                                        const HeadView& yv, hipStream_t stream, bool causal);
// Whether a causal batched GEMM of this layout and shape takes the causal path
// (the pipeline, with the square operand); otherwise it computes everything.
bool gemm_batched_causal_taken(GemmLayout l, size_t m, size_t n, size_t k);
// Fused causal attention (attention.hip), head width 64. D (batches x length
// FP32) is the backward's workspace.
constexpr size_t kAttentionMaxLength = size_t{1} << 20;
constexpr size_t kAttentionMaxBatches = 65535;
// Where the rows of batch b live: head b % heads of sequence b / heads, its
// row t at element (sequence * length + t) * stride + head * 64 of a tensor
// (q, k, v: qkv_stride; o, dout: o_stride; dq, dk, dv: grad_stride). The
// C ABI's [batches][length][64] tensors are heads 1, strides 64; the model
// reads q, k and v straight from its [tokens][3 width] projection and writes
// o into its [tokens][width] rows. length * stride stays below 2^30.
struct AttnLayout {
    int heads = 1;
    int qkv_stride = 64;
    int o_stride = 64;
    int grad_stride = 64;
};
hipError_t launch_attention_forward(void* out, void* lse, const void* q, const void* k,
                                    const void* v, size_t batches, size_t length, float scale,
                                    hipStream_t stream, AttnLayout layout = {});
hipError_t launch_attention_backward(void* dq, void* dk, void* dv, const void* dout, const void* q,
                                     const void* k, const void* v, const void* o, const void* lse,
                                     void* dsum, size_t batches, size_t length, float scale,
                                     hipStream_t stream, AttnLayout layout = {});
// Rows of a causal tile and the k-step both divide this: a causal softmax
// writing its zeros up to the end of each such block covers what the causal
// GEMMs read.
constexpr int kCausalZeroSpan = 256;

// Row reductions.
constexpr size_t kLayerNormMaxCols = size_t{1} << 24;
constexpr size_t kLayerNormMaxRows = size_t{0x7fffffff} * 8;
constexpr size_t kBiasGradientChunkRows = 256;
constexpr size_t kBiasGradientMaxCols = size_t{65535} * 256;
constexpr size_t kBiasGradientMaxRows = size_t{0x7fffffff} * kBiasGradientChunkRows;
constexpr size_t kSoftmaxMaxLength = 1024;
constexpr size_t kSoftmaxMaxBatches = 65535;
constexpr size_t kCrossEntropyMaxCols = size_t{1} << 16;
constexpr size_t kCrossEntropyMaxRows = size_t{0x7fffffff} * 8;

// Workspace of the bias gradient: an FP32 sum and its error per column per
// started chunk of 256 rows (ref src/kernels/bias_gradient.cuh:25-27).
constexpr size_t bias_gradient_workspace(size_t rows, size_t cols) {
    return (rows + kBiasGradientChunkRows - 1) / kBiasGradientChunkRows * cols * 8;
}

// Workspace of the LayerNorm backward: the dbeta and dgamma chunk partials,
// one bias-gradient region each.
constexpr size_t layernorm_backward_workspace(size_t rows, size_t cols) {
    return 2 * bias_gradient_workspace(rows, cols);
}

hipError_t launch_layernorm_forward(void* y, void* mean, void* rstd, const void* x,
                                    const void* gamma, const void* beta, size_t rows, size_t cols,
                                    float eps, hipStream_t stream);
// LayerNorm backward in two launches: the dbeta and dgamma chunk partials from
// one pass over dy and x, then dx, whose kernel also merges the partials.
// With dx_half, RN16 of every dx value written goes there too (the values
// flint_fp32_to_fp16 of dx would give). workspace:
// layernorm_backward_workspace(rows, cols) bytes.
// LayerNorm backward's last step, the merge of its dbeta and dgamma chunk
// partials, as a description another launch can carry (cols == 0: none).
struct ParamsMerge {
    float* dbeta = nullptr;
    float* dgamma = nullptr;
    const float* part0 = nullptr;   // dbeta's chunk partials
    const float* part1 = nullptr;   // dgamma's
    size_t chunks = 0;
    int cols = 0;
    int accumulate = 0;
};
// With `deferred`, a plan that ends in a separate merge launch leaves that
// launch out and describes it in *deferred instead (cols = 0 when the merge
// was done); the caller then runs it with launch_params_merge or passes it to
// launch_linear_grads_finish, before the workspace is used again.
hipError_t launch_layernorm_backward(void* dx, void* dgamma, void* dbeta, const void* dy,
                                     const void* x, const void* mean, const void* rstd,
                                     const void* gamma, size_t rows, size_t cols,
                                     bool accumulate_dx, bool accumulate_params, void* workspace,
                                     hipStream_t stream, void* dx_half = nullptr,
                                     ParamsMerge* deferred = nullptr);
hipError_t launch_params_merge(const ParamsMerge& merge, hipStream_t stream);
hipError_t launch_bias_gradient(void* dbias, const void* dy, size_t rows, size_t cols,
                                bool accumulate, void* workspace, hipStream_t stream);
// The same two passes with the partials in the library's per-device scratch
// array (kBiasGradientScratchBytes; no allocation). Sizes whose partials do
// not fit return hipErrorInvalidValue.
constexpr size_t kBiasGradientScratchBytes = size_t{4} << 20;
hipError_t launch_bias_gradient_noalloc(void* dbias, const void* dy, size_t rows, size_t cols,
                                        bool accumulate, hipStream_t stream);
// Merges per-chunk (sum, error) partials left in workspace into out (cols FP32).
hipError_t launch_bias_gradient_finish(void* out, const void* workspace, size_t rows,
                                       size_t cols, bool accumulate, hipStream_t stream);
// launch_bias_gradient's first pass alone: the chunk partials into workspace.
hipError_t launch_bias_partials(void* workspace, const void* dy, size_t rows, size_t cols,
                                hipStream_t stream);
// One linear layer's gradients finished in one launch (the GPT-2 model's
// backward): dw's k-split partials summed as launch_tn_reduce sums them (none
// when splits == 1) and db's chunk partials merged as
// launch_bias_gradient_finish merges them; the same bits as the two launches.
hipError_t launch_linear_grads_finish(void* dw, const void* dw_partials, size_t m, size_t n,
                                      int splits, bool accumulate_w, void* db,
                                      const void* db_workspace, size_t rows, size_t cols,
                                      bool accumulate_b, hipStream_t stream,
                                      const ParamsMerge* also = nullptr);
// zero_span 0 writes every chunk of a row (the ABI functions); Z > 0 (a
// multiple of 8) writes the masked zeros only up to the end of the Z-column
// block holding the diagonal, for consumers that read no further (the model's
// causal GEMMs, whose tiles are at most 256 rows and k-steps divide 256).
hipError_t launch_causal_softmax_forward(void* p, const void* s, size_t rows, size_t length,
                                         hipStream_t stream, int zero_span = 0);
hipError_t launch_causal_softmax_backward(void* ds, const void* p, const void* dp, size_t rows,
                                          size_t length, float scale, hipStream_t stream,
                                          int zero_span = 0);
// The model's stored-probability attention with the scores (dP) kept out of
// memory (attention_stored.hip): P = causal_softmax_forward(RN16(scale q kᵀ))
// and dS = causal_softmax_backward(p, RN16(dout vᵀ)), the same bits as the
// batched NT product followed by the softmax pass. Head width 64, lengths a
// multiple of 32 up to 1,024 (attn_scores_fusable); q, k, v, dout are
// [batches][length][64], p and ds [batches][length][length] (ds not aliasing
// p); zero_span as for the softmax passes.
bool attn_scores_fusable(size_t length, size_t head_width);
// qv / kv (dov / vv): the operands as heads views, or null for
// [batches][length][64].
hipError_t launch_attn_scores_softmax(void* p, const void* q, const void* k, size_t batches,
                                      size_t length, size_t head_width, float scale,
                                      hipStream_t stream, int zero_span,
                                      const HeadView* qv = nullptr, const HeadView* kv = nullptr);
hipError_t launch_attn_scores_softmax_backward(void* ds, const void* p, const void* dout,
                                               const void* v, size_t batches, size_t length,
                                               size_t head_width, float scale,
                                               hipStream_t stream, int zero_span,
                                               const HeadView* dov = nullptr,
                                               const HeadView* vv = nullptr);
hipError_t launch_softmax_cross_entropy(void* dlogits, void* row_loss, const void* logits,
                                        const void* targets, float scale, size_t rows,
                                        size_t vocab, size_t cols, hipStream_t stream);

// Data movement.
constexpr size_t kEmbeddingMaxWidth = size_t{1} << 24;
constexpr size_t kEmbeddingMaxVocab = size_t{1} << 16;
constexpr size_t kEmbeddingMaxRows = size_t{0x7fffffff} * 8;
constexpr size_t kEmbeddingBackwardMaxWidth = kBiasGradientMaxCols;
constexpr size_t kEmbeddingBackwardMaxRows = 0xffffffffu;
constexpr size_t kEmbeddingBackwardMaxPositionValues = kBiasGradientMaxCols;
constexpr size_t kHeadsMaxRowWidth = size_t{1} << 24;
constexpr size_t kHeadsMaxRows = size_t{0x7fffffff} * 8;

hipError_t launch_copy(void* dst, const void* src, size_t bytes, hipStream_t stream);
// Zeroes bytes at dst (16-byte aligned) with a kernel, not a memset node.
hipError_t launch_fill_zero(void* dst, size_t bytes, hipStream_t stream);
hipError_t launch_fp32_to_fp16(void* y, const void* x, size_t count, hipStream_t stream);
hipError_t launch_heads(void* y, const void* x, size_t batches, size_t length, size_t heads,
                        size_t head_width, size_t row_width, size_t first, bool merge,
                        hipStream_t stream);
// The three q / k / v parts of a [rows][3 * heads * head_width] matrix split
// into (merge: from) three heads layouts in one launch (the model's attention);
// hipErrorInvalidValue past 2^32 16-byte chunks.
hipError_t launch_heads3(void* wide, void* const parts[3], size_t batches, size_t length,
                         size_t heads, size_t head_width, bool merge, hipStream_t stream);
hipError_t launch_embedding_forward(void* x, const void* tokens, const void* wte,
                                    const void* wpe, size_t rows, size_t length, size_t width,
                                    hipStream_t stream);
size_t embedding_backward_workspace(size_t sequences, size_t length, size_t vocab, size_t width);
hipError_t launch_embedding_backward(void* dwte, void* dwpe, const void* dx, const void* tokens,
                                     size_t sequences, size_t length, size_t vocab, size_t width,
                                     bool accumulate_wte, bool accumulate_wpe, void* workspace,
                                     hipStream_t stream);

// AdamW over many tensors (optimizer.hip). Each tensor is cut into chunks of
// kAdamwChunk elements, one workgroup each; a launch takes up to kAdamwGroup
// tensors by value. block_start[i] is tensor i's first workgroup in the launch
// (block_start[count] the launch's workgroups); partial_offset is the launch's
// first chunk among all of the step's chunks.
constexpr int kAdamwGroup = 64;   // 64 x 56-byte entries + starts: under 4 KB of kernel arguments
constexpr unsigned long long kAdamwChunk = 8192;
constexpr size_t kAdamwMaxTensors = 4096;

struct AdamwTensorArgs {
    float* p;
    const float* g;
    float* m;
    float* v;
    __half* h;
    unsigned long long n;
    float decay;   // 1 - lr * weight_decay
};

struct AdamwGroup {
    AdamwTensorArgs t[kAdamwGroup];
    int block_start[kAdamwGroup + 1];
    int count;
    int partial_offset;
};
static_assert(sizeof(AdamwGroup) <= 4096, "AdamwGroup is passed as a kernel argument");

// Workspace of a step over `chunks` chunks: FP64 partials, then the decision.
size_t adamw_workspace(size_t chunks);
hipError_t launch_adamw_sumsq(const AdamwGroup& group, int blocks, void* workspace, const void* state,
                              hipStream_t stream);
hipError_t launch_adamw_decide(size_t chunks, void* workspace, void* state, const flint_adamw_options& o,
                               hipStream_t stream);
hipError_t launch_adamw_update(const AdamwGroup& group, int blocks, size_t chunks, const void* workspace,
                               const flint_adamw_options& o, hipStream_t stream);
hipError_t launch_train_state_init(void* state, float loss_scale, hipStream_t stream);

}  // namespace flint
