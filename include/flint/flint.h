/* libflint: the GPT-2 training hot path on AMD Instinct MI355X (gfx950).
 *
 * This header is the drop-in boundary. Every declaration below keeps the name,
 * argument order, argument types and meaning of the function it replaces in
 * bayareahomelander/Flint's include/flint/flint.h (cited per function as
 * ref flint.h:LINE), so a caller that binds the reference library through
 * ctypes, or links it from C or C++, binds this one unchanged. The text of the
 * comments is this library's own.
 *
 * Conventions shared by every function:
 *  - Matrices are row-major, contiguous, in device memory. FP16 is IEEE binary16,
 *    FP32 binary32. Sizes are element counts (size_t), flags are int (nonzero =
 *    true).
 *  - Work is queued on `stream` and returns without waiting for the GPU, except
 *    flint_gpt2_mean_loss. A null stream is the null (default) HIP stream.
 *  - Kernel functions never allocate device memory. A function that needs scratch
 *    space takes a caller-owned workspace sized by its *_workspace query.
 *  - Every output value rounds once, to nearest-even, from an FP32 result.
 *  - A failing call returns a nonzero flint_status and records a message that
 *    flint_last_error returns on the calling thread.
 */
#ifndef FLINT_FLINT_H
#define FLINT_FLINT_H

#include <stddef.h>

/* Only functions marked FLINT_API are exported; the library builds with hidden
 * visibility. */
#define FLINT_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes (ref flint.h:26-32). FLINT_ERROR_CUDA keeps its reference name
 * and value; here it reports a failed HIP runtime call. */
typedef int flint_status;
enum {
    FLINT_OK = 0,
    FLINT_ERROR_INVALID_ARGUMENT = 1,
    FLINT_ERROR_CUDA = 2
};

/* "0.1.0" (ref flint.h:35). */
FLINT_API const char* flint_version(void);

/* "ok", "invalid argument", "CUDA error", or "unknown status" (ref flint.h:38). */
FLINT_API const char* flint_status_string(flint_status status);

/* This thread's message for its latest failed call; "" before any failure.
 * A successful call does not clear it (ref flint.h:42). */
FLINT_API const char* flint_last_error(void);

/* The stream type keeps the reference's declaration (ref flint.h:46) so that
 * code compiled against either header agrees on it. On this library the value
 * is a hipStream_t (struct ihipStream_t*): one opaque pointer either way, passed
 * as it is; HIP callers cast their stream to flint_stream. */
typedef struct CUstream_st* flint_stream;

/* Device-to-device byte copy; ranges must not overlap (ref flint.h:51). */
FLINT_API flint_status flint_copy(void* dst, const void* src, size_t bytes, flint_stream stream);

/* y(m x n, FP16) = x(m x k, FP16) * w(n x k, FP16)^T, FP32 accumulation, one
 * rounding per output. k a positive multiple of 8 up to 65,536; m, n up to
 * 8,388,480; pointers 16-byte aligned; y overlaps neither input. m or n of 0 is
 * a no-op that checks nothing (ref flint.h:63). */
FLINT_API flint_status flint_gemm_nt(void* y, const void* x, const void* w, size_t m, size_t n,
                                     size_t k, flint_stream stream);

/* As flint_gemm_nt, adding bias[col] (n FP32) to the FP32 sums before rounding
 * (ref flint.h:71). */
FLINT_API flint_status flint_gemm_nt_bias(void* y, const void* x, const void* w, const void* bias,
                                          size_t m, size_t n, size_t k, flint_stream stream);

/* s = x w^T + bias in FP32; pre = RN16(s); y = RN16(GELU_tanh(s)) (ref flint.h:81). */
FLINT_API flint_status flint_gemm_nt_bias_gelu(void* y, void* pre, const void* x, const void* w,
                                               const void* bias, size_t m, size_t n, size_t k,
                                               flint_stream stream);

/* y(FP32) = residual(FP32) + (x w^T + bias), FP32 adds, no FP16 rounding; n even
 * (ref flint.h:92). */
FLINT_API flint_status flint_gemm_nt_bias_residual(void* y, const void* x, const void* w,
                                                   const void* bias, const void* residual,
                                                   size_t m, size_t n, size_t k,
                                                   flint_stream stream);

/* y(m x n) = x(m x k) * w(k x n), all FP16; n a multiple of 8 (ref flint.h:101). */
FLINT_API flint_status flint_gemm_nn(void* y, const void* x, const void* w, size_t m, size_t n,
                                     size_t k, flint_stream stream);

/* y = RN16((x w) * GELU_tanh'(pre)), pre m x n FP16; GELU' is 0 at -inf, 1 at
 * +inf, NaN at NaN (ref flint.h:112). */
FLINT_API flint_status flint_gemm_nn_dgelu(void* y, const void* x, const void* w,
                                           const void* pre, size_t m, size_t n, size_t k,
                                           flint_stream stream);

/* y(m x n, FP32) = x(k x m)^T w(k x n), or y += that with accumulate. m, n
 * multiples of 8; k from 1 to 65,536. Outputs with few tiles split k; the splits'
 * partial sums go to the workspace flint_gemm_tn_workspace sizes and are added
 * in split order, y = old + (p0 + p1 + ...), so results are deterministic
 * (ref flint.h:132). */
FLINT_API flint_status flint_gemm_tn(void* y, const void* x, const void* w, size_t m, size_t n,
                                     size_t k, int accumulate, void* workspace,
                                     size_t workspace_bytes, flint_stream stream);

/* Workspace bytes flint_gemm_tn needs on the current GPU: 0 or splits*m*n*4; it
 * depends on the GPU's compute-unit count (ref flint.h:138). */
FLINT_API flint_status flint_gemm_tn_workspace(size_t m, size_t n, size_t k, size_t* bytes);

/* dbias[j] (+)= sum_r dy[r, j], dy rows x cols FP16, compensated FP32 (TwoSum)
 * in 256-row chunks, merged in a fixed order (ref flint.h:153). */
FLINT_API flint_status flint_bias_gradient(void* dbias, const void* dy, size_t rows, size_t cols,
                                           int accumulate, void* workspace,
                                           size_t workspace_bytes, flint_stream stream);

/* 8 * cols bytes per started chunk of 256 rows (ref flint.h:159). */
FLINT_API flint_status flint_bias_gradient_workspace(size_t rows, size_t cols, size_t* bytes);

/* y[j] = RN16(scale * x[j] w[j]^T) for j < batches; m <= 1,024, batches <= 65,535
 * (ref flint.h:173). */
FLINT_API flint_status flint_gemm_nt_batched(void* y, const void* x, const void* w, size_t batches,
                                             size_t m, size_t n, size_t k, float scale,
                                             flint_stream stream);

/* y[j] = RN16(x[j] w[j]) (ref flint.h:181). */
FLINT_API flint_status flint_gemm_nn_batched(void* y, const void* x, const void* w, size_t batches,
                                             size_t m, size_t n, size_t k, flint_stream stream);

/* y[j] = RN16(x[j]^T w[j]), FP16 output, k never split (ref flint.h:190). */
FLINT_API flint_status flint_gemm_tn_batched(void* y, const void* x, const void* w, size_t batches,
                                             size_t m, size_t n, size_t k, flint_stream stream);

/* Per row of x (rows x cols FP32): mean and biased variance by compensated
 * sums, rstd = 1/sqrt(var + eps), y = RN16(fma((x - mean) * rstd, gamma, beta));
 * mean and rstd stored per row (ref flint.h:211). */
FLINT_API flint_status flint_layernorm_forward(void* y, void* mean, void* rstd, const void* x,
                                               const void* gamma, const void* beta, size_t rows,
                                               size_t cols, float eps, flint_stream stream);

/* dx (+)= rstd (g - mean(g) - xhat mean(g xhat)), g = dy gamma; dgamma (+)= column
 * sums of dy xhat; dbeta (+)= column sums of dy, exactly flint_bias_gradient's
 * (ref flint.h:236). */
FLINT_API flint_status flint_layernorm_backward(void* dx, void* dgamma, void* dbeta,
                                                const void* dy, const void* x, const void* mean,
                                                const void* rstd, const void* gamma, size_t rows,
                                                size_t cols, int accumulate_dx,
                                                int accumulate_params, void* workspace,
                                                size_t workspace_bytes, flint_stream stream);

/* flint_bias_gradient_workspace's size (ref flint.h:245). */
FLINT_API flint_status flint_layernorm_backward_workspace(size_t rows, size_t cols,
                                                          size_t* bytes);

/* x[s*length + t] = wte[tokens[.]] + wpe[t], FP32; tokens uint16 (ref flint.h:266). */
FLINT_API flint_status flint_embedding_forward(void* x, const void* tokens, const void* wte,
                                               const void* wpe, size_t sequences, size_t length,
                                               size_t vocab, size_t width, flint_stream stream);

/* dwte[v] (+)= sum of dx rows whose token is v (ascending row order, compensated);
 * dwpe[t] (+)= sum over sequences, as flint_bias_gradient sums columns
 * (ref flint.h:298). */
FLINT_API flint_status flint_embedding_backward(void* dwte, void* dwpe, const void* dx,
                                                const void* tokens, size_t sequences,
                                                size_t length, size_t vocab, size_t width,
                                                int accumulate_wte, int accumulate_wpe,
                                                void* workspace, size_t workspace_bytes,
                                                flint_stream stream);

/* Workspace of flint_embedding_backward (ref flint.h:308). */
FLINT_API flint_status flint_embedding_backward_workspace(size_t sequences, size_t length,
                                                          size_t vocab, size_t width,
                                                          size_t* bytes);

/* y = RN16(x), count values, NaN stays NaN (ref flint.h:317). */
FLINT_API flint_status flint_fp32_to_fp16(void* y, const void* x, size_t count,
                                          flint_stream stream);

/* y[b, h, t, c] = x[b * length + t, first + h * head_width + c], as bits
 * (ref flint.h:336). */
FLINT_API flint_status flint_heads_split(void* y, const void* x, size_t batches, size_t length,
                                         size_t heads, size_t head_width, size_t row_width,
                                         size_t first, flint_stream stream);

/* The inverse of flint_heads_split; columns outside the split stay untouched
 * (ref flint.h:346). */
FLINT_API flint_status flint_heads_merge(void* y, const void* x, size_t batches, size_t length,
                                         size_t heads, size_t head_width, size_t row_width,
                                         size_t first, flint_stream stream);

/* p[b, t, c] = RN16(exp(s - max) / sum) over c <= t, +0 for c > t; length a
 * multiple of 8 up to 1,024 (ref flint.h:368). */
FLINT_API flint_status flint_causal_softmax_forward(void* p, const void* s, size_t batches,
                                                    size_t length, flint_stream stream);

/* ds = RN16(scale * p * (dp - D)), D = sum over c <= t of p dp as a compensated
 * pair; +0 for c > t; ds may be dp (ref flint.h:390). */
FLINT_API flint_status flint_causal_softmax_backward(void* ds, const void* p, const void* dp,
                                                     size_t batches, size_t length, float scale,
                                                     flint_stream stream);

/* Per row over the first vocab columns: row_loss = log(sum) - (l_t - max);
 * dlogits = RN16(scale * (p - [c = target])), +0 at c >= vocab (ref flint.h:430). */
FLINT_API flint_status flint_softmax_cross_entropy(void* dlogits, void* row_loss,
                                                   const void* logits, const void* targets,
                                                   float scale, size_t rows, size_t vocab,
                                                   size_t cols, flint_stream stream);

/* GPT-2 assembled from the functions above (ref flint.h:438-573). */
typedef struct flint_gpt2 flint_gpt2;

/* Model shape (ref flint.h:455-466); same field order and types. */
typedef struct {
    size_t layers;
    size_t heads;
    size_t width;
    size_t block_size;
    size_t vocab;
    size_t padded_vocab;
    size_t sequences;
    size_t length;
    int separate_buffers;
    int backward;
} flint_gpt2_config;

/* A master weight or its gradient (ref flint.h:470-475). */
typedef struct {
    const char* name;
    void* data;
    size_t rows;
    size_t cols;
} flint_gpt2_parameter_info;

/* Device bytes flint_gpt2_create would allocate (ref flint.h:482). */
FLINT_API flint_status flint_gpt2_bytes(const flint_gpt2_config* config, size_t* bytes);

/* Allocates a model; weights start uninitialised (ref flint.h:491). */
FLINT_API flint_status flint_gpt2_create(const flint_gpt2_config* config, flint_gpt2** model);

/* Frees a model; null is a no-op (ref flint.h:495). */
FLINT_API void flint_gpt2_destroy(flint_gpt2* model);

/* Number of master weights, 0 for null (ref flint.h:498). */
FLINT_API size_t flint_gpt2_parameter_count(const flint_gpt2* model);

/* The index-th master weight, PyTorch named_parameters order (ref flint.h:503). */
FLINT_API flint_status flint_gpt2_parameter(const flint_gpt2* model, size_t index,
                                            flint_gpt2_parameter_info* info);

/* FP32 master weights -> FP16 compute copies (ref flint.h:509). */
FLINT_API flint_status flint_gpt2_sync_weights(flint_gpt2* model, flint_stream stream);

/* Forward pass to logits, row_loss and dlogits (ref flint.h:522). */
FLINT_API flint_status flint_gpt2_forward(flint_gpt2* model, const void* tokens,
                                          const void* targets, float scale, flint_stream stream);

/* Backward pass to every master weight's gradient (ref flint.h:552). */
FLINT_API flint_status flint_gpt2_backward(flint_gpt2* model, const void* tokens, int accumulate,
                                           flint_stream stream);

/* The index-th gradient (ref flint.h:559). */
FLINT_API flint_status flint_gpt2_gradient(const flint_gpt2* model, size_t index,
                                           flint_gpt2_parameter_info* info);

/* Where the forward pass leaves logits, dlogits and row_loss (ref flint.h:566). */
FLINT_API flint_status flint_gpt2_outputs(const flint_gpt2* model, const void** logits,
                                          const void** dlogits, const void** row_loss);

/* Waits for stream and returns the FP64 mean of row_loss (ref flint.h:573). */
FLINT_API flint_status flint_gpt2_mean_loss(flint_gpt2* model, flint_stream stream, double* loss);

#ifdef __cplusplus
}
#endif

#endif /* FLINT_FLINT_H */
