/* libflint: fused causal attention (the reference's roadmap item M3, ref
 * README.md:146), which replaces the materialised scores and probabilities of
 * the GPT-2 step (ref src/api/gpt2.cpp:511-514 forward, :597-603 backward).
 *
 * No counterpart in the reference's ABI: these are additive entry points.
 *
 * q, k, v, o, dout, dq, dk, dv hold batches x length x head_width FP16 values
 * (one [length][head_width] matrix per batch, as flint_heads_split writes them);
 * lse holds batches x length FP32 values. head_width must be 64. Scores are
 * scale * q k^T with key t' visible to query t when t' <= t.
 */
#ifndef FLINT_FLINT_ATTENTION_H
#define FLINT_FLINT_ATTENTION_H

#include "flint/flint.h"

#ifdef __cplusplus
extern "C" {
#endif

/* o[t] = sum over t' <= t of softmax(scale q[t] k^T)[t'] v[t'] (RN16 of an
 * FP32 result), and lse[t] = log(sum over t' <= t of exp(scale q[t] . k[t'])),
 * the natural log-sum-exp the backward pass needs. The length x length scores
 * are never stored: exponentials are taken in FP32 with a running maximum, and
 * the probabilities enter the product with v as FP16. */
FLINT_API flint_status flint_attention_forward(void* o, void* lse, const void* q, const void* k,
                                               const void* v, size_t batches, size_t length,
                                               size_t head_width, float scale,
                                               flint_stream stream);

/* Workspace flint_attention_backward needs: batches x length FP32 values. */
FLINT_API flint_status flint_attention_backward_workspace(size_t batches, size_t length,
                                                         size_t head_width, size_t* bytes);

/* dq, dk, dv: the gradients of sum(dout * o) for the o flint_attention_forward
 * returned with this q, k, v, scale and its lse. Deterministic (fixed
 * summation order, no atomics). dq, dk and dv must not overlap each other or
 * any input. */
FLINT_API flint_status flint_attention_backward(void* dq, void* dk, void* dv, const void* dout,
                                                const void* q, const void* k, const void* v,
                                                const void* o, const void* lse, size_t batches,
                                                size_t length, size_t head_width, float scale,
                                                void* workspace, size_t workspace_bytes,
                                                flint_stream stream);

/* The GPT-2 model with the fused attention in each block's place of the
 * reference's stored scores and probabilities (flint_heads_split, the batched
 * products, flint_causal_softmax_* and flint_heads_merge): the kernels above
 * read each head's q, k and v rows inside the qkv projection and write their
 * output rows into the attention projection's input, so a block keeps the
 * projection and the log-sum-exp instead of q, k, v and the probabilities.
 * Everything else is flint_gpt2_bytes / flint_gpt2_create's model, and every
 * other flint_gpt2_* function takes it. The results pass the same accuracy
 * bounds but differ in the last bits from the stored-probability model, which
 * is the one equal to the public kernels called one by one. The head width
 * (width / heads) must be 64. */
FLINT_API flint_status flint_gpt2_bytes_fused(const flint_gpt2_config* config, size_t* bytes);
FLINT_API flint_status flint_gpt2_create_fused(const flint_gpt2_config* config,
                                               flint_gpt2** model);

#ifdef __cplusplus
}
#endif

#endif /* FLINT_FLINT_ATTENTION_H */
