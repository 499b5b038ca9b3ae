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

#ifdef __cplusplus
}
#endif

#endif /* FLINT_FLINT_ATTENTION_H */
