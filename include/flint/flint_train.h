/* libflint training-step extension for MI355X: AdamW with global gradient
 * clipping and a dynamic loss scale, updating FP32 master weights and their
 * FP16 compute copies with no host synchronisation: three kernels (sum of
 * squares, decide, update), the first and last launched once per group of up
 * to 64 tensors.
 *
 * No counterpart in the reference's ABI. The reference's training step (ref
 * scripts/gpt2_torch.py:161-192, constants :37-42) runs on PyTorch:
 * GradScaler.unscale_, clip_grad_norm_(params, 1.0), AdamW (lr 6e-4, betas
 * (0.9, 0.95), eps 1e-8, weight decay 0.1 on tensors of two or more dimensions,
 * none on the others) and GradScaler.step/update. This is the same step for
 * callers that hold the model's master weights and gradients on the device,
 * e.g. through flint_gpt2_parameter and flint_gpt2_gradient.
 *
 * Per call, over all tensors together:
 *   inv = 1 / loss_scale; g = grad * inv (FP32), non-finite anywhere -> skip:
 *   no tensor changes, step stays, loss_scale *= backoff_factor, tracker = 0.
 *   Otherwise norm = ||g||_2 over every tensor; c = min(1, max_grad_norm /
 *   (norm + 1e-6)) when max_grad_norm > 0; g = g * c; step += 1; then per
 *   element, as torch.optim.AdamW:
 *     p *= 1 - lr * weight_decay
 *     m = m + (1 - beta1) (g - m);  v = beta2 v + (1 - beta2) g^2
 *     p -= (lr / (1 - beta1^step)) * m / (sqrt(v) / sqrt(1 - beta2^step) + eps)
 *     param_half = RN16(p)
 *   and the loss scale grows by growth_factor after growth_interval
 *   consecutive finite steps (GradScaler.update).
 * The norm is summed in FP64 over fixed per-block partials merged in a fixed
 * order: the same inputs give the same bits on every run. */
#ifndef FLINT_TRAIN_H
#define FLINT_TRAIN_H

#include "flint/flint.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One tensor of the update: FP32 param, grad (scaled by the loss scale),
 * exp_avg, exp_avg_sq, each count values, 16-byte aligned and not overlapping;
 * param_half (count FP16 values) or null. */
typedef struct {
    void* param;
    const void* grad;
    void* exp_avg;
    void* exp_avg_sq;
    void* param_half;
    size_t count;
    float weight_decay;
} flint_adamw_tensor;

/* Hyper-parameters; flint_adamw_defaults fills the reference's. */
typedef struct {
    float lr;
    float beta1;
    float beta2;
    float eps;
    float max_grad_norm;   /* <= 0: no clipping */
    float growth_factor;   /* GradScaler: 2 */
    float backoff_factor;  /* GradScaler: 0.5 */
    int growth_interval;   /* GradScaler: 2000 */
} flint_adamw_options;

/* The step's device-resident state (32 bytes, 16-byte aligned device memory). */
typedef struct {
    float loss_scale;
    int growth_tracker;   /* consecutive finite steps since the scale last changed */
    int step;             /* optimizer steps taken; skipped calls do not count */
    int found_inf;        /* the last call saw a non-finite gradient (and skipped) */
    double grad_norm;     /* the last call's unscaled gradient norm (inf or NaN if skipped) */
    double clip_coef;     /* the last call's clipping factor */
} flint_train_state;

/* lr 6e-4, betas (0.9, 0.95), eps 1e-8, max_grad_norm 1, growth 2, backoff
 * 0.5, interval 2000 (the reference's constants and GradScaler's defaults). */
FLINT_API flint_status flint_adamw_defaults(flint_adamw_options* options);

/* Writes a fresh state (loss_scale, zero tracker and step) to device memory. */
FLINT_API flint_status flint_train_state_init(void* state, float loss_scale, flint_stream stream);

/* Workspace bytes flint_adamw_step needs for these tensors. */
FLINT_API flint_status flint_adamw_workspace(const flint_adamw_tensor* tensors, size_t count,
                                             size_t* bytes);

/* One clipped, loss-scaled AdamW step over count tensors (count up to 4096). */
FLINT_API flint_status flint_adamw_step(const flint_adamw_tensor* tensors, size_t count, void* state,
                                        const flint_adamw_options* options, void* workspace,
                                        size_t workspace_bytes, flint_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* FLINT_TRAIN_H */
