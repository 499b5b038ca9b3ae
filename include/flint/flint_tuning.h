/* libflint: plan overrides for tests and tuning sweeps.
 *
 * No counterpart in the reference's ABI. Several entry points choose among
 * alternative plans that compute the same bits (a GEMM's tile, a fused step
 * or its unfused form). flint_set_tuning forces one of them, process-wide,
 * so that a test can compare the plans bit for bit and a sweep can time them
 * in one process. The library reads no environment variable: with nothing
 * set, every entry point runs its default plan.
 *
 * Names and values:
 *   "gemm_pipe"     "0" (no pipeline kernel) or "bm,bn,stages[,bk[,waves[,loaders]]]"
 *   "gemm_config"   "bm,bn,bk,stages,waves_m[,waves]" (the non-pipeline kernel)
 *   "gemm_group_m", "gemm_slots"   positive integers (the non-pipeline kernel)
 *   "attn_causal", "fused_grads", "fused_sums", "ln_defer", "ln_fused",
 *   "emb_together", "attn_order", "attn_scores", "emb_scan"   "0" selects the alternative plan
 *   "ce_threads"    "256", "512" or "1024"
 *   "partials_cpl"  "1", "2" or "4"
 * A value the plan cannot use leaves its default in place. Set and clear
 * overrides only while no call of the library runs on another thread, and
 * not between a GPT-2 model's forward and its backward: the backward reads
 * what the forward's plans left (the model keeps the forward's attention
 * layout, but the causal zero span of the stored probabilities follows the
 * overrides of each call).
 */
#ifndef FLINT_FLINT_TUNING_H
#define FLINT_FLINT_TUNING_H

#include "flint/flint.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Sets `name` to a copy of `value`, or clears it when value is null.
 * An unknown name (or a null one) is FLINT_ERROR_INVALID_ARGUMENT. */
FLINT_API flint_status flint_set_tuning(const char* name, const char* value);

#ifdef __cplusplus
}
#endif

#endif /* FLINT_FLINT_TUNING_H */
