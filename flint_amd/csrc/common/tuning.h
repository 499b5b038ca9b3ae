// Plan overrides: named values that force one of a kernel's alternative plans
// (a GEMM tile, the unfused form of a fused step), set through
// flint_set_tuning. Tests use them to check that every plan gives the same
// bits, and tuning sweeps to time the alternatives in one process. The
// library reads no environment variable: with nothing set, every entry point
// runs its default plan, and the same arguments always give the same results.
#pragma once

namespace flint {

enum class Tune : int {
    kGemmPipe,      // "0": no pipeline GEMM; "bm,bn,stages[,bk]": that pipeline tile
    kGemmConfig,    // "bm,bn,bk,stages,waves_m[,waves]": that gemm.hip configuration
    kGemmGroupM,    // gemm.hip's grouped tile order width
    kGemmSlots,     // gemm.hip's persistent workgroup count
    kAttnCausal,    // "0": the model's attention products computed in full
    kFusedGrads,    // "0": the model's weight and bias gradients by the entry points
    kFusedSums,     // "0": the model's LayerNorm backward by the entry point
    kLnDefer,       // "0": the model merges each LayerNorm's partials at once
    kLnFused,       // "0": LayerNorm backward's partials and dx in two launches
    kCeThreads,     // 256 | 512 | 1024: softmax + cross-entropy workgroup size
    kEmbTogether,   // "0": the position gradient in its own launch
    kAttnOrder,     // "0": the fused attention's plain longest-first order
    kPartialsCpl,   // 1 | 2 | 4: bias-gradient partials' columns per lane
    kAttnScores,    // "0": the model's scores and dP through the batched product
                    // and the softmax passes (no fused scores + softmax)
    kEmbScan,       // "0": the embedding backward's token rows through the sort
    kCount
};

// The value set for `t`, or nullptr when none is (one atomic load).
const char* tuning(Tune t);
// Whether `t` is set to exactly `value`.
bool tuning_is(Tune t, const char* value);
// Whether `t` is set to "0" (turns the default plan's alternative on).
inline bool tuning_off(Tune t) { return tuning_is(t, "0"); }

}  // namespace flint
