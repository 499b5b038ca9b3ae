// C-ABI entry points of the fused causal attention (include/flint/flint_attention.h):
// a Checker chain and the launches of kernels/attention.hip.
#include <cmath>

#include "common/args.h"
#include "flint/flint_attention.h"
#include "kernels/kernels.h"

namespace {

using flint::Checker;

Checker& attention_sizes(Checker& c, size_t batches, size_t length, size_t head_width) {
    return c.require(head_width == 64, "head_width (%zu) must be 64", head_width)
        .require(length <= flint::kAttentionMaxLength, "length (%zu) can be up to %zu", length,
                 flint::kAttentionMaxLength)
        .require(batches <= flint::kAttentionMaxBatches, "batches (%zu) can be up to %zu", batches,
                 flint::kAttentionMaxBatches);
}

}  // namespace

extern "C" {

FLINT_API flint_status flint_attention_forward(void* o, void* lse, const void* q, const void* k,
                                               const void* v, size_t batches, size_t length,
                                               size_t head_width, float scale,
                                               flint_stream stream) {
    Checker c("flint_attention_forward");
    attention_sizes(c, batches, length, head_width)
        .require(std::isfinite(scale), "scale (%g) must be finite", double(scale));
    if (!c.ok() || batches == 0 || length == 0) return c.status();
    const size_t mat = batches * length * head_width * 2;
    c.buffers({{"o", o, mat},
               {"lse", lse, batches * length * 4},
               {"q", q, mat},
               {"k", k, mat},
               {"v", v, mat}},
              2);
    if (!c.ok()) return c.status();
    FLINT_HIP_CHECK(flint::launch_attention_forward(o, lse, q, k, v, batches, length, scale,
                                                    flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_attention_backward_workspace(size_t batches, size_t length,
                                                         size_t head_width, size_t* bytes) {
    Checker c("flint_attention_backward_workspace");
    if (!attention_sizes(c.require(bytes != nullptr, "bytes is null"), batches, length, head_width)
             .ok())
        return c.status();
    *bytes = batches * length * 4;
    return FLINT_OK;
}

FLINT_API flint_status flint_attention_backward(void* dq, void* dk, void* dv, const void* dout,
                                                const void* q, const void* k, const void* v,
                                                const void* o, const void* lse, size_t batches,
                                                size_t length, size_t head_width, float scale,
                                                void* workspace, size_t workspace_bytes,
                                                flint_stream stream) {
    Checker c("flint_attention_backward");
    attention_sizes(c, batches, length, head_width)
        .require(std::isfinite(scale), "scale (%g) must be finite", double(scale));
    if (!c.ok() || batches == 0 || length == 0) return c.status();
    const size_t mat = batches * length * head_width * 2;
    const size_t needed = batches * length * 4;
    c.require(workspace_bytes >= needed, "needs %zu bytes of workspace, given %zu", needed,
              workspace_bytes)
        .buffers({{"dq", dq, mat},
                  {"dk", dk, mat},
                  {"dv", dv, mat},
                  {"workspace", workspace, needed},
                  {"dout", dout, mat},
                  {"q", q, mat},
                  {"k", k, mat},
                  {"v", v, mat},
                  {"o", o, mat},
                  {"lse", lse, batches * length * 4}},
                 4);
    if (!c.ok()) return c.status();
    FLINT_HIP_CHECK(flint::launch_attention_backward(dq, dk, dv, dout, q, k, v, o, lse, workspace,
                                                     batches, length, scale,
                                                     flint::to_hip(stream)));
    return FLINT_OK;
}

}  // extern "C"
