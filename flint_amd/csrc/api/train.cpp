// C ABI of the training-step extension (include/flint/flint_train.h): argument
// checks, the cut of every tensor into chunks, and the launches of
// kernels/optimizer.hip. No counterpart in the reference's ABI; the step it
// implements is ref scripts/gpt2_torch.py:161-192 with the constants at :37-42.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <string>
#include <vector>

#include "common/args.h"
#include "kernels/kernels.h"

using flint::fail;

namespace {

constexpr size_t kMaxCount = size_t{1} << 40;   // elements per tensor

size_t chunks_of(size_t n) { return (n + flint::kAdamwChunk - 1) / flint::kAdamwChunk; }

flint_status check_tensors(const char* name, const flint_adamw_tensor* tensors, size_t count, size_t* chunks) {
    if (count > 0 && tensors == nullptr) return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: tensors is null", name);
    if (count > flint::kAdamwMaxTensors)
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: %zu tensors, at most %zu", name, count,
                    flint::kAdamwMaxTensors);
    size_t total = 0;
    for (size_t i = 0; i < count; ++i) {
        const size_t n = tensors[i].count;
        if (n > kMaxCount) return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: tensor %zu has %zu values", name, i, n);
        if (!std::isfinite(tensors[i].weight_decay) || tensors[i].weight_decay < 0)
            return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: tensor %zu: weight_decay must be finite and >= 0",
                        name, i);
        total += chunks_of(n);
    }
    if (total > size_t{1} << 30) return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: too many values", name);
    *chunks = total;
    return FLINT_OK;
}

flint_status check_options(const char* name, const flint_adamw_options* o) {
    if (o == nullptr) return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: options is null", name);
    if (!(o->lr >= 0) || !std::isfinite(o->lr)) return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: lr must be finite and >= 0", name);
    if (!(o->beta1 >= 0 && o->beta1 < 1) || !(o->beta2 >= 0 && o->beta2 < 1))
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: betas must lie in [0, 1)", name);
    if (!(o->eps > 0) || !std::isfinite(o->eps)) return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: eps must be positive", name);
    if (!std::isfinite(o->max_grad_norm)) return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: max_grad_norm must be finite", name);
    if (!(o->growth_factor >= 1) || !std::isfinite(o->growth_factor) || !(o->backoff_factor > 0 && o->backoff_factor <= 1))
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: growth_factor must be >= 1 and backoff_factor in (0, 1]", name);
    if (o->growth_interval < 1) return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: growth_interval must be >= 1", name);
    return FLINT_OK;
}

// No buffer of one tensor may overlap a buffer of another: a tensor listed
// twice (a tied weight passed for both uses) would be stepped twice, and two
// tensors sharing moments would race inside one launch. Each tensor's own
// buffers are checked apart already, so after sorting all ranges by address
// a range that overlaps any earlier one overlaps the earlier range reaching
// furthest, which then belongs to another tensor.
flint_status check_apart(const char* name, const flint_adamw_tensor* tensors, size_t count) {
    struct Range {
        uintptr_t begin, end;
        size_t tensor;
        const char* what;
    };
    std::vector<Range> ranges;
    ranges.reserve(count * 5);
    for (size_t i = 0; i < count; ++i) {
        const flint_adamw_tensor& t = tensors[i];
        if (t.count == 0) continue;
        const auto add = [&](const void* p, size_t bytes, const char* what) {
            if (p != nullptr) {
                const uintptr_t b = reinterpret_cast<uintptr_t>(p);
                ranges.push_back({b, b + bytes, i, what});
            }
        };
        add(t.param, t.count * 4, "param");
        add(t.exp_avg, t.count * 4, "exp_avg");
        add(t.exp_avg_sq, t.count * 4, "exp_avg_sq");
        add(t.param_half, t.count * 2, "param_half");
        add(t.grad, t.count * 4, "grad");
    }
    std::sort(ranges.begin(), ranges.end(), [](const Range& a, const Range& b) { return a.begin < b.begin; });
    const Range* reach = nullptr;
    for (const Range& r : ranges) {
        if (reach != nullptr && r.begin < reach->end && r.tensor != reach->tensor)
            return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: tensor %zu's %s and tensor %zu's %s overlap", name,
                        reach->tensor, reach->what, r.tensor, r.what);
        if (reach == nullptr || r.end > reach->end) reach = &r;
    }
    return FLINT_OK;
}

}  // namespace

FLINT_API flint_status flint_adamw_defaults(flint_adamw_options* options) {
    if (options == nullptr) return fail(FLINT_ERROR_INVALID_ARGUMENT, "flint_adamw_defaults: options is null");
    *options = flint_adamw_options{6e-4f, 0.9f, 0.95f, 1e-8f, 1.0f, 2.0f, 0.5f, 2000};
    return FLINT_OK;
}

FLINT_API flint_status flint_train_state_init(void* state, float loss_scale, flint_stream stream) {
    constexpr const char* name = "flint_train_state_init";
    if (!(loss_scale > 0) || !std::isfinite(loss_scale))
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: loss_scale must be positive and finite", name);
    if (flint_status s = flint::Checker(name).buffers({{"state", state, sizeof(flint_train_state)}}, 1).status();
        s != FLINT_OK)
        return s;
    FLINT_HIP_CHECK(flint::launch_train_state_init(state, loss_scale, flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_adamw_workspace(const flint_adamw_tensor* tensors, size_t count, size_t* bytes) {
    constexpr const char* name = "flint_adamw_workspace";
    if (bytes == nullptr) return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: bytes is null", name);
    size_t chunks = 0;
    if (flint_status s = check_tensors(name, tensors, count, &chunks); s != FLINT_OK) return s;
    *bytes = flint::adamw_workspace(chunks);
    return FLINT_OK;
}

FLINT_API flint_status flint_adamw_step(const flint_adamw_tensor* tensors, size_t count, void* state,
                                        const flint_adamw_options* options, void* workspace,
                                        size_t workspace_bytes, flint_stream stream) {
    constexpr const char* name = "flint_adamw_step";
    size_t chunks = 0;
    if (flint_status s = check_tensors(name, tensors, count, &chunks); s != FLINT_OK) return s;
    if (flint_status s = check_options(name, options); s != FLINT_OK) return s;
    const size_t needed = flint::adamw_workspace(chunks);
    if (workspace_bytes < needed)
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: needs %zu bytes of workspace, given %zu", name, needed,
                    workspace_bytes);
    if (flint_status s = flint::Checker(name)
                             .buffers({{"state", state, sizeof(flint_train_state)}, {"workspace", workspace, needed}}, 2)
                             .status();
        s != FLINT_OK)
        return s;
    // Each tensor's buffers: aligned, in range, the outputs apart from each
    // other, from the gradient, and from the state and workspace.
    for (size_t i = 0; i < count; ++i) {
        const flint_adamw_tensor& t = tensors[i];
        if (t.count == 0) continue;
        const size_t b4 = t.count * 4;
        flint::Span buffers[7] = {
            {"param", t.param, b4},           {"exp_avg", t.exp_avg, b4}, {"exp_avg_sq", t.exp_avg_sq, b4},
            {"param_half", t.param_half, t.count * 2}, {"grad", t.grad, b4},
            {"state", state, sizeof(flint_train_state)}, {"workspace", workspace, needed},
        };
        size_t outputs = 4;
        if (t.param_half == nullptr) {   // no FP16 copy: check the other six
            buffers[3] = buffers[4];
            buffers[4] = buffers[5];
            buffers[5] = buffers[6];
            outputs = 3;
        }
        const size_t n = t.param_half == nullptr ? 6 : 7;
        if (flint_status s = flint::Checker(name).buffers(buffers, n, outputs).status(); s != FLINT_OK) {
            const std::string why = flint_last_error();
            return fail(s, "%s (tensor %zu)", why.c_str(), i);
        }
    }
    if (flint_status s = check_apart(name, tensors, count); s != FLINT_OK) return s;
    if (chunks == 0) return FLINT_OK;
    const hipStream_t st = flint::to_hip(stream);

    // Groups of up to kAdamwGroup non-empty tensors per launch.
    std::vector<flint::AdamwGroup> groups;
    std::vector<int> blocks;
    int offset = 0;
    for (size_t i = 0; i < count;) {
        flint::AdamwGroup g{};
        g.partial_offset = offset;
        int b = 0;
        while (i < count && g.count < flint::kAdamwGroup) {
            const flint_adamw_tensor& t = tensors[i++];
            if (t.count == 0) continue;
            flint::AdamwTensorArgs& a = g.t[g.count];
            a.p = static_cast<float*>(t.param);
            a.g = static_cast<const float*>(t.grad);
            a.m = static_cast<float*>(t.exp_avg);
            a.v = static_cast<float*>(t.exp_avg_sq);
            a.h = static_cast<__half*>(t.param_half);
            a.n = t.count;
            a.decay = float(1.0 - double(options->lr) * double(t.weight_decay));
            g.block_start[g.count] = b;
            b += int(chunks_of(t.count));
            ++g.count;
        }
        if (g.count == 0) break;
        g.block_start[g.count] = b;
        offset += b;
        groups.push_back(g);
        blocks.push_back(b);
    }
    for (size_t k = 0; k < groups.size(); ++k)
        FLINT_HIP_CHECK(flint::launch_adamw_sumsq(groups[k], blocks[k], workspace, state, st));
    FLINT_HIP_CHECK(flint::launch_adamw_decide(chunks, workspace, state, *options, st));
    for (size_t k = 0; k < groups.size(); ++k)
        FLINT_HIP_CHECK(flint::launch_adamw_update(groups[k], blocks[k], chunks, workspace, *options, st));
    return FLINT_OK;
}
