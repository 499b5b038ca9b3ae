#include "common/tuning.h"

#include <atomic>
#include <cstring>
#include <mutex>
#include <set>
#include <string>

#include "common/common.h"
#include "flint/flint_tuning.h"

namespace flint {
namespace {

constexpr const char* kNames[] = {"gemm_pipe",  "gemm_config",  "gemm_group_m", "gemm_slots",
                                  "attn_causal", "fused_grads", "fused_sums",   "ln_defer",
                                  "ln_fused",    "ce_threads",  "emb_together", "attn_order",
                                  "partials_cpl", "attn_scores", "emb_scan"};
static_assert(sizeof(kNames) / sizeof(kNames[0]) == size_t(Tune::kCount), "one name per knob");

// Values are interned and never freed, so a pointer a reader loaded stays
// valid whatever is set later.
std::atomic<const char*> g_values[size_t(Tune::kCount)];
std::mutex g_mutex;
std::set<std::string>& interned() {
    static std::set<std::string> s;
    return s;
}

}  // namespace

const char* tuning(Tune t) { return g_values[size_t(t)].load(std::memory_order_acquire); }

bool tuning_is(Tune t, const char* value) {
    const char* v = tuning(t);
    return v != nullptr && std::strcmp(v, value) == 0;
}

}  // namespace flint

extern "C" FLINT_API flint_status flint_set_tuning(const char* name, const char* value) {
    using namespace flint;
    if (name == nullptr) return fail(FLINT_ERROR_INVALID_ARGUMENT, "flint_set_tuning: name is null");
    for (size_t i = 0; i < size_t(Tune::kCount); ++i) {
        if (std::strcmp(name, kNames[i]) != 0) continue;
        const char* stored = nullptr;
        if (value != nullptr) {
            std::lock_guard<std::mutex> lock(g_mutex);
            stored = interned().insert(value).first->c_str();
        }
        g_values[i].store(stored, std::memory_order_release);
        return FLINT_OK;
    }
    return fail(FLINT_ERROR_INVALID_ARGUMENT, "flint_set_tuning: unknown name \"%s\"", name);
}
