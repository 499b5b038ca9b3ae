// AdamW with global gradient clipping and a dynamic loss scale, over many
// tensors at once (the step after backward; spec ref scripts/gpt2_torch.py:
// 37-42 and 161-192, which runs torch.optim.AdamW, clip_grad_norm_ and
// GradScaler).
//
// Three kernels per step, all on the caller's stream and none waiting on the
// host:
//   adamw_sumsq   one workgroup per 8,192-element chunk of a tensor: the sum
//                 of (grad / loss_scale)^2 over the chunk, in FP64, reduced in a
//                 fixed tree, to partials[chunk]. A non-finite gradient makes its
//                 partial non-finite.
//   adamw_decide  one workgroup: sums the partials in a fixed order, decides
//                 skip / clip factor / bias corrections, and updates the
//                 device state (loss scale, growth tracker, step count).
//   adamw_update  one workgroup per chunk again: the elementwise AdamW update
//                 and the FP16 copy, or nothing when the step was skipped.
// HBM traffic per element: 4 bytes in the first kernel, 16 read + 12 written
// (+2 with the FP16 copy) in the last; 34 bytes in all. Tensors are passed by
// value in groups of up to kAdamwGroup per launch (kernel arguments), so no
// table lives in device memory.
#include "kernels.h"

#include <hip/hip_fp16.h>

#include <cmath>

namespace flint {
namespace {

constexpr int kThreads = 256;
static_assert(kAdamwChunk % (4 * kThreads * 4) == 0, "whole float4 rounds per chunk");

struct Decision {
    float inv_scale;   // 1 / loss scale used for this step's gradients
    float clip;        // clipping factor (1 without clipping)
    float step_size;   // lr / (1 - beta1^step)
    float bc2_sqrt;    // sqrt(1 - beta2^step)
    int skip;          // non-finite gradients: change nothing
    int pad[3];
};

__device__ inline double block_sum(double v, double* lds) {
    lds[threadIdx.x] = v;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if (int(threadIdx.x) < s) lds[threadIdx.x] += lds[threadIdx.x + s];
        __syncthreads();
    }
    return lds[0];
}

// The tensor of workgroup b and the chunk's first element.
__device__ inline int find_tensor(const AdamwGroup& g, int b) {
    int i = 0;
    while (i + 1 < g.count && g.block_start[i + 1] <= b) ++i;
    return i;
}

__global__ void __launch_bounds__(kThreads) adamw_sumsq(AdamwGroup group, double* partials,
                                                         const flint_train_state* state) {
    __shared__ double lds[kThreads];
    const int b = blockIdx.x;
    const int i = find_tensor(group, b);
    const AdamwTensorArgs& t = group.t[i];
    const unsigned long long begin = (unsigned long long)(b - group.block_start[i]) * kAdamwChunk;
    const unsigned long long end = begin + kAdamwChunk < t.n ? begin + kAdamwChunk : t.n;
    const float inv = float(1.0 / double(state->loss_scale));
    double acc = 0;
    constexpr int kPer = int(kAdamwChunk / (4 * kThreads));   // float4s per thread in a chunk
    if (end - begin == kAdamwChunk) {
        // A whole chunk: every load issued before the first add, the adds in
        // the order of the loop below (the same sum).
        float4 gv[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k)
            gv[k] = *reinterpret_cast<const float4*>(t.g + begin + 4ull * threadIdx.x +
                                                     4ull * kThreads * k);
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const float a = gv[k].x * inv, bb = gv[k].y * inv, c = gv[k].z * inv, d = gv[k].w * inv;
            acc += double(a) * a + double(bb) * bb + double(c) * c + double(d) * d;
        }
        const double sum = block_sum(acc, lds);
        if (threadIdx.x == 0) partials[group.partial_offset + b] = sum;
        return;
    }
    for (unsigned long long e = begin + 4ull * threadIdx.x; e < end; e += 4ull * kThreads) {
        if (e + 3 < end) {
            const float4 g = *reinterpret_cast<const float4*>(t.g + e);
            const float a = g.x * inv, bb = g.y * inv, c = g.z * inv, d = g.w * inv;
            acc += double(a) * a + double(bb) * bb + double(c) * c + double(d) * d;
        } else {
            for (unsigned long long k = e; k < end; ++k) {
                const float a = t.g[k] * inv;
                acc += double(a) * a;
            }
        }
    }
    const double sum = block_sum(acc, lds);
    if (threadIdx.x == 0) partials[group.partial_offset + b] = sum;
}

__global__ void __launch_bounds__(kThreads) adamw_decide(const double* partials, int count,
                                                          flint_train_state* state, Decision* decision,
                                                          float max_grad_norm, float beta1, float beta2,
                                                          float lr, float growth_factor,
                                                          float backoff_factor, int growth_interval) {
    __shared__ double lds[kThreads];
    double acc = 0;
    // Eight loads in flight per thread, added in order (the same sum).
    int k = threadIdx.x;
    for (; k + 7 * kThreads < count; k += 8 * kThreads) {
        double v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = partials[k + j * kThreads];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc += v[j];
    }
    for (; k < count; k += kThreads) acc += partials[k];
    const double sumsq = block_sum(acc, lds);
    if (threadIdx.x != 0) return;
    flint_train_state s = *state;
    Decision d{};
    d.inv_scale = float(1.0 / double(s.loss_scale));
    if (!isfinite(sumsq)) {
        d.skip = 1;
        s.found_inf = 1;
        s.grad_norm = sqrt(sumsq);
        s.clip_coef = 0;
        s.loss_scale *= backoff_factor;
        s.growth_tracker = 0;
    } else {
        const double norm = sqrt(sumsq);
        double clip = 1.0;
        if (max_grad_norm > 0) clip = fmin(1.0, double(max_grad_norm) / (norm + 1e-6));
        d.clip = float(clip);
        s.found_inf = 0;
        s.grad_norm = norm;
        s.clip_coef = d.clip;
        s.step += 1;
        d.step_size = float(double(lr) / (1.0 - pow(double(beta1), double(s.step))));
        d.bc2_sqrt = float(sqrt(1.0 - pow(double(beta2), double(s.step))));
        if (s.growth_tracker + 1 == growth_interval) {
            s.loss_scale *= growth_factor;
            s.growth_tracker = 0;
        } else {
            s.growth_tracker += 1;
        }
    }
    *state = s;
    *decision = d;
}

struct Moments {
    float beta1, beta2, eps;
};

__device__ inline void adamw_element(float& p, float g, float& m, float& v, float decay, const Decision& d,
                                     const Moments& mo) {
    g = g * d.inv_scale;
    g = g * d.clip;
    p = p * decay;
    m = m + (1.0f - mo.beta1) * (g - m);
    v = v * mo.beta2 + (1.0f - mo.beta2) * (g * g);
    const float denom = sqrtf(v) / d.bc2_sqrt + mo.eps;
    p = p - d.step_size * (m / denom);
}

__global__ void __launch_bounds__(kThreads) adamw_update(AdamwGroup group, const Decision* decision,
                                                          Moments mo) {
    const Decision d = *decision;
    if (d.skip) return;
    const int b = blockIdx.x;
    const int i = find_tensor(group, b);
    const AdamwTensorArgs& t = group.t[i];
    const unsigned long long begin = (unsigned long long)(b - group.block_start[i]) * kAdamwChunk;
    const unsigned long long end = begin + kAdamwChunk < t.n ? begin + kAdamwChunk : t.n;
    if (end - begin == kAdamwChunk) {
        // A whole chunk in rounds of 4 float4s a thread, each round's loads
        // issued before its arithmetic. Every access streams (non-temporal):
        // param, m and v are touched once a step, this is the gradient's last
        // read, and the FP16 copy waits for the next forward. The FP16 pairs
        // go out as one 8-byte store (buffers are 16-byte aligned, e is a
        // multiple of 4).
        typedef float f4v __attribute__((ext_vector_type(4)));
        typedef unsigned u2v __attribute__((ext_vector_type(2)));
        constexpr int kPer = int(kAdamwChunk / (4 * kThreads)), kRound = 4;
        auto load_nt = [](const float* q) {
            return __builtin_bit_cast(float4, __builtin_nontemporal_load(reinterpret_cast<const f4v*>(q)));
        };
        auto store_nt = [](float* q, const float4& x) {
            __builtin_nontemporal_store(__builtin_bit_cast(f4v, x), reinterpret_cast<f4v*>(q));
        };
#pragma unroll
        for (int r0 = 0; r0 < kPer; r0 += kRound) {
            float4 p[kRound], g[kRound], m[kRound], v[kRound];
#pragma unroll
            for (int k = 0; k < kRound; ++k) {
                const unsigned long long e = begin + 4ull * threadIdx.x + 4ull * kThreads * (r0 + k);
                p[k] = load_nt(t.p + e);
                g[k] = load_nt(t.g + e);
                m[k] = load_nt(t.m + e);
                v[k] = load_nt(t.v + e);
            }
#pragma unroll
            for (int k = 0; k < kRound; ++k) {
                const unsigned long long e = begin + 4ull * threadIdx.x + 4ull * kThreads * (r0 + k);
                adamw_element(p[k].x, g[k].x, m[k].x, v[k].x, t.decay, d, mo);
                adamw_element(p[k].y, g[k].y, m[k].y, v[k].y, t.decay, d, mo);
                adamw_element(p[k].z, g[k].z, m[k].z, v[k].z, t.decay, d, mo);
                adamw_element(p[k].w, g[k].w, m[k].w, v[k].w, t.decay, d, mo);
                store_nt(t.p + e, p[k]);
                store_nt(t.m + e, m[k]);
                store_nt(t.v + e, v[k]);
                if (t.h) {
                    const u2v h = {__builtin_bit_cast(unsigned, __floats2half2_rn(p[k].x, p[k].y)),
                                   __builtin_bit_cast(unsigned, __floats2half2_rn(p[k].z, p[k].w))};
                    __builtin_nontemporal_store(h, reinterpret_cast<u2v*>(t.h + e));
                }
            }
        }
        return;
    }
    for (unsigned long long e = begin + 4ull * threadIdx.x; e < end; e += 4ull * kThreads) {
        if (e + 3 < end) {
            float4 p = *reinterpret_cast<const float4*>(t.p + e);
            const float4 g = *reinterpret_cast<const float4*>(t.g + e);
            float4 m = *reinterpret_cast<const float4*>(t.m + e);
            float4 v = *reinterpret_cast<const float4*>(t.v + e);
            adamw_element(p.x, g.x, m.x, v.x, t.decay, d, mo);
            adamw_element(p.y, g.y, m.y, v.y, t.decay, d, mo);
            adamw_element(p.z, g.z, m.z, v.z, t.decay, d, mo);
            adamw_element(p.w, g.w, m.w, v.w, t.decay, d, mo);
            *reinterpret_cast<float4*>(t.p + e) = p;
            *reinterpret_cast<float4*>(t.m + e) = m;
            *reinterpret_cast<float4*>(t.v + e) = v;
            if (t.h) {
                __half2 lo = __floats2half2_rn(p.x, p.y), hi = __floats2half2_rn(p.z, p.w);
                __half2* h = reinterpret_cast<__half2*>(t.h + e);
                h[0] = lo;
                h[1] = hi;
            }
        } else {
            for (unsigned long long k = e; k < end; ++k) {
                float p = t.p[k], m = t.m[k], v = t.v[k];
                adamw_element(p, t.g[k], m, v, t.decay, d, mo);
                t.p[k] = p;
                t.m[k] = m;
                t.v[k] = v;
                if (t.h) t.h[k] = __float2half_rn(p);
            }
        }
    }
}

__global__ void train_state_init(flint_train_state* state, float loss_scale) {
    flint_train_state s{};
    s.loss_scale = loss_scale;
    *state = s;
}

}  // namespace

size_t adamw_decision_offset(size_t chunks) { return (chunks * sizeof(double) + 255) / 256 * 256; }

size_t adamw_workspace(size_t chunks) { return adamw_decision_offset(chunks) + 256; }

hipError_t launch_adamw_sumsq(const AdamwGroup& group, int blocks, void* workspace, const void* state,
                              hipStream_t stream) {
    hipLaunchKernelGGL(adamw_sumsq, dim3(blocks), dim3(kThreads), 0, stream, group,
                       static_cast<double*>(workspace), static_cast<const flint_train_state*>(state));
    return hipGetLastError();
}

hipError_t launch_adamw_decide(size_t chunks, void* workspace, void* state, const flint_adamw_options& o,
                               hipStream_t stream) {
    auto* decision = reinterpret_cast<Decision*>(static_cast<char*>(workspace) + adamw_decision_offset(chunks));
    hipLaunchKernelGGL(adamw_decide, dim3(1), dim3(kThreads), 0, stream, static_cast<const double*>(workspace),
                       int(chunks), static_cast<flint_train_state*>(state), decision, o.max_grad_norm, o.beta1,
                       o.beta2, o.lr, o.growth_factor, o.backoff_factor, o.growth_interval);
    return hipGetLastError();
}

hipError_t launch_adamw_update(const AdamwGroup& group, int blocks, size_t chunks, const void* workspace,
                               const flint_adamw_options& o, hipStream_t stream) {
    const auto* decision =
        reinterpret_cast<const Decision*>(static_cast<const char*>(workspace) + adamw_decision_offset(chunks));
    hipLaunchKernelGGL(adamw_update, dim3(blocks), dim3(kThreads), 0, stream, group, decision,
                       Moments{o.beta1, o.beta2, o.eps});
    return hipGetLastError();
}

hipError_t launch_train_state_init(void* state, float loss_scale, hipStream_t stream) {
    hipLaunchKernelGGL(train_state_init, dim3(1), dim3(1), 0, stream, static_cast<flint_train_state*>(state),
                       loss_scale);
    return hipGetLastError();
}

}  // namespace flint
