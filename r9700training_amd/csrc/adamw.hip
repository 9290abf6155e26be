// adamw.hip -- the LoRA factors' AdamW on the card: the reference's Optimiser::step
// (src/optim.cpp:213-296, include/r97/optim.h) over device f32 master weights, moments and
// accumulation buffers.
//
// Bit for bit with the reference's host optimiser: every element operation is the reference's f32
// operation in its order (correctly rounded, never contracted into an FMA; the square root
// through f64, measured: the f32 one differs from the correctly rounded value in ~15% of inputs); the global
// norm is the reference's -- one double partial a fixed 4096-element chunk of the parameters'
// concatenation, each summed in element order (a chunk that spans two parameters continues in the
// next parameter's launch), the partials added on the host in chunk order; the schedule and the
// bias corrections are the reference's host expressions.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <vector>

#include "../../include/r97q.h"
#include "status.h"

// hipcc contracts a * b + c into one FMA by default (one rounding instead of the reference's two):
// contraction is off for this file's arithmetic (written with plain operators: the __f*_rn helpers
// are header functions, compiled outside this pragma, whose products still contract).
#pragma clang fp contract(off)

namespace {

constexpr int64_t kNormChunk = 4096;

__global__ __launch_bounds__(256) void accumulate_kernel(float* __restrict__ acc, const float* __restrict__ g, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) acc[i] = acc[i] + g[i];
}

__global__ __launch_bounds__(256) void scale_kernel(float* __restrict__ x, int64_t n, float s) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = x[i] * s;
}

// chunk c of the concatenation over this parameter's range [off, off + n): the partial continues
// the previous parameter's (a chunk that starts before `off`) or starts at zero
__global__ __launch_bounds__(64) void norm_partials_kernel(const float* __restrict__ x, int64_t n, int64_t off,
                                                           int64_t c0, int64_t c1, double* __restrict__ partials) {
    const int64_t c = c0 + (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (c >= c1) return;
    const int64_t lo = c * kNormChunk, hi = lo + kNormChunk;
    const int64_t a = lo > off ? lo : off, b = hi < off + n ? hi : off + n;
    double part = lo < off ? partials[c] : 0.0;
    for (int64_t e = a; e < b; ++e) {
        const double v = (double)x[e - off];
        part += v * v;
    }
    partials[c] = part;
}

// the AdamW element update (src/optim.cpp:271-281), then the accumulation buffer cleared
__global__ __launch_bounds__(256) void update_kernel(float* __restrict__ w, float* __restrict__ m, float* __restrict__ v,
                                                     float* __restrict__ acc, int64_t n, float lr, float b1, float b2,
                                                     float omb1, float omb2, float eps, float wd, float bc1, float bc2) {
    const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (j >= n) return;
    const float g = acc[j];
    const float mj = b1 * m[j] + omb1 * g;
    const float vj = b2 * v[j] + omb2 * g * g;
    m[j] = mj;
    v[j] = vj;
    const float mh = mj / bc1;
    const float vh = vj / bc2;
    const float wj = w[j];
    // sqrt through f64: the f32 square root here is not always the correctly rounded one, the f64
    // one rounded to f32 is (53 >= 2 * 24 + 2 significant bits: the double rounding is innocuous)
    const float sq = (float)sqrt((double)vh);
    w[j] = wj - lr * (mh / (sq + eps) + wd * wj);
    acc[j] = 0.0f;
}

__global__ __launch_bounds__(256) void to_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const uint32_t u = __float_as_uint(x[i]);
    y[i] = (u & 0x7FFFFFFFu) > 0x7F800000u ? (uint16_t)((u >> 16) | 0x0040u)
                                            : (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

unsigned blocks(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

int64_t total_of(const R97qAdamWParam* p, int32_t count) {
    int64_t t = 0;
    for (int32_t i = 0; i < count; ++i) t += p[i].n;
    return t;
}

}  // namespace

extern "C" {

// src/optim.cpp:113-126
float r97q_scheduled_lr(const R97qAdamWConfig* cfg, int32_t step) {
    if (step <= 0) return 0.0f;
    const double base = cfg->lr > 0.0f ? double(cfg->lr) : 0.0;
    if (cfg->warmup_steps > 0 && step <= cfg->warmup_steps) {
        const double r = double(step) / double(cfg->warmup_steps);
        return float(base * r);
    }
    if (cfg->total_steps <= 0 || cfg->total_steps <= cfg->warmup_steps) return cfg->lr;
    const double floor_v = base * (cfg->lr_floor_frac >= 0.0f ? double(cfg->lr_floor_frac) : 0.0);
    const double horizon = double(cfg->total_steps - cfg->warmup_steps);
    const double tt = double(step - cfg->warmup_steps);
    const double t = tt < horizon ? tt : horizon;
    const double angle = 3.14159265358979323846 * t / horizon;
    return float(floor_v + (base - floor_v) * 0.5 * (1.0 + std::cos(angle)));
}

int64_t r97q_adamw_workspace_bytes(const R97qAdamWParam* params, int32_t count) {
    if (!params || count <= 0) return -1;
    return (total_of(params, count) + kNormChunk - 1) / kNormChunk * (int64_t)sizeof(double);
}

int r97q_adamw_step(const R97qAdamWConfig* cfg, const R97qAdamWParam* params, const float* const* grads,
                    int32_t count, int32_t* updates, int32_t* pending, int32_t* applied, void* workspace,
                    int64_t workspace_bytes, R97IqrStream stream) {
    r97q::clear_error();
    const char* who = "r97q_adamw_step";
    if (!cfg || !params || !grads || count <= 0 || !updates || !pending || cfg->accum_steps <= 0) {
        r97q::set_error("%s: null argument, no parameters or accum_steps < 1", who);
        return R97Q_EINVAL;
    }
    for (int32_t i = 0; i < count; ++i)
        if (!params[i].w || !params[i].m || !params[i].v || !params[i].acc || !grads[i] || params[i].n <= 0) {
            r97q::set_error("%s: parameter %d: null buffer or n <= 0", who, (int)i);
            return R97Q_EINVAL;
        }
    const hipStream_t s = (hipStream_t)stream;
    if (applied) *applied = 0;
    for (int32_t i = 0; i < count; ++i)
        hipLaunchKernelGGL(accumulate_kernel, dim3(blocks(params[i].n, 256)), dim3(256), 0, s, params[i].acc, grads[i],
                           params[i].n);
    if (int e = r97q::launch_status("adamw accumulate")) return e;
    if (++*pending < cfg->accum_steps) return R97Q_OK;

    // the mean of the accumulated gradients (x 1/k; exact for k = 1)
    const float inv_k = 1.0f / float(*pending);
    if (inv_k != 1.0f)
        for (int32_t i = 0; i < count; ++i)
            hipLaunchKernelGGL(scale_kernel, dim3(blocks(params[i].n, 256)), dim3(256), 0, s, params[i].acc, params[i].n,
                               inv_k);
    // the global-norm clip (src/optim.cpp:131-184)
    if (cfg->clip_norm > 0.0f) {
        const int64_t need = r97q_adamw_workspace_bytes(params, count);
        if (workspace_bytes < need || !workspace) {
            r97q::set_error("%s: workspace %lld bytes, needs %lld", who, (long long)workspace_bytes, (long long)need);
            return R97Q_EWORKSPACE;
        }
        double* partials = static_cast<double*>(workspace);
        int64_t off = 0;
        for (int32_t i = 0; i < count; ++i) {
            const int64_t c0 = off / kNormChunk, c1 = (off + params[i].n + kNormChunk - 1) / kNormChunk;
            hipLaunchKernelGGL(norm_partials_kernel, dim3(blocks(c1 - c0, 64)), dim3(64), 0, s, params[i].acc,
                               params[i].n, off, c0, c1, partials);
            off += params[i].n;
        }
        std::vector<double> h((size_t)(need / (int64_t)sizeof(double)));
        if (hipMemcpyAsync(h.data(), partials, (size_t)need, hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess) {
            r97q::set_error("%s: reading the norm's partials back failed", who);
            return R97Q_ELAUNCH;
        }
        double sq = 0.0;
        for (double p : h) sq += p;
        const float norm = float(std::sqrt(sq));
        if (norm > cfg->clip_norm && norm > 0.0f) {
            const float sc = cfg->clip_norm / norm;
            for (int32_t i = 0; i < count; ++i)
                hipLaunchKernelGGL(scale_kernel, dim3(blocks(params[i].n, 256)), dim3(256), 0, s, params[i].acc,
                                   params[i].n, sc);
        }
    }
    const int32_t t = *updates + 1;
    const float lr = r97q_scheduled_lr(cfg, t);
    const float b1 = cfg->beta1, b2 = cfg->beta2;
    const float bc1 = 1.0f - std::pow(b1, float(t));
    const float bc2 = 1.0f - std::pow(b2, float(t));
    for (int32_t i = 0; i < count; ++i) {
        const float wd = params[i].decay && cfg->weight_decay != 0.0f ? cfg->weight_decay : 0.0f;
        hipLaunchKernelGGL(update_kernel, dim3(blocks(params[i].n, 256)), dim3(256), 0, s, params[i].w, params[i].m,
                           params[i].v, params[i].acc, params[i].n, lr, b1, b2, 1.0f - b1, 1.0f - b2, cfg->eps, wd,
                           bc1, bc2);
    }
    if (int e = r97q::launch_status("adamw update")) return e;
    ++*updates;
    *pending = 0;
    if (applied) *applied = 1;
    return R97Q_OK;
}

int r97q_f32_to_bf16(const float* x, uint16_t* y, int64_t n, R97IqrStream stream) {
    r97q::clear_error();
    if (!x || !y || n < 0) {
        r97q::set_error("r97q_f32_to_bf16: null buffer or n < 0");
        return R97Q_EINVAL;
    }
    if (n == 0) return R97Q_OK;
    hipLaunchKernelGGL(to_bf16_kernel, dim3(blocks(n, 256)), dim3(256), 0, (hipStream_t)stream, x, y, n);
    return r97q::launch_status("r97q_f32_to_bf16");
}

}  // extern "C"
