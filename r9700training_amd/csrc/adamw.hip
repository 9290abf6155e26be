// adamw.hip -- the LoRA factors' AdamW on the card: the reference's Optimiser::step
// (src/optim.cpp:223-307, include/r97/optim.h) over device f32 master weights, moments and
// accumulation buffers.
//
// Bit for bit with the reference's host optimiser: every element operation is the reference's f32
// operation in its order (correctly rounded, never contracted into an FMA; the square root
// through f64, measured: the f32 one differs from the correctly rounded value in ~15% of inputs); the global
// norm is the reference's -- one double partial a fixed 4096-element chunk of the parameters'
// concatenation, each summed in element order (a chunk that spans two parameters continues across
// them), the partials added in chunk order; the schedule and the bias corrections are the
// reference's host expressions.
//
// Launches: an update is one elementwise pass over every parameter (a table of up to kTable
// parameters a launch), reading this call's gradients and/or the accumulation buffers, and writing
// the weights, both moments, the cleared buffers and (optionally) the weights' bf16 copies. The
// reference's in-place passes over the buffers (the sum, the mean, the clip's scaling) are folded
// into that pass as the same f32 operations on the value. With clipping, two launches come first:
// the chunk partials, then one thread that adds them and leaves the clip factor on the card -- no
// host read-back, nothing to synchronise.
//
// Staged gradients (R97Q_ADAMW_GRADS_STAGED): the gradients are the device rows' f32 staging
// buffers; the call takes each value as the reference's grad_stage flush leaves it in a zero-filled
// leaf (one bf16 rounding, src/adjoint/device/grad_stage.cpp:69-73) and clears the buffers in the
// same pass -- the flush, the leaf fill and the optimiser's step in one.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "../../include/r97q.h"
#include "status.h"

// hipcc contracts a * b + c into one FMA by default (one rounding instead of the reference's two):
// contraction is off for this file's arithmetic (written with plain operators: the __f*_rn helpers
// are header functions, compiled outside this pragma, whose products still contract).
#pragma clang fp contract(off)

namespace {

constexpr int64_t kNormChunk = 4096;
constexpr int kTable = 16;        // parameters a launch (the table travels in the kernel arguments)
constexpr int64_t kScaleBytes = 16;  // the workspace's head: the clip factor (f32), then the partials

// where this call's gradient total comes from
constexpr int kFromAcc = 1;  // the accumulation buffers (earlier calls' sums)
constexpr int kFromG = 2;    // this call's gradients
constexpr int kStaged = 4;   // ... staged: rounded once to bf16, and the staging buffers cleared

struct Row {
    float* w;
    float* m;
    float* v;
    float* acc;
    float* g;
    uint16_t* wb;
    int64_t n;
    int64_t off;     // first element in the parameters' concatenation
    int64_t block0;  // first block of this parameter in the launch
    float wd;
};

struct Table {
    Row r[kTable];
    int count;
};

__device__ __forceinline__ int row_of_block(const Table& t, int64_t block) {
    int i = 0;
    while (i + 1 < t.count && block >= t.r[i + 1].block0) ++i;
    return i;
}

__device__ __forceinline__ uint16_t bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x7FFFFFFFu) > 0x7F800000u ? (uint16_t)((u >> 16) | 0x0040u)
                                           : (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// this call's gradient value (staged: as the flush leaves it in the leaf)
__device__ __forceinline__ float grad_of(const Row& r, int64_t j, int mode) {
    const float g = r.g[j];
    return (mode & kStaged) ? __uint_as_float((uint32_t)bf16_rne(g) << 16) : g;
}

// the accumulated gradient as the reference's buffer holds it when the update reads it:
// (acc + g) (the last call's accumulation), x 1/k (the mean, when k > 1)
__device__ __forceinline__ float grad_total(const Row& r, int64_t j, int mode, float inv_k) {
    float x;
    if ((mode & kFromAcc) && (mode & kFromG))
        x = r.acc[j] + grad_of(r, j, mode);
    else if (mode & kFromG)
        x = grad_of(r, j, mode);  // the buffer held zero: 0 + g is g (a -0 that would turn +0 changes no result)
    else
        x = r.acc[j];
    return inv_k != 1.0f ? x * inv_k : x;
}

__global__ __launch_bounds__(256) void accumulate_kernel(const Table t, int mode) {
    const Row& r = t.r[row_of_block(t, blockIdx.x)];
    const int64_t j = ((int64_t)blockIdx.x - r.block0) * 256 + threadIdx.x;
    if (j >= r.n) return;
    r.acc[j] = r.acc[j] + grad_of(r, j, mode);
    if (mode & kStaged) r.g[j] = 0.0f;
}

// chunk c of the concatenation, over the part of it this launch's parameters hold; a chunk that
// starts before the launch's first element continues the partial an earlier launch left
__global__ __launch_bounds__(64) void norm_partials_kernel(const Table t, int mode, float inv_k, int64_t c0,
                                                           int64_t c1, double* __restrict__ partials) {
    const int64_t c = c0 + (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (c >= c1) return;
    const int64_t first = t.r[0].off, end = t.r[t.count - 1].off + t.r[t.count - 1].n;
    const int64_t lo = c * kNormChunk, hi = lo + kNormChunk;
    int64_t e = lo > first ? lo : first;
    const int64_t stop = hi < end ? hi : end;
    double part = lo < first ? partials[c] : 0.0;
    int i = 0;
    while (e >= t.r[i].off + t.r[i].n) ++i;
    for (; e < stop; ++e) {
        if (e >= t.r[i].off + t.r[i].n) ++i;
        const double v = (double)grad_total(t.r[i], e - t.r[i].off, mode, inv_k);
        part += v * v;
    }
    partials[c] = part;
}

// src/optim.cpp:131-184: the norm from the chunk partials (added in chunk order), and the factor
// the clip multiplies by (1 when it does not bite: x * 1 is x)
__global__ void clip_factor_kernel(const double* __restrict__ partials, int64_t chunks, float clip,
                                   float* __restrict__ factor) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    double sq = 0.0;
    for (int64_t c = 0; c < chunks; ++c) sq += partials[c];
    const float norm = (float)sqrt(sq);
    *factor = norm > clip && norm > 0.0f ? clip / norm : 1.0f;
}

// the AdamW element update (src/optim.cpp:278-289); the accumulation buffer cleared when it was read
__global__ __launch_bounds__(256) void update_kernel(const Table t, int mode, float inv_k,
                                                     const float* __restrict__ clip, float lr, float b1, float b2,
                                                     float omb1, float omb2, float eps, float bc1, float bc2) {
    const Row& r = t.r[row_of_block(t, blockIdx.x)];
    const int64_t j = ((int64_t)blockIdx.x - r.block0) * 256 + threadIdx.x;
    if (j >= r.n) return;
    float g = grad_total(r, j, mode, inv_k);
    if (clip) g = g * *clip;
    const float mj = b1 * r.m[j] + omb1 * g;
    const float vj = b2 * r.v[j] + omb2 * g * g;
    r.m[j] = mj;
    r.v[j] = vj;
    const float mh = mj / bc1;
    const float vh = vj / bc2;
    const float wj = r.w[j];
    // sqrt through f64: the f32 square root here is not always the correctly rounded one, the f64
    // one rounded to f32 is (53 >= 2 * 24 + 2 significant bits: the double rounding is innocuous)
    const float sq = (float)sqrt((double)vh);
    const float wn = wj - lr * (mh / (sq + eps) + r.wd * wj);
    r.w[j] = wn;
    if (mode & kFromAcc) r.acc[j] = 0.0f;
    if (mode & kStaged) r.g[j] = 0.0f;
    if (r.wb) r.wb[j] = bf16_rne(wn);
}

__global__ __launch_bounds__(256) void to_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = bf16_rne(x[i]);
}

unsigned blocks(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

int64_t total_of(const R97qAdamWParam* p, int32_t count) {
    int64_t t = 0;
    for (int32_t i = 0; i < count; ++i) t += p[i].n;
    return t;
}

// the launch tables: parameters [first, first + kTable) of the call, their offsets in the concatenation
template <class F>
int for_each_table(const R97qAdamWParam* p, float* const* grads, int32_t count, float weight_decay, F&& f) {
    int64_t off = 0;
    for (int32_t first = 0; first < count; first += kTable) {
        Table t{};
        t.count = count - first < kTable ? count - first : kTable;
        int64_t nblocks = 0;
        for (int i = 0; i < t.count; ++i) {
            const R97qAdamWParam& q = p[first + i];
            t.r[i] = Row{q.w, q.m, q.v, q.acc, grads[first + i], q.w_bf16, q.n, off, nblocks,
                         q.decay && weight_decay != 0.0f ? weight_decay : 0.0f};
            off += q.n;
            nblocks += blocks(q.n, 256);
        }
        if (int e = f(t, nblocks)) return e;
    }
    return R97Q_OK;
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
    return kScaleBytes + (total_of(params, count) + kNormChunk - 1) / kNormChunk * (int64_t)sizeof(double);
}

int r97q_adamw_step(const R97qAdamWConfig* cfg, const R97qAdamWParam* params, float* const* grads,
                    int32_t count, int32_t flags, int32_t* updates, int32_t* pending, int32_t* applied,
                    void* workspace, int64_t workspace_bytes, R97IqrStream stream) {
    r97q::clear_error();
    const char* who = "r97q_adamw_step";
    if (!cfg || !params || !grads || count <= 0 || !updates || !pending || cfg->accum_steps <= 0 ||
        (flags & ~R97Q_ADAMW_GRADS_STAGED)) {
        r97q::set_error("%s: null argument, no parameters, accum_steps < 1 or unknown flags", who);
        return R97Q_EINVAL;
    }
    for (int32_t i = 0; i < count; ++i)
        if (!params[i].w || !params[i].m || !params[i].v || !params[i].acc || !grads[i] || params[i].n <= 0) {
            r97q::set_error("%s: parameter %d: null buffer or n <= 0", who, (int)i);
            return R97Q_EINVAL;
        }
    const bool clipping = cfg->clip_norm > 0.0f;
    const int64_t need = r97q_adamw_workspace_bytes(params, count);
    if (clipping && (workspace_bytes < need || !workspace)) {
        r97q::set_error("%s: workspace %lld bytes, needs %lld", who, (long long)workspace_bytes, (long long)need);
        return R97Q_EWORKSPACE;
    }
    const hipStream_t s = (hipStream_t)stream;
    if (applied) *applied = 0;
    const int staged = (flags & R97Q_ADAMW_GRADS_STAGED) ? kStaged : 0;
    const int32_t before = *pending;
    if (++*pending < cfg->accum_steps) {
        // not the update's call: add the gradients into the buffers
        return for_each_table(params, grads, count, 0.0f, [&](const Table& t, int64_t nb) {
            hipLaunchKernelGGL(accumulate_kernel, dim3((unsigned)nb), dim3(256), 0, s, t, kFromG | staged);
            return r97q::launch_status("adamw accumulate");
        });
    }
    const int mode = (before > 0 ? kFromAcc : 0) | kFromG | staged;
    const float inv_k = 1.0f / float(*pending);  // the mean (x 1/k; k = 1 leaves the sum as it is)
    float* factor = nullptr;
    if (clipping) {
        factor = static_cast<float*>(workspace);
        double* partials = reinterpret_cast<double*>(static_cast<uint8_t*>(workspace) + kScaleBytes);
        int e = for_each_table(params, grads, count, 0.0f, [&](const Table& t, int64_t) {
            const int64_t end = t.r[t.count - 1].off + t.r[t.count - 1].n;
            const int64_t c0 = t.r[0].off / kNormChunk, c1 = (end + kNormChunk - 1) / kNormChunk;
            hipLaunchKernelGGL(norm_partials_kernel, dim3(blocks(c1 - c0, 64)), dim3(64), 0, s, t, mode, inv_k, c0, c1,
                               partials);
            return r97q::launch_status("adamw norm partials");
        });
        if (e) return e;
        const int64_t chunks = (total_of(params, count) + kNormChunk - 1) / kNormChunk;
        hipLaunchKernelGGL(clip_factor_kernel, dim3(1), dim3(64), 0, s, partials, chunks, cfg->clip_norm, factor);
        if (int e2 = r97q::launch_status("adamw clip factor")) return e2;
    }
    const int32_t t = *updates + 1;
    const float lr = r97q_scheduled_lr(cfg, t);
    const float b1 = cfg->beta1, b2 = cfg->beta2;
    const float bc1 = 1.0f - std::pow(b1, float(t));
    const float bc2 = 1.0f - std::pow(b2, float(t));
    int e = for_each_table(params, grads, count, cfg->weight_decay, [&](const Table& tb, int64_t nb) {
        hipLaunchKernelGGL(update_kernel, dim3((unsigned)nb), dim3(256), 0, s, tb, mode, inv_k, (const float*)factor, lr,
                           b1, b2, 1.0f - b1, 1.0f - b2, cfg->eps, bc1, bc2);
        return r97q::launch_status("adamw update");
    });
    if (e) return e;
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
