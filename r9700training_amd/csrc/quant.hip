// quant.hip -- the coded trunk's activation quantiser on the card: quant_act_i8g and
// had_quant_act_i8g (the reference's host rows src/adjoint/host/quant.cpp:179-372) and their
// straight-through adjoint.
//
// One workgroup a (row, group). The arithmetic is the host rows' own, in f64: the group's values
// (rotated by the unnormalised Walsh-Hadamard transform for the Hadamard op, the same butterfly
// stages), amax, scale = amax * (1/127) (1 for an all-zero group), u = v * (1/scale), the code
// rint(u) clamped to +-127; so the codes and the (f32) scales are the host rows' bits. The adjoint
// takes the written f32 scale back: d = (|v * (1/s)| > 127 ? 0 : g / s), rotated back (W^T = W),
// added into dx once in f32.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "../../include/r97q.h"
#include "iqr_device.h"
#include "status.h"

namespace r97q {
namespace {

constexpr int kQThreads = 256;
constexpr int64_t kMaxRotated = 4096;  // the rotated group lives in LDS as f64
constexpr double kTop = 127.0;

__device__ __forceinline__ double load_x(const void* x, int32_t dtype, int64_t i) {
    if (dtype == R97Q_BF16) return (double)bf16_to_f32(static_cast<const uint16_t*>(x)[i]);
    return (double)static_cast<const float*>(x)[i];
}

// the unnormalised Walsh-Hadamard transform of v[0, t) in LDS (src/adjoint/host/quant.cpp:181-191)
__device__ void fwht_lds(double* v, int64_t t) {
    for (int64_t h = 1; h < t; h <<= 1) {
        for (int64_t p = threadIdx.x; p < t / 2; p += kQThreads) {
            const int64_t j = (p / h) * 2 * h + p % h;
            const double a = v[j], b = v[j + h];
            v[j] = a + b;
            v[j + h] = a - b;
        }
        __syncthreads();
    }
}

__device__ double block_max(double m, double* red) {
    for (int o = 32; o > 0; o >>= 1) {
        const double other = __shfl_xor(m, o);
        m = other > m ? other : m;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    double r = red[0];
    for (int w = 1; w < kQThreads / 64; ++w) r = red[w] > r ? red[w] : r;
    __syncthreads();
    return r;
}

// grid (ngrp, rows)
__global__ __launch_bounds__(kQThreads) void quant_kernel(const void* __restrict__ x, int32_t dtype, int64_t n,
                                                          int64_t group, int32_t rotated, int8_t* __restrict__ codes,
                                                          float* __restrict__ scale) {
    __shared__ double v[kMaxRotated];
    __shared__ double red[kQThreads / 64];
    const int64_t r = blockIdx.y, g = blockIdx.x, ngrp = gridDim.x;
    const int64_t k0 = g * group;
    const int64_t w = group < n - k0 ? group : n - k0;  // a short last group
    const int64_t base = r * n + k0;
    double m = 0.0;
    if (rotated) {
        for (int64_t i = threadIdx.x; i < group; i += kQThreads) v[i] = load_x(x, dtype, base + i);
        __syncthreads();
        fwht_lds(v, group);
        for (int64_t i = threadIdx.x; i < w; i += kQThreads) m = fabs(v[i]) > m ? fabs(v[i]) : m;
    } else {
        for (int64_t i = threadIdx.x; i < w; i += kQThreads) {
            const double a = fabs(load_x(x, dtype, base + i));
            m = a > m ? a : m;
        }
    }
    const double amax = block_max(m, red);
    const double s = amax > 0.0 ? amax * (1.0 / kTop) : 1.0;
    const double inv = 1.0 / s;
    for (int64_t i = threadIdx.x; i < w; i += kQThreads) {
        const double vi = rotated ? v[i] : load_x(x, dtype, base + i);
        const double c = rint(vi * inv);  // nearest, ties to even
        codes[base + i] = (int8_t)(c > kTop ? kTop : c < -kTop ? -kTop : c);
    }
    if (threadIdx.x == 0) scale[r * ngrp + g] = (float)s;
}

// dx[row, group] += W^T (live * g / s)   (src/adjoint/host/quant.cpp:349-368)
__global__ __launch_bounds__(kQThreads) void quant_bwd_kernel(const void* __restrict__ x, int32_t dtype, int64_t n,
                                                              int64_t group, int32_t rotated,
                                                              const float* __restrict__ scale,
                                                              const float* __restrict__ gc, float* __restrict__ dx) {
    __shared__ double v[kMaxRotated];
    __shared__ double d[kMaxRotated];
    const int64_t r = blockIdx.y, g = blockIdx.x, ngrp = gridDim.x;
    const int64_t k0 = g * group;
    const int64_t w = group < n - k0 ? group : n - k0;
    const int64_t base = r * n + k0;
    const double s = (double)scale[r * ngrp + g];
    const double inv = 1.0 / s;
    if (rotated) {
        for (int64_t i = threadIdx.x; i < group; i += kQThreads) v[i] = load_x(x, dtype, base + i);
        __syncthreads();
        fwht_lds(v, group);
        for (int64_t i = threadIdx.x; i < group; i += kQThreads)
            d[i] = fabs(v[i] * inv) > kTop ? 0.0 : (double)gc[base + i] / s;
        __syncthreads();
        fwht_lds(d, group);
        for (int64_t i = threadIdx.x; i < group; i += kQThreads) dx[base + i] = (float)((double)dx[base + i] + d[i]);
    } else {
        for (int64_t i = threadIdx.x; i < w; i += kQThreads) {
            const double vi = load_x(x, dtype, base + i);
            const double di = fabs(vi * inv) > kTop ? 0.0 : (double)gc[base + i] / s;
            dx[base + i] = (float)((double)dx[base + i] + di);
        }
    }
}

// src/adjoint/host/quant.cpp:150-177: the effective group; 0 when the record is outside the rules
int64_t effective_group(int64_t n, int64_t group, int32_t rotated) {
    if (rotated) {
        if (group <= 0 || (group & (group - 1)) != 0 || n % group != 0) return 0;
        return group;
    }
    return (group <= 0 || group > n) ? n : group;
}

int check_args(const void* x, int32_t dtype, int64_t rows, int64_t n, int64_t group, int32_t rotated, const char* who,
               int64_t* eff) {
    if (!x || rows <= 0 || n <= 0 || (dtype != R97Q_BF16 && dtype != R97Q_F32)) {
        set_error("%s: null activation, rows or n < 1, or a dtype other than bf16 / f32", who);
        return R97Q_EINVAL;
    }
    *eff = effective_group(n, group, rotated);
    if (*eff == 0) {
        set_error("%s: 'group' must be a power of two that divides 'n'", who);
        return R97Q_EINVAL;
    }
    if (rotated && *eff > kMaxRotated) {
        set_error("%s: a rotated group of %lld is wider than this kernel's %lld", who, (long long)*eff,
                  (long long)kMaxRotated);
        return R97Q_EUNSUPPORTED;
    }
    if (rows > 65535) {
        set_error("%s: %lld rows; at most 65535 a call", who, (long long)rows);
        return R97Q_EUNSUPPORTED;
    }
    return R97Q_OK;
}

}  // namespace
}  // namespace r97q

using namespace r97q;

extern "C" {

int r97q_quant_act_i8g(const void* x, int32_t x_dtype, int64_t rows, int64_t n, int64_t group, int32_t rotated,
                       int8_t* codes, float* scale, R97IqrStream stream) {
    clear_error();
    const char* who = rotated ? "had_quant_act_i8g" : "quant_act_i8g";
    int64_t eff = 0;
    if (int e = check_args(x, x_dtype, rows, n, group, rotated, who, &eff)) return e;
    if (!codes || !scale) {
        set_error("%s: null codes or scale", who);
        return R97Q_EINVAL;
    }
    const int64_t ngrp = (n + eff - 1) / eff;
    hipLaunchKernelGGL(quant_kernel, dim3((unsigned)ngrp, (unsigned)rows), dim3(kQThreads), 0, (hipStream_t)stream, x,
                       x_dtype, n, eff, rotated, codes, scale);
    return launch_status("quant_kernel");
}

int r97q_quant_act_i8g_bwd(const void* x, int32_t x_dtype, int64_t rows, int64_t n, int64_t group, int32_t rotated,
                           const float* scale, const float* g, float* dx, R97IqrStream stream) {
    clear_error();
    const char* who = rotated ? "had_quant_act_i8g adjoint" : "quant_act_i8g adjoint";
    int64_t eff = 0;
    if (int e = check_args(x, x_dtype, rows, n, group, rotated, who, &eff)) return e;
    if (!scale || !g || !dx) {
        set_error("%s: null scale, cotangent or dx", who);
        return R97Q_EINVAL;
    }
    const int64_t ngrp = (n + eff - 1) / eff;
    hipLaunchKernelGGL(quant_bwd_kernel, dim3((unsigned)ngrp, (unsigned)rows), dim3(kQThreads), 0,
                       (hipStream_t)stream, x, x_dtype, n, eff, rotated, scale, g, dx);
    return launch_status("quant_bwd_kernel");
}

}  // extern "C"
