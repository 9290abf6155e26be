// fused_quant.hip -- the fused quantiser producers on the card: rmsnorm_had_quant_i8g,
// gated_had_quant_i8g and gate_had_quant_i8g (the reference's host rows
// src/adjoint/host/quant.cpp:896-1405 and device rows src/adjoint/device/quant.hip:959-961).
//
// Each applies an elementwise part to its inputs -- the RMS norm x * rs * (w + wadd) * mult, the
// gated activation silu(gate) * up over gate_up's two halves, or the gate sigmoid(a) * b
// (src/adjoint/host/elementwise.cpp:278-347, 459-641) -- then had_quant_act_i8g over the part's
// output: per group of `group` columns, the unnormalised Walsh-Hadamard transform, scale = amax / 127,
// codes = clamp(rint(v / scale), +-127). The adjoint is the parts' adjoints composed in the order
// the host row composes them: the codes' cotangent divided by the forward's scale, dropped where
// |v / scale| > 127, rotated back; the output write's cotangent added; then the part's adjoint.
//
// One workgroup a row, four waves; each wave takes whole groups. A lane holds max(1, group / 64)
// values of a group (element lane + 64 k), so a group of 64 or more is one wave and a smaller
// group shares a wave with its neighbours. The butterfly stages run in the host's order (h = 1, 2,
// 4, ...): the stages below 64 exchange with lane ^ h, the rest stay in a lane's registers. The
// part's output is formed in f64 from the inputs the way the host twin forms it, so the rotated
// values, the clamp decision and the codes are the host row's; the row's sums (the norm's sum of
// squares and its adjoint's shared term) run in a different order than the host's sequential loops,
// which moves them by an f64 ulp at most. This file is built with -ffp-contract=off so no FMA
// changes a rounding the host loop makes.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "../../include/r97q.h"
#include "iqr_device.h"
#include "status.h"

namespace r97q {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxLogGroup = 10;  // the reference's rows serve groups up to 1024 (quant.hip:129-137)

struct Args {
    const void* x0;
    const void* x1;
    int32_t dtype;
    int64_t n;
    double eps, wadd, mult;
    int8_t* codes;      // forward
    float* scale;       // forward: written; adjoint: the forward's
    uint16_t* y_out;    // forward, may be null
    const float* gc;    // adjoint: the codes' cotangent
    const float* gout;  // adjoint: the output write's cotangent, may be null
    float* dx0;
    float* dx1;
};

__device__ __forceinline__ double ld(const void* p, int32_t dt, int64_t i) {
    if (dt == R97Q_BF16) return (double)bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    if (dt == R97Q_F32) return (double)static_cast<const float*>(p)[i];
    return static_cast<const double*>(p)[i];
}

// src/adjoint/host/elementwise.cpp:121
__device__ __forceinline__ double sigm(double x) { return 1.0 / (1.0 + exp(-x)); }

template <int G>
struct Geo {
    static constexpr int V = G >= 64 ? G / 64 : 1;  // values a lane holds
    static constexpr int L = G >= 64 ? 64 : G;       // lanes a group spans
    static constexpr int E = 64 * V;                  // columns one wave step covers
};

// the unnormalised Walsh-Hadamard transform of each group (src/adjoint/host/quant.cpp:181-191)
template <int G>
__device__ __forceinline__ void fwht(double (&v)[Geo<G>::V], int lane) {
    constexpr int V = Geo<G>::V;
#pragma unroll
    for (int h = 1; h < G; h <<= 1) {
        if (h < 64) {
#pragma unroll
            for (int k = 0; k < V; ++k) {
                const double o = __shfl_xor(v[k], h);
                v[k] = (lane & h) ? o - v[k] : v[k] + o;
            }
        } else {
            const int hb = h / 64;
#pragma unroll
            for (int k = 0; k < V; ++k)
                if (!(k & hb)) {
                    const double a = v[k], b = v[k + hb];
                    v[k] = a + b;
                    v[k + hb] = a - b;
                }
        }
    }
}

// the four waves' partial sums, added in wave order; every thread gets the total
__device__ double block_sum(double s, double* red) {
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    double t = red[0];
    for (int w = 1; w < kWaves; ++w) t += red[w];
    __syncthreads();
    return t;
}

// the norm's 1 / sqrt(mean(x^2) + eps) of row r (src/adjoint/host/elementwise.cpp:526-529)
__device__ double row_rs(const Args& a, int64_t r, double* red) {
    double ss = 0.0;
    for (int64_t j = threadIdx.x; j < a.n; j += kThreads) {
        const double x = ld(a.x0, a.dtype, r * a.n + j);
        ss += x * x;
    }
    return 1.0 / sqrt(block_sum(ss, red) / (double)a.n + a.eps);
}

// the part's output at column j of row r (elementwise.cpp:284-289, 322-324, 530-537)
template <int PART>
__device__ __forceinline__ double part_y(const Args& a, int64_t r, int64_t j, double rs) {
    if constexpr (PART == R97Q_PART_RMSNORM) {
        return ld(a.x0, a.dtype, r * a.n + j) * rs * (ld(a.x1, a.dtype, j) + a.wadd) * a.mult;
    } else if constexpr (PART == R97Q_PART_SILU_MUL) {
        const int64_t b = r * 2 * a.n + j;
        const double g = ld(a.x0, a.dtype, b);
        return g * sigm(g) * ld(a.x0, a.dtype, b + a.n);
    } else {
        const int64_t b = r * a.n + j;
        return sigm(ld(a.x0, a.dtype, b)) * ld(a.x1, a.dtype, b);
    }
}

// grid (rows): codes, scale and (when asked) the part's output rounded to f32 then bf16
template <int PART, int G>
__global__ __launch_bounds__(kThreads) void fused_fwd_kernel(Args a) {
    using Gm = Geo<G>;
    __shared__ double red[kWaves];
    const int64_t r = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const double rs = PART == R97Q_PART_RMSNORM ? row_rs(a, r, red) : 0.0;
    const int64_t n = a.n, ngrp = n / G, steps = (n + Gm::E - 1) / Gm::E;
    for (int64_t st = wave; st < steps; st += kWaves) {
        const int64_t e0 = st * Gm::E + lane;
        const bool valid = e0 < n;  // groups are whole: a lane's values are all in or all out
        double v[Gm::V];
#pragma unroll
        for (int k = 0; k < Gm::V; ++k) {
            v[k] = valid ? part_y<PART>(a, r, e0 + 64 * k, rs) : 0.0;
            if (valid && a.y_out) a.y_out[r * n + e0 + 64 * k] = f32_to_bf16((float)v[k]);
        }
        fwht<G>(v, lane);
        double m = 0.0;
#pragma unroll
        for (int k = 0; k < Gm::V; ++k) m = fabs(v[k]) > m ? fabs(v[k]) : m;
#pragma unroll
        for (int o = 1; o < Gm::L; o <<= 1) {
            const double other = __shfl_xor(m, o);
            m = other > m ? other : m;
        }
        const double s = m > 0.0 ? m * (1.0 / 127.0) : 1.0;  // quant.cpp:222-224
        const double inv = 1.0 / s;
        if (valid) {
#pragma unroll
            for (int k = 0; k < Gm::V; ++k) {
                const double c = rint(v[k] * inv);
                a.codes[r * n + e0 + 64 * k] = (int8_t)(c > 127.0 ? 127.0 : c < -127.0 ? -127.0 : c);
            }
            if (lane % Gm::L == 0) a.scale[r * ngrp + e0 / G] = (float)s;
        }
    }
}

// grid (rows): dx0 (and dx1 for the gate) += the composed adjoint. The norm takes two passes over
// its row: the first forms the shared term t = sum r_j x_j c_j, the second writes dx with it.
template <int PART, int G>
__global__ __launch_bounds__(kThreads) void fused_bwd_kernel(Args a) {
    using Gm = Geo<G>;
    __shared__ double red[kWaves];
    const int64_t r = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t n = a.n, ngrp = n / G, steps = (n + Gm::E - 1) / Gm::E;
    const double rs = PART == R97Q_PART_RMSNORM ? row_rs(a, r, red) : 0.0;
    double t = 0.0;
    constexpr int passes = PART == R97Q_PART_RMSNORM ? 2 : 1;
    for (int pass = 0; pass < passes; ++pass) {
        double tp = 0.0;
        for (int64_t st = wave; st < steps; st += kWaves) {
            const int64_t e0 = st * Gm::E + lane;
            const bool valid = e0 < n;
            double v[Gm::V], d[Gm::V];
#pragma unroll
            for (int k = 0; k < Gm::V; ++k) v[k] = valid ? part_y<PART>(a, r, e0 + 64 * k, rs) : 0.0;
            fwht<G>(v, lane);
            // the straight-through rule at the forward's scale (quant.cpp:349-368)
#pragma unroll
            for (int k = 0; k < Gm::V; ++k) {
                const int64_t e = e0 + 64 * k;
                d[k] = 0.0;
                if (valid) {
                    const double s = (double)a.scale[r * ngrp + e / G];
                    d[k] = fabs(v[k] * (1.0 / s)) > 127.0 ? 0.0 : (double)a.gc[r * n + e] / s;
                }
            }
            fwht<G>(d, lane);
            if (!valid) continue;
#pragma unroll
            for (int k = 0; k < Gm::V; ++k) {
                const int64_t j = e0 + 64 * k;
                const double rr = a.gout ? d[k] + (double)a.gout[r * n + j] : d[k];
                if constexpr (PART == R97Q_PART_RMSNORM) {
                    // elementwise.cpp:628-640
                    const double x = ld(a.x0, a.dtype, r * n + j), c = ld(a.x1, a.dtype, j) + a.wadd;
                    if (pass == 0) {
                        tp += rr * x * c;
                    } else {
                        const double shared = rs * rs * rs * x * t / (double)n;
                        float* o = a.dx0 + r * n + j;
                        *o = (float)((double)*o + a.mult * (rs * c * rr - shared));
                    }
                } else if constexpr (PART == R97Q_PART_SILU_MUL) {
                    // elementwise.cpp:305-311
                    const int64_t b = r * 2 * n + j;
                    const double g = ld(a.x0, a.dtype, b), u = ld(a.x0, a.dtype, b + n), sg = sigm(g);
                    a.dx0[b] = (float)((double)a.dx0[b] + rr * u * (sg * (1.0 + g * (1.0 - sg))));
                    a.dx0[b + n] = (float)((double)a.dx0[b + n] + rr * (g * sigm(g)));
                } else {
                    // elementwise.cpp:342-345
                    const int64_t b = r * n + j;
                    const double x = ld(a.x0, a.dtype, b), bv = ld(a.x1, a.dtype, b), sx = sigm(x);
                    a.dx0[b] = (float)((double)a.dx0[b] + rr * (sx * (1.0 - sx)) * bv);
                    a.dx1[b] = (float)((double)a.dx1[b] + rr * sigm(x));
                }
            }
        }
        if (PART == R97Q_PART_RMSNORM && pass == 0) t = block_sum(tp, red);
    }
}

template <int PART, int LG>
void launch_part(bool bwd, int64_t rows, const Args& a, hipStream_t s) {
    if constexpr (LG > kMaxLogGroup) {
        return;
    } else {
        if (bwd)
            hipLaunchKernelGGL((fused_bwd_kernel<PART, 1 << LG>), dim3((unsigned)rows), dim3(kThreads), 0, s, a);
        else
            hipLaunchKernelGGL((fused_fwd_kernel<PART, 1 << LG>), dim3((unsigned)rows), dim3(kThreads), 0, s, a);
    }
}

template <int PART, int LG = 0>
void dispatch_group(int lg, bool bwd, int64_t rows, const Args& a, hipStream_t s) {
    if constexpr (LG <= kMaxLogGroup) {
        if (lg == LG) return launch_part<PART, LG>(bwd, rows, a, s);
        dispatch_group<PART, LG + 1>(lg, bwd, rows, a, s);
    }
}

const char* part_name(int32_t part) {
    return part == R97Q_PART_RMSNORM ? "rmsnorm_had_quant_i8g"
           : part == R97Q_PART_SILU_MUL ? "gated_had_quant_i8g"
                                        : "gate_had_quant_i8g";
}

// the record rules the reference's rows apply (quant.hip:129-159, the group; elementwise.cpp, the
// parts' operands): 0 and log2(group) in *lg, or an error code with the message set
int check_args(int32_t part, const void* x0, const void* x1, int32_t dtype, int64_t rows, int64_t n, int64_t group,
               const char* who, int* lg) {
    if (part < R97Q_PART_RMSNORM || part > R97Q_PART_SIGMOID_MUL) {
        set_error("fused quantiser: part %d is not rmsnorm (0), silu_mul (1) or sigmoid_mul (2)", (int)part);
        return R97Q_EINVAL;
    }
    if (!x0 || (part != R97Q_PART_SILU_MUL && !x1)) {
        set_error("%s: null %s", who, !x0 ? "first input" : part == R97Q_PART_RMSNORM ? "gain" : "second input");
        return R97Q_EINVAL;
    }
    if (dtype != R97Q_BF16 && dtype != R97Q_F32 && dtype != R97Q_F64) {
        set_error("%s: the inputs are bf16, f32 or f64", who);
        return R97Q_EINVAL;
    }
    if (rows <= 0 || n <= 0) {
        set_error("%s: rows and n must be positive", who);
        return R97Q_EINVAL;
    }
    if (group <= 0 || (group & (group - 1)) != 0 || n % group != 0) {
        set_error("%s: 'group' must be a power of two that divides 'n' (n=%lld group=%lld)", who, (long long)n,
                  (long long)group);
        return R97Q_EINVAL;
    }
    if (group > (1 << kMaxLogGroup)) {
        set_error("%s: a group of %lld is wider than the rows serve (%d)", who, (long long)group, 1 << kMaxLogGroup);
        return R97Q_EUNSUPPORTED;
    }
    if (rows > 0x7fffffffLL) {
        set_error("%s: %lld rows; at most 2^31 - 1 a call", who, (long long)rows);
        return R97Q_EUNSUPPORTED;
    }
    *lg = 0;
    while ((1LL << *lg) < group) ++*lg;
    return R97Q_OK;
}

void launch(int32_t part, int lg, bool bwd, int64_t rows, const Args& a, hipStream_t s) {
    if (part == R97Q_PART_RMSNORM) dispatch_group<R97Q_PART_RMSNORM>(lg, bwd, rows, a, s);
    else if (part == R97Q_PART_SILU_MUL) dispatch_group<R97Q_PART_SILU_MUL>(lg, bwd, rows, a, s);
    else dispatch_group<R97Q_PART_SIGMOID_MUL>(lg, bwd, rows, a, s);
}

}  // namespace
}  // namespace r97q

using namespace r97q;

extern "C" {

int r97q_fused_had_quant_i8g(int32_t part, const void* x0, const void* x1, int32_t x_dtype, int64_t rows, int64_t n,
                             int64_t group, double eps, double wadd, double mult, int8_t* codes, float* scale,
                             uint16_t* y_out, R97IqrStream stream) {
    clear_error();
    int lg = 0;
    const char* who = part_name(part);
    if (int e = check_args(part, x0, x1, x_dtype, rows, n, group, who, &lg)) return e;
    if (!codes || !scale) {
        set_error("%s: null codes or scale", who);
        return R97Q_EINVAL;
    }
    Args a{x0, x1, x_dtype, n, eps, wadd, mult, codes, scale, y_out, nullptr, nullptr, nullptr, nullptr};
    launch(part, lg, false, rows, a, (hipStream_t)stream);
    return launch_status("fused_fwd_kernel");
}

int r97q_fused_had_quant_i8g_bwd(int32_t part, const void* x0, const void* x1, int32_t x_dtype, int64_t rows,
                                 int64_t n, int64_t group, double eps, double wadd, double mult, const float* scale,
                                 const float* g_codes, const float* g_out, float* dx0, float* dx1,
                                 R97IqrStream stream) {
    clear_error();
    int lg = 0;
    const char* who = part_name(part);
    if (int e = check_args(part, x0, x1, x_dtype, rows, n, group, who, &lg)) return e;
    if (!scale || !g_codes || !dx0 || (part == R97Q_PART_SIGMOID_MUL && !dx1)) {
        set_error("%s adjoint: null scale, codes' cotangent or %s", who, !dx0 ? "dx0" : "dx1");
        return R97Q_EINVAL;
    }
    Args a{x0, x1, x_dtype, n, eps, wadd, mult, nullptr, const_cast<float*>(scale), nullptr, g_codes, g_out, dx0,
           dx1};
    launch(part, lg, true, rows, a, (hipStream_t)stream);
    return launch_status("fused_bwd_kernel");
}

}  // extern "C"
