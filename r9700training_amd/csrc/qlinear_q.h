// qlinear_q.h -- the coded product's forward kernel (qlinear_q.hip): gemm_nt_q's twin over int8
// activation codes and the stored weight's int8 code grid.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace r97q {
namespace q {

constexpr int kBM = 256;     // tokens a workgroup
constexpr int kBN = 128;     // outputs a workgroup
constexpr int kGroup = 128;  // columns a scale group (a step)

struct Params {
    const int8_t* a;           // the activation codes [T, K] int8, row-major
    const float* a_scale;      // [T, K/128] f32
    const int8_t* codes;       // the weight's codes [N, K] int8, row-major
    const uint16_t* scale;     // the weight's scales [N, K/128] bf16
    int64_t T, N, K;
    void* out;                 // Y [T, N], f32 or bf16
    int out_f32;
    int mtiles, otiles;
};

int launch_forward(const Params& p, hipStream_t s);

}  // namespace q
}  // namespace r97q
