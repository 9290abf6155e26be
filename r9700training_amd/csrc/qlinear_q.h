// qlinear_q.h -- the coded product's forward kernel (qlinear_q.hip): gemm_nt_q's twin over int8
// activation codes and the weight's int8-code form.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace r97q {
namespace q {

constexpr int kBM = 256;     // tokens a workgroup
constexpr int kBN = 128;     // outputs a workgroup
constexpr int kGroup = 128;  // columns a scale group (a step)

struct Params {
    const int8_t* act;         // the token codes' tiled copy (qtok_tile_kernel), ldt rows
    const float* sa_t;         // a_scale transposed, [K/128][ldt] f32
    int64_t T, N, K;           // the weight is [N, K]
    int64_t ldt;               // T rounded up to kBM
    const uint8_t* units;      // the weight's int8-code form: [N/8][K/4] units of 8 rows x 4 columns
    const uint16_t* scale_t;   // [K/128][N] bf16
    void* out;                 // Y [T, N], f32 or bf16
    int out_f32;
    int mtiles, otiles;
};

int64_t tok_ld(int64_t T);                 // T rounded up to kBM
int64_t tok_tile_bytes(int64_t T, int64_t K);  // the tiled copy's bytes
// the tiled copy of a [T, K] int8 and a_scale [T, K/128] f32 transposed into sa_t [K/128][ldt]
int launch_tokens(const int8_t* a, const float* a_scale, int64_t T, int64_t K, int8_t* dst, float* sa_t,
                  hipStream_t s);
int launch_forward(const Params& p, hipStream_t s);

}  // namespace q
}  // namespace r97q
