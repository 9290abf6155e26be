// qlinear_fused.h -- parameters and launchers of the fused IQR-decode + MFMA kernels
// (qlinear_fused.hip, compiled once per code width with -DR97Q_BITS=3..6).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace r97q {

constexpr int kBM = 512;      // tokens per workgroup
constexpr int kWaveM = 64;    // tokens per wave
constexpr int kBN = 128;      // output features (fwd) / output columns (dX) per workgroup
constexpr int kStep = 64;     // reduction depth per main-loop step
constexpr int kThreads = 512;

struct FwdParams {
    const uint16_t* X;
    int64_t T, N, K;
    const uint32_t* stream;
    const uint16_t* scale_t;
    uint32_t a24, b;
    int64_t run_rows;
    const uint16_t* P;  // [T, 2r] bf16: hi | lo of s.t
    const uint16_t* B;  // [N, r] bf16
    int rank;
    void* Y;
    int y_f32;
    int mtiles, ntiles;
};

struct DxParams {
    const uint16_t* dY;
    int64_t T, N, K;
    const uint32_t* stream;
    const uint16_t* scale_t;
    uint32_t a24, b;
    int64_t run_rows;
    const uint16_t* P;   // [T, 2r] bf16: hi | lo of dt
    const uint16_t* At;  // [K, r] bf16
    int rank;
    void* dX;
    int dx_f32;
    int accumulate;
    const float* a_scale;  // null, or f32 [T, a_scale_ld]: dX[m, k] is multiplied by a_scale[m, k/128]
    int64_t a_scale_ld;
    int mtiles, ktiles;
};

template <int BITS>
void launch_fwd(const FwdParams& p, hipStream_t s);
template <int BITS>
void launch_dx(const DxParams& p, hipStream_t s);

}  // namespace r97q
