// probe.hip -- the measured ceiling the base products are judged against on this card: sustained
// v_mfma_f32_32x32x16_bf16 issue with nothing else to do. Every wave of 256 workgroups x 8 waves
// (one workgroup a CU, two waves a SIMD: the fused kernels' shape) keeps eight independent
// accumulators busy with operands already in registers, so the matrix cores never wait for memory;
// the operands are random bf16 values (the power a real product draws) or zeros (the clock the card
// holds when the datapath barely toggles). Not part of any product path.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/r97q.h"
#include "status.h"

namespace {

typedef __bf16 bf16x8 __attribute__((__vector_size__(16)));
typedef float f32x16 __attribute__((__vector_size__(64)));

__device__ __forceinline__ uint32_t mix(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7FEB352Du;
    x ^= x >> 15;
    x *= 0x846CA68Bu;
    x ^= x >> 16;
    return x;
}

// a bf16 of magnitude 2^-7 .. 2^3 with a random sign and mantissa, or zero
__device__ __forceinline__ uint32_t operand_pair(uint32_t h, int zero) {
    if (zero) return 0u;
    const uint32_t lo = (h & 0x807Fu) | ((120u + (h >> 8) % 10u) << 7);
    const uint32_t g = mix(h);
    const uint32_t hi = (g & 0x807Fu) | ((120u + (g >> 8) % 10u) << 7);
    return lo | (hi << 16);
}

__global__ __launch_bounds__(512, 1) void mfma_probe_kernel(int iters, int zero, float* out) {
    const int lane = threadIdx.x & 63;
    uint4 a[4], b[8];
    uint32_t h = mix(blockIdx.x * 512u + threadIdx.x + 1u);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = uint4{operand_pair(h = mix(h), zero), operand_pair(h = mix(h), zero), operand_pair(h = mix(h), zero),
                     operand_pair(h = mix(h), zero)};
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        b[i] = uint4{operand_pair(h = mix(h), zero), operand_pair(h = mix(h), zero), operand_pair(h = mix(h), zero),
                     operand_pair(h = mix(h), zero)};
    }
    f32x16 acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = (f32x16){};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i)
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[(i >> 2) + 2 * (j & 1)]),
                                                                 __builtin_bit_cast(bf16x8, b[(i & 3) + 4 * (j >> 1)]),
                                                                 acc[i], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) s += acc[i][lane & 15];
    out[blockIdx.x * 512 + threadIdx.x] = s;
}

}  // namespace

extern "C" int64_t r97q_mfma_probe_flops(int32_t iters) {
    return (int64_t)2 * 32 * 32 * 16 * 32 * iters * 8 * 256;
}

extern "C" int r97q_mfma_probe(int32_t iters, int32_t zero_operands, float* out, int64_t out_count,
                               R97IqrStream stream) {
    r97q::clear_error();
    if (iters <= 0 || !out || out_count < (int64_t)256 * 512) {
        r97q::set_error("r97q_mfma_probe: iters %d, out_count %lld (iters > 0 and an out buffer of at least 256 * 512 "
                        "floats)", (int)iters, (long long)out_count);
        return R97Q_EINVAL;
    }
    hipLaunchKernelGGL(mfma_probe_kernel, dim3(256), dim3(512), 0, (hipStream_t)stream, (int)iters,
                       (int)(zero_operands != 0), out);
    return r97q::launch_status("mfma_probe_kernel");
}
