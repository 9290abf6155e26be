// qlinear_q.hip -- the coded (i8a8h) product's forward on CDNA4 (gfx950): gemm_nt_q's twin
// (src/adjoint/host/linear.cpp:245-282),
//
//   Y[m, n] = sum_g ( sum_{k in g} a[m, k] * code[n, k] ) * a_scale[m, g] * scale[n, g]
//
// over int8 activation codes a [T, K] (row-major) with their f32 group scales a_scale [T, K/128]
// and the stored weight's two grids as the reference keeps them (src/stored_weight.h:24-33): int8
// codes [N, K] row-major and bf16 scales [N, K/128]. The group sums are exact: the int8 MFMA
// (v_mfma_i32_32x32x32_i8) accumulates each 128-column group in int32; one f32 fold a group
// (convert, scale product, fma) adds it into the f32 accumulator, as the reference's f64 loop adds
// `sub`.
//
// Shape of a launch. A workgroup owns a 256-token x 128-output tile: 8 waves, wave w the 64 tokens
// 64*(w%4).. and the 64 outputs 64*(w/4).. (2 x 2 tiles of 32 x 32). The reduction walks one group
// (128 columns) a step through a three-stage LDS ring: every operand of a step -- the 256 token
// rows' 128 code bytes, the 128 weight rows' 128 code bytes, the 256 activation scales and the 128
// weight scales -- streams global -> LDS with direct loads (global_load_lds, no registers; a
// 16-byte load's 8 lanes cover a 128-byte row, the XOR chunk swizzle chosen by the address each
// lane reads), two steps ahead. Each wave reads its token and weight fragments back from the
// step's stage; per 32 x 32 tile the four 32-deep MFMAs of the group run as one int32 chain, then
// the tile is folded into f32. One barrier a step: after it the stage of the step after next is
// free to refill and the next step's stage is complete.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "iqr_device.h"
#include "qlinear_q.h"
#include "status.h"

namespace r97q {
namespace q {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((__vector_size__(64)));
typedef __attribute__((address_space(3))) void lds_void;

// one stage of the ring: token rows [256][128] | weight rows [128][128] | a_scale [256] f32 |
// scale [128] (the aligned dword holding each output's bf16) | a pad the two waves without a
// scale to load fill, so that every wave issues the same number of loads a step. A direct load of
// 4 bytes or fewer puts lane i's data at 4i.
constexpr int kTokOff = 0;
constexpr int kWOff = kBM * kGroup;
constexpr int kSaOff = kWOff + kBN * kGroup;
constexpr int kSbOff = kSaOff + kBM * 4;
constexpr int kPadOff = kSbOff + kBN * 4;
constexpr int kStageBytes = kPadOff + 2 * 256;
constexpr int kStages = 3;
static_assert(kStages * kStageBytes <= 160 * 1024, "the ring fits a gfx950 CU's LDS");

__device__ __forceinline__ i32x16 mfma_i8(i32x4 a, i32x4 b, i32x16 c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ i32x4 as_i32x4(uint4 v) { return __builtin_bit_cast(i32x4, v); }

// XOR swizzle of a 128-byte LDS row's eight 16-byte chunks: 16 consecutive rows reading one
// logical chunk land on 16 distinct 16-byte bank groups.
__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

__device__ __forceinline__ int chunk_off(int row, int chunk) { return row * 128 + ((chunk ^ swz(row)) << 4); }

// consecutive workgroup ids are dealt round-robin over the 8 XCDs; renumber so each XCD's
// workgroups take one contiguous run of tiles (tokens outer, outputs inner)
__device__ __forceinline__ int xcd_tile(int bid, int nwg) {
    const int xcd = bid & 7, local = bid >> 3;
    const int base = nwg >> 3, rem = nwg & 7;
    return xcd * base + (xcd < rem ? xcd : rem) + local;
}

template <int SIZE>
__device__ __forceinline__ void to_lds(const void* src, uint8_t* dst) {
    if constexpr (SIZE == 16) __builtin_amdgcn_global_load_lds(src, (lds_void*)dst, 16, 0, 0);
    else __builtin_amdgcn_global_load_lds(src, (lds_void*)dst, 4, 0, 0);
}

__global__ __launch_bounds__(512, 1) void qlinear_q_kernel(const Params p) {
    // the ring's stages as separate arrays, and a loop unrolled by three so every step reads one
    // array and fills another by name: the compiler then sees that the direct loads in flight do
    // not write the stage a wave reads, and waits for them only where the barrier protocol says
    __shared__ __attribute__((aligned(16))) uint8_t st0[kStageBytes], st1[kStageBytes], st2[kStageBytes];
    const int tile = xcd_tile(blockIdx.x, p.mtiles * p.otiles);
    const int mt = tile / p.otiles, ot = tile % p.otiles;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int half = lane >> 5, l32 = lane & 31;
    const int wm = wave & 3, wn = wave >> 2;
    const int64_t mw = (int64_t)mt * kBM;  // the workgroup's first token
    const int64_t o0 = (int64_t)ot * kBN;  // the workgroup's first output
    const int64_t K = p.K, G = K / kGroup;
    const int nsteps = (int)G;

    // The loads of one step, issued by every wave (seven a wave): 4 x 1 KiB of token rows (rows
    // 32w + 8q + lane/8, q < 4) and 2 x 1 KiB of weight rows (rows 16w + 8q + lane/8, q < 2) --
    // lane i takes the logical chunk (i%8) ^ swz(row) of its row, so LDS holds the rows swizzled;
    // then waves 0-3 the a_scale of rows 64w + lane, waves 4-5 the aligned dword holding the bf16
    // scale of outputs 64(w-4) + lane, and waves 6-7 the a_scale of wave 0's rows again into the
    // pad (4 bytes a lane each). Rows past T read row T-1 (their products land in rows never
    // stored).
    const int lr = lane >> 3, lc = lane & 7;
    const int8_t* tsrc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int r = 32 * wave + 8 * q + lr;
        int64_t m = mw + r;
        if (m > p.T - 1) m = p.T - 1;
        tsrc[q] = p.a + m * K + 16 * (lc ^ swz(r));
    }
    const int8_t* wsrc[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int r = 16 * wave + 8 * q + lr;
        wsrc[q] = p.codes + (o0 + r) * K + 16 * (lc ^ swz(r));
    }
    const float* sasrc = p.a_scale;
    int64_t sbi = 0;  // waves 4-5: the lane's output's first scale element, n * G
    if (wave < 4 || wave >= 6) {
        int64_t m = mw + 64 * (wave < 4 ? wave : 0) + lane;
        if (m > p.T - 1) m = p.T - 1;
        sasrc = p.a_scale + m * G;
    } else {
        sbi = (o0 + 64 * (wave - 4) + lane) * G;
    }
    auto issue = [&](int s, uint8_t* st) {
        if (s > nsteps - 1) s = nsteps - 1;  // past the walk: the last step again, into a stage never read
#pragma unroll
        for (int q = 0; q < 4; ++q) to_lds<16>(tsrc[q] + (int64_t)s * kGroup, st + kTokOff + (32 * wave + 8 * q) * 128);
#pragma unroll
        for (int q = 0; q < 2; ++q) to_lds<16>(wsrc[q] + (int64_t)s * kGroup, st + kWOff + (16 * wave + 8 * q) * 128);
        if (wave < 4) to_lds<4>(sasrc + s, st + kSaOff + 256 * wave);
        else if (wave < 6) to_lds<4>(p.scale + ((sbi + s) & ~(int64_t)1), st + kSbOff + 256 * (wave - 4));
        else to_lds<4>(sasrc + s, st + kPadOff + 256 * (wave - 6));
    };
    // this wave's loads of the next step landed (those of the step after stay in flight), then the
    // workgroup barrier: every wave's loads of the next step are in LDS, and every wave is done
    // reading the stage the step after next refills
    auto step_end = [&]() {
        __builtin_amdgcn_s_waitcnt(0x0F77);  // vmcnt(7): one step's seven loads outstanding
        __builtin_amdgcn_s_barrier();
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = (f32x16){};

    // step s: the loads of step s+2 into `fill`, the MFMAs of step s from `st`. The four tiles
    // (mi, ni) in the order (0,0) (1,0) (0,1) (1,1): each tile's int32 chain is issued before the
    // previous tile's f32 fold, so the fold's VALU runs under the next chain's MFMAs.
    auto step = [&](int s, const uint8_t* st, uint8_t* fill) {
        issue(s + 2, fill);
        // the wave's token fragments: block mi, slice j (columns 32j + 16*half ..); its weight
        // fragments of output blocks 0 and 1
        uint4 tk[2][4], wf[2][4];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                tk[mi][j] = *reinterpret_cast<const uint4*>(st + kTokOff + chunk_off(64 * wm + 32 * mi + l32, 2 * j + half));
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                wf[ni][j] = *reinterpret_cast<const uint4*>(st + kWOff + chunk_off(64 * wn + 32 * ni + l32, 2 * j + half));
        // the weight scale of the lane's column of each output block: the half of its dword that
        // (n*G + s) picks
        float sb[2];
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const int nl = 64 * wn + 32 * ni + l32;
            const uint32_t w = *reinterpret_cast<const uint32_t*>(st + kSbOff + 4 * nl);
            sb[ni] = bf16_to_f32((uint16_t)(((o0 + nl) * G + s) & 1 ? w >> 16 : w));
        }
        // a_scale of the lane's 16 rows of each token block: four runs of four consecutive rows,
        // 32mi + 8q + 4*half + 0..3
        float4 sa[2][4];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                sa[mi][q] = *reinterpret_cast<const float4*>(st + kSaOff + 4 * (64 * wm + 32 * mi + 8 * q + 4 * half));
        auto chain = [&](int mi, int ni) {
            i32x16 g = mfma_i8(as_i32x4(tk[mi][0]), as_i32x4(wf[ni][0]), (i32x16){});
#pragma unroll
            for (int j = 1; j < 4; ++j) g = mfma_i8(as_i32x4(tk[mi][j]), as_i32x4(wf[ni][j]), g);
            return g;
        };
        // the f32 fold of tile (mi, ni)
        auto fold = [&](int mi, int ni, const i32x16& g) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float r[4] = {sa[mi][q].x, sa[mi][q].y, sa[mi][q].z, sa[mi][q].w};
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    acc[mi][ni][4 * q + u] = __builtin_fmaf((float)g[4 * q + u], r[u] * sb[ni], acc[mi][ni][4 * q + u]);
            }
        };
        // the fold's 48 VALU operations spread over the next chain's 4 MFMAs
        auto overlap = []() {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 12, 0);  // VALU
            }
        };
        const i32x16 g00 = chain(0, 0);
        __builtin_amdgcn_sched_barrier(0);
        const i32x16 g10 = chain(1, 0);
        fold(0, 0, g00);
        overlap();
        __builtin_amdgcn_sched_barrier(0);
        const i32x16 g01 = chain(0, 1);
        fold(1, 0, g10);
        overlap();
        __builtin_amdgcn_sched_barrier(0);
        const i32x16 g11 = chain(1, 1);
        fold(0, 1, g01);
        overlap();
        __builtin_amdgcn_sched_barrier(0);
        fold(1, 1, g11);
        step_end();
    };

    issue(0, st0);
    issue(1, st1);
    step_end();
    for (int s = 0; s < nsteps; s += 3) {
        step(s, st0, st2);
        if (s + 1 >= nsteps) break;
        step(s + 1, st1, st0);
        if (s + 2 >= nsteps) break;
        step(s + 2, st2, st1);
    }

    // accumulator element e of tile (mi, ni) is row 32*mi + 8*(e/4) + 4*half + e%4, column 32*ni + l32
    const int64_t m0 = mw + 64 * wm;
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int64_t row = m0 + 32 * mi + 8 * (e >> 2) + 4 * half + (e & 3);
            if (row >= p.T) continue;
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                const int64_t col = o0 + 64 * wn + 32 * ni + l32;
                if (p.out_f32)
                    reinterpret_cast<float*>(p.out)[row * p.N + col] = acc[mi][ni][e];
                else
                    reinterpret_cast<uint16_t*>(p.out)[row * p.N + col] = f32_to_bf16(acc[mi][ni][e]);
            }
        }
}

}  // namespace

int launch_forward(const Params& p, hipStream_t s) {
    hipLaunchKernelGGL(qlinear_q_kernel, dim3((unsigned)(p.mtiles * p.otiles)), dim3(512), 0, s, p);
    return launch_status("qlinear_q_kernel");
}

}  // namespace q
}  // namespace r97q
