// qlinear_q.hip -- the coded (i8a8h) product's forward on CDNA4 (gfx950): gemm_nt_q's twin
// (src/adjoint/host/linear.cpp:245-282),
//
//   Y[m, n] = sum_g ( sum_{k in g} a[m, k] * code[n, k] ) * a_scale[m, g] * scale[n, g]
//
// over int8 activation codes a [T, K] with their f32 group scales a_scale [T, K/128] and the
// weight's int8-code form (code [N, K] int8 in 8 x 4 units, bf16 scale [K/128, N]). The group
// sums are exact: v_mfma_i32_32x32x32_i8 accumulates each 128-column group in int32; one f32
// rescale a group (convert, scale product, fma) folds it into the f32 accumulator, as the
// reference's f64 loop folds `sub`.
//
// Shape of a launch. A workgroup owns a 256-token x 128-output tile: 8 waves, wave w the 64 tokens
// 64*(w%4).. and the 64 outputs 64*(w/4).. (2 x 2 tiles of 32 x 32). The reduction walks one group
// (128 columns) a step:
//   * the token codes come straight into registers from their tiled copy (qtok_tile_kernel: every
//     32-row x 32-column fragment one coalesced 1 KiB load), one step ahead;
//   * the step's weight tile (128 outputs x 128 columns int8, 16 KiB) is read from the int8-code
//     form by all 512 lanes (one 32-byte unit each, rows regrouped with v_perm) into one half of a
//     double-buffered, XOR-swizzled LDS tile, one step ahead; each wave reads its 64 rows back as
//     MFMA fragments;
//   * the step's scales (the workgroup's 256 a_scale values, its 128 weight scales) go through a
//     double-buffered LDS slot the same way, one step ahead;
//   * per 32 x 32 tile the four 32-deep MFMAs of the group run as one int32 chain, then the tile
//     is rescaled into f32 while the next tile's chain runs;
//   * one barrier a step.
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

constexpr int kTileBytes = kBN * kGroup;  // one int8 weight tile: 128 rows x 128 bytes

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

// this wave's LDS accesses done, then the workgroup barrier (vector-memory loads not waited for)
__device__ __forceinline__ void tile_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
}

// ---------------------------------------------------------------- the token operand's copy
// dst: fragment (s, rb, j) -- group s, 32-row block rb, 32-column slice j -- is 1 KiB at
// ((s * nrb + rb) * 4 + j) * 1024, lane l's 16 bytes (row 32rb + l%32, columns 128s + 32j +
// 16(l/32) ..) at 16l; nrb = ldt / 32 and rows past T are zero. sa_t [G][ldt] = a_scale
// transposed (zero past T). One workgroup a (group, row block): thread t reads row t/8's 16-byte
// chunk t%8.
__global__ __launch_bounds__(256) void qtok_tile_kernel(const int8_t* __restrict__ a, const float* __restrict__ sa,
                                                        int64_t T, int64_t K, int8_t* __restrict__ dst,
                                                        float* __restrict__ sa_t) {
    const int64_t s = blockIdx.x, rb = blockIdx.y, nrb = gridDim.y;
    const int i = threadIdx.x >> 3, c = threadIdx.x & 7;
    const int64_t m = 32 * rb + i;
    uint4 v = {0u, 0u, 0u, 0u};
    if (m < T) v = *reinterpret_cast<const uint4*>(a + m * K + 128 * s + 16 * c);
    const int64_t frag = (s * nrb + rb) * 4 + (c >> 1);
    *reinterpret_cast<uint4*>(dst + frag * 1024 + (32 * (c & 1) + i) * 16) = v;
    if (threadIdx.x < 32) {  // thread t: row 32rb + t's scale of group s
        const int64_t G = K / kGroup, r = 32 * rb + threadIdx.x;
        sa_t[s * (nrb * 32) + r] = r < T ? sa[r * G + s] : 0.0f;
    }
}

// ---------------------------------------------------------------- the product
template <int WAVES>
struct Geo {
    static_assert(WAVES == 8, "8 waves: 4 token groups x 2 output halves");
    static constexpr int kMI = 2;  // 32-token blocks a wave
    static constexpr int kNI = 2;  // 32-output blocks a wave
};

__global__ __launch_bounds__(512, 1) void qlinear_q_kernel(const Params p) {
    constexpr int kMI = Geo<8>::kMI, kNI = Geo<8>::kNI;
    // two weight tiles, then two scale slots (the step's 256 a_scale values and 128 weight scales, f32)
    constexpr int kScaleBytes = (kBM + kBN) * 4;
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kTileBytes + 2 * kScaleBytes];
    const int tile = xcd_tile(blockIdx.x, p.mtiles * p.otiles);
    const int mt = tile / p.otiles, ot = tile % p.otiles;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int half = lane >> 5, l32 = lane & 31;
    const int wm = wave & 3, wn = wave >> 2;
    const int64_t mw = (int64_t)mt * kBM;      // the workgroup's first token
    const int64_t m0 = mw + 64 * wm;           // the wave's first token
    const int64_t o0 = (int64_t)ot * kBN;      // the workgroup's first output
    const int nsteps = (int)(p.K / kGroup);
    const int64_t nrb = p.ldt / 32;  // the copy covers every workgroup's rows (ldt = mtiles * kBM)

    const int8_t* tok[kMI];
#pragma unroll
    for (int mi = 0; mi < kMI; ++mi) tok[mi] = p.act + ((m0 >> 5) + mi) * 4 * 1024 + lane * 16;
    const int64_t tok_step = nrb * 4 * 1024;
    auto load_tokens = [&](int s, uint4 (&t)[kMI][4]) {
#pragma unroll
        for (int mi = 0; mi < kMI; ++mi)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                t[mi][j] = *reinterpret_cast<const uint4*>(tok[mi] + (int64_t)s * tok_step + j * 1024);
    };

    // the weight tile's fill: thread t takes the 8 x 4 unit (rows 8(t/32).., columns 4(t%32)..)
    const int r8 = threadIdx.x >> 5, c4 = threadIdx.x & 31;
    const uint8_t* unit = p.units + (((o0 >> 3) + r8) * (p.K >> 2) + c4) * 32;
    auto fill_load = [&](int s, uint4 (&u)[2]) {
        const uint8_t* src = unit + (int64_t)s * (kGroup / 4) * 32;
        u[0] = *reinterpret_cast<const uint4*>(src);
        u[1] = *reinterpret_cast<const uint4*>(src + 16);
    };
    // unit byte 16*(c/2) + 2i + c%2 is row i, column c: row i's four columns are bytes 2i, 2i+1 of
    // the first half and of the second half
    auto fill_store = [&](uint8_t* t, const uint4 (&u)[2]) {
        const uint32_t lo[4] = {u[0].x, u[0].y, u[0].z, u[0].w};
        const uint32_t hi[4] = {u[1].x, u[1].y, u[1].z, u[1].w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t v = __builtin_amdgcn_perm(hi[i >> 1], lo[i >> 1], (i & 1) ? 0x07060302u : 0x05040100u);
            const int row = 8 * r8 + i;
            *reinterpret_cast<uint32_t*>(t + chunk_off(row, c4 >> 2) + 4 * (c4 & 3)) = v;
        }
    };
    // the step's scales: wave 0 loads the workgroup's 256 a_scale values (four a lane), lanes 0-31
    // of wave 1 its 128 weight scales (four bf16 a lane, widened to f32)
    auto scales_load = [&](int s, float4& v) {
        if (wave == 0) {
            v = *reinterpret_cast<const float4*>(p.sa_t + (int64_t)s * p.ldt + mw + 4 * lane);
        } else if (wave == 1 && lane < 32) {
            const uint2 b = *reinterpret_cast<const uint2*>(p.scale_t + (int64_t)s * p.N + o0 + 4 * lane);
            v = make_float4(bf16_to_f32((uint16_t)b.x), bf16_to_f32((uint16_t)(b.x >> 16)),
                            bf16_to_f32((uint16_t)b.y), bf16_to_f32((uint16_t)(b.y >> 16)));
        }
    };
    auto scales_store = [&](uint8_t* slot, const float4& v) {
        if (wave == 0) *reinterpret_cast<float4*>(slot + 16 * lane) = v;
        else if (wave == 1 && lane < 32) *reinterpret_cast<float4*>(slot + kBM * 4 + 16 * lane) = v;
    };
    // the wave's weight fragments of output block ni of a tile, slice j (columns 32j + 16*half ..)
    auto read_w = [&](const uint8_t* t, int ni, uint4 (&w)[4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            w[j] = *reinterpret_cast<const uint4*>(t + chunk_off(64 * wn + 32 * ni + l32, 2 * j + half));
    };

    f32x16 acc[kMI][kNI];
#pragma unroll
    for (int mi = 0; mi < kMI; ++mi)
#pragma unroll
        for (int ni = 0; ni < kNI; ++ni) acc[mi][ni] = (f32x16){};

    uint8_t* const slots = lds + 2 * kTileBytes;
    uint4 tk[kMI][4], tn[kMI][4], wf[4], fu[2];
    float4 sv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    fill_load(0, fu);
    load_tokens(0, tk);
    scales_load(0, sv);
    fill_store(lds, fu);
    scales_store(slots, sv);
    tile_barrier();
    for (int s = 0; s < nsteps; ++s) {
        const uint8_t* cur = lds + (s & 1) * kTileBytes;
        uint8_t* nxt = lds + ((s + 1) & 1) * kTileBytes;
        const uint8_t* scur = slots + (s & 1) * kScaleBytes;
        uint8_t* snxt = slots + ((s + 1) & 1) * kScaleBytes;
        const int sn = s + 1 < nsteps ? s + 1 : s;
        fill_load(sn, fu);
        load_tokens(sn, tn);
        scales_load(sn, sv);
#pragma unroll
        for (int ni = 0; ni < kNI; ++ni) {
            read_w(cur, ni, wf);
            i32x16 g[kMI];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int mi = 0; mi < kMI; ++mi)
                    g[mi] = mfma_i8(as_i32x4(tk[mi][j]), as_i32x4(wf[j]), j == 0 ? (i32x16){} : g[mi]);
            // the weight scale of the lane's column of block ni; a_scale of its 16 rows of token
            // block mi (four runs of four consecutive rows: 32mi + 8q + 4*half + 0..3)
            const float sb = *reinterpret_cast<const float*>(scur + kBM * 4 + 4 * (64 * wn + 32 * ni + l32));
#pragma unroll
            for (int mi = 0; mi < kMI; ++mi)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 v =
                        *reinterpret_cast<const float4*>(scur + 4 * (64 * wm + 32 * mi + 8 * q + 4 * half));
                    const float sa[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        acc[mi][ni][4 * q + u] =
                            __builtin_fmaf((float)g[mi][4 * q + u], sa[u] * sb, acc[mi][ni][4 * q + u]);
                }
        }
        fill_store(nxt, fu);
        scales_store(snxt, sv);
#pragma unroll
        for (int mi = 0; mi < kMI; ++mi)
#pragma unroll
            for (int j = 0; j < 4; ++j) tk[mi][j] = tn[mi][j];
        tile_barrier();
    }

    // accumulator element e of tile (mi, ni) is row 32*mi + 8*(e/4) + 4*half + e%4, column 32*ni + l32
#pragma unroll
    for (int mi = 0; mi < kMI; ++mi)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int64_t row = m0 + 32 * mi + 8 * (e >> 2) + 4 * half + (e & 3);
            if (row >= p.T) continue;
#pragma unroll
            for (int ni = 0; ni < kNI; ++ni) {
                const int64_t col = o0 + 64 * wn + 32 * ni + l32;
                if (p.out_f32)
                    reinterpret_cast<float*>(p.out)[row * p.N + col] = acc[mi][ni][e];
                else
                    reinterpret_cast<uint16_t*>(p.out)[row * p.N + col] = f32_to_bf16(acc[mi][ni][e]);
            }
        }
}

}  // namespace

int64_t tok_ld(int64_t T) { return (T + kBM - 1) / kBM * kBM; }

int64_t tok_tile_bytes(int64_t T, int64_t K) { return tok_ld(T) * K; }

int launch_tokens(const int8_t* a, const float* a_scale, int64_t T, int64_t K, int8_t* dst, float* sa_t,
                  hipStream_t s) {
    hipLaunchKernelGGL(qtok_tile_kernel, dim3((unsigned)(K / kGroup), (unsigned)(tok_ld(T) / 32)), dim3(256), 0, s, a,
                       a_scale, T, K, dst, sa_t);
    return launch_status("qtok_tile_kernel");
}

int launch_forward(const Params& p, hipStream_t s) {
    hipLaunchKernelGGL(qlinear_q_kernel, dim3((unsigned)(p.mtiles * p.otiles)), dim3(512), 0, s, p);
    return launch_status("qlinear_q_kernel");
}

}  // namespace q
}  // namespace r97q
