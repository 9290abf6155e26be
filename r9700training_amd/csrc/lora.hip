// lora.hip -- the adapter's skinny kernels on gfx950: the rank-r down products t = X.A^T and
// dt = s.dY.B, and the factor gradients dA += dt^T.X and dB += s.dY^T.t.
//
// The reference rows are the float lora_shrink / lora_expand twins and adjoints
// (src/adjoint/host/lora.cpp:226-244, 260-328, 416-441, 451-521); their f64 sums are carried here
// in f32 MFMA accumulators over exact bf16 products, with the f32 adapter activations split into a
// [hi | lo] pair of bf16 (hi = bf16(v), lo = bf16(v - hi)) wherever they enter an MFMA, so the
// adapter path keeps ~16 significant bits.
//
//   lora_down_kernel   one workgroup = 16 token rows x the whole reduction, its 4 waves a quarter
//                      each (v_mfma_f32_16x16x32_bf16), reduced through LDS in a fixed order; it
//                      writes the f32 result and its [hi | lo] splits for the fused kernels'
//                      epilogues (row-major) and for the gradient kernel (transposed).
//   lora_grads_kernel  dA and dB in one launch: a workgroup = 64 output columns x a token chunk;
//                      the token tile (X or dY) is staged in LDS with coalesced loads and read
//                      back transposed with ds_read_b64_tr_b16, the [hi | lo] split of dt or s.t
//                      is the other operand; chunks combine with f32 atomics (as the reference's
//                      device rows add into the step's f32 gradient stage).
//   transpose2_kernel  B [N, r] -> B^T [rd, N] (zero rows up to the 16-wide rank) and
//                      A [r, K] -> A^T [K, r], in one launch.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "iqr_device.h"
#include "lora.h"
#include "status.h"

namespace r97q {
namespace {

typedef __bf16 bf16x8 __attribute__((__vector_size__(16)));
typedef float f32x4 __attribute__((__vector_size__(16)));
typedef short s16x4 __attribute__((__vector_size__(4 * sizeof(short))));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// hi = bf16(v), lo = bf16(v - hi): v == hi + lo to ~2^-16 relative
__device__ __forceinline__ void split(float v, uint16_t& hi, uint16_t& lo) {
    hi = f32_to_bf16(v);
    lo = f32_to_bf16(v - bf16_to_f32(hi));
}

// ---------------------------------------------------------------- down
template <int RD>
__global__ __launch_bounds__(256) void lora_down_kernel(DownArgs a) {
    __shared__ float red[4][16][RD];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row16 = lane & 15, grp = lane >> 4;
    const int64_t m0 = (int64_t)blockIdx.x * 16;
    int64_t row = m0 + row16;
    if (row > a.T - 1) row = a.T - 1;
    const int64_t kq = a.Kin / 4;  // a multiple of 32
    const uint16_t* ap = a.In + row * a.Kin + wave * kq + 8 * grp;
    const uint16_t* wp = a.W + (int64_t)row16 * a.Kin + wave * kq + 8 * grp;
    constexpr int NB = RD / 16;
    f32x4 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = (f32x4){};
    int64_t k = 0;
    for (; k + 128 <= kq; k += 128) {
        uint4 av[4], bv[4][NB];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            av[u] = *reinterpret_cast<const uint4*>(ap + k + 32 * u);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                bv[u][nb] = *reinterpret_cast<const uint4*>(wp + (int64_t)16 * nb * a.Kin + k + 32 * u);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) acc[nb] = mfma16(as_bf16x8(av[u]), as_bf16x8(bv[u][nb]), acc[nb]);
    }
    for (; k < kq; k += 32) {
        const bf16x8 av = as_bf16x8(*reinterpret_cast<const uint4*>(ap + k));
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            acc[nb] = mfma16(av, as_bf16x8(*reinterpret_cast<const uint4*>(wp + (int64_t)16 * nb * a.Kin + k)), acc[nb]);
    }
    // 16x16 accumulator: element e is row 4*grp + e, column row16
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int e = 0; e < 4; ++e) red[wave][4 * grp + e][16 * nb + row16] = acc[nb][e];
    __syncthreads();
    for (int i = threadIdx.x; i < 16 * RD; i += 256) {
        const int ml = i / RD, j = i % RD;
        const int64_t m = m0 + ml;
        if (j >= a.r || m >= a.ldt) continue;
        const float v = ((red[0][ml][j] + red[1][ml][j]) + red[2][ml][j]) + red[3][ml][j];
        uint16_t hi = 0, lo = 0;
        if (m < a.T) {
            if (a.out) a.out[m * a.r + j] = a.sa * v;
            split(a.sb * v, hi, lo);
            if (a.P) {
                a.P[m * 2 * a.r + j] = hi;
                a.P[m * 2 * a.r + a.r + j] = lo;
            }
        }
        // the transposed splits are zero past T: the gradient kernel reduces over whole 32-row steps
        if (a.Pt) {
            a.Pt[(int64_t)j * a.ldt + m] = hi;
            a.Pt[(int64_t)(a.r + j) * a.ldt + m] = lo;
        }
        if (a.Pt2) {
            uint16_t h2 = 0, l2 = 0;
            if (m < a.T) split(a.s2 * a.U2[m * a.r + j], h2, l2);
            a.Pt2[(int64_t)j * a.ldt + m] = h2;
            a.Pt2[(int64_t)(a.r + j) * a.ldt + m] = l2;
        }
    }
}

// ---------------------------------------------------------------- grads
// C[v][c] = sum_m Pt[v][m] V[m][c] over the chunk's rows, v = 0..2r-1 (hi rows then lo rows);
// out gets scale * (C[j][c] + C[r+j][c]).
template <int R>
__global__ __launch_bounds__(256) void lora_grads_kernel(GradArgs ga) {
    constexpr int R2 = 2 * R;
    constexpr int VB = (R2 + 15) / 16;  // 16-row blocks of the [hi | lo] operand
    __shared__ __attribute__((aligned(16))) uint16_t tile[32 * 64];
    __shared__ float cred[R2 < 16 ? 16 : R2][64];
    const GradOne& g = ga.one[blockIdx.z];
    const int64_t C = g.C;
    const int64_t c0 = (int64_t)blockIdx.x * 64;
    if (c0 >= C) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int i16 = lane & 15, grp = lane >> 4;
    const int64_t mb = (int64_t)blockIdx.y * ga.chunk;
    int64_t me = mb + ga.chunk;
    if (me > ga.ldt) me = ga.ldt;
    f32x4 acc[VB];
#pragma unroll
    for (int vb = 0; vb < VB; ++vb) acc[vb] = (f32x4){};
    // staging: thread t loads row t/8 (of 32), 16 bytes at column chunk t%8 (of 8): coalesced
    const int lr = threadIdx.x >> 3, lc = threadIdx.x & 7;
    for (int64_t m = mb; m < me; m += 32) {
        int64_t row = m + lr;
        if (row > ga.T - 1) row = ga.T - 1;  // rows past T meet zero splits
        const uint4 v = *reinterpret_cast<const uint4*>(g.V + row * C + c0 + 8 * lc);
        __syncthreads();
        *reinterpret_cast<uint4*>(&tile[lr * 64 + 8 * lc]) = v;
        __syncthreads();
        // B operand (m x c): lane 16*grp + i needs V[m + 8*grp + 0..7][c0 + 16*wave + i]; two
        // transposing reads give rows 4h..4h+3 of the group: lane 16*grp + 4e + q addresses
        // row 8*grp + 4h + e, columns 16*wave + 4q .. +3
        const int e = i16 >> 2, q = i16 & 3;
        s16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4*)((__attribute__((address_space(3))) uint16_t*)tile + (8 * grp + e) * 64 + 16 * wave + 4 * q));
        s16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4*)((__attribute__((address_space(3))) uint16_t*)tile + (8 * grp + 4 + e) * 64 + 16 * wave + 4 * q));
        const uint4 bw = {(uint32_t)(uint16_t)lo4[0] | ((uint32_t)(uint16_t)lo4[1] << 16),
                          (uint32_t)(uint16_t)lo4[2] | ((uint32_t)(uint16_t)lo4[3] << 16),
                          (uint32_t)(uint16_t)hi4[0] | ((uint32_t)(uint16_t)hi4[1] << 16),
                          (uint32_t)(uint16_t)hi4[2] | ((uint32_t)(uint16_t)hi4[3] << 16)};
        const bf16x8 bv = as_bf16x8(bw);
        // A operand (v x m): lane 16*grp + i holds Pt[16*vb + i][m + 8*grp .. +7]
#pragma unroll
        for (int vb = 0; vb < VB; ++vb) {
            const int vr = 16 * vb + i16;
            uint4 aw = {0u, 0u, 0u, 0u};
            if (vr < R2) aw = *reinterpret_cast<const uint4*>(g.Pt + (int64_t)vr * ga.ldt + m + 8 * grp);
            acc[vb] = mfma16(as_bf16x8(aw), bv, acc[vb]);
        }
    }
    // acc element e of block vb: row v = 16*vb + 4*grp + e, column 16*wave + i16
#pragma unroll
    for (int vb = 0; vb < VB; ++vb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int vr = 16 * vb + 4 * grp + e;
            if (vr < R2) cred[vr][16 * wave + i16] = acc[vb][e];
        }
    __syncthreads();
    for (int i = threadIdx.x; i < R * 64; i += 256) {
        const int j = i / 64, cc = i % 64;
        const int64_t c = c0 + cc;
        if (c >= C) continue;
        const float v = g.scale * (cred[j][cc] + cred[R + j][cc]);
        float* d = g.transposed ? g.out + c * R + j : g.out + (int64_t)j * C + c;
        atomicAdd(d, v);
    }
}

// ---------------------------------------------------------------- transposes
// y 0: Bt[q][n] = B[n][q] for q < r, 0 for r <= q < rd;  y 1: At[k][j] = A[j][k]
__global__ __launch_bounds__(256) void transpose2_kernel(const uint16_t* __restrict__ B,
                                                         uint16_t* __restrict__ Bt, int64_t N,
                                                         const uint16_t* __restrict__ A,
                                                         uint16_t* __restrict__ At, int64_t K, int r,
                                                         int rd) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (blockIdx.y == 0) {
        if (i >= (int64_t)rd * N) return;
        const int64_t q = i / N, n = i % N;
        Bt[i] = q < r ? B[n * r + q] : (uint16_t)0;
    } else {
        if (i >= (int64_t)r * K) return;
        const int64_t k = i / r, j = i % r;
        At[i] = A[j * K + k];
    }
}

template <int RD>
int down_r(const DownArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(lora_down_kernel<RD>, dim3((unsigned)((a.ldt + 15) / 16)), dim3(256), 0, s, a);
    return launch_status("lora_down_kernel");
}

template <int R>
int grads_r(const GradArgs& g, int64_t cmax, int nz, hipStream_t s) {
    const int64_t chunks = (g.ldt + g.chunk - 1) / g.chunk;
    hipLaunchKernelGGL(lora_grads_kernel<R>, dim3((unsigned)((cmax + 63) / 64), (unsigned)chunks, (unsigned)nz),
                       dim3(256), 0, s, g);
    return launch_status("lora_grads_kernel");
}

}  // namespace

int down_rank(int r) { return (r + 15) / 16 * 16; }

int64_t grad_ld(int64_t T) { return (T + 31) / 32 * 32; }

int launch_lora_down(const DownArgs& a, hipStream_t s) {
    switch (down_rank(a.r)) {
        case 16: return down_r<16>(a, s);
        case 32: return down_r<32>(a, s);
        case 64: return down_r<64>(a, s);
        default:
            set_error("lora down: rank %d not served", a.r);
            return R97Q_EUNSUPPORTED;
    }
}

int launch_lora_grads(int r, GradArgs g, int nz, hipStream_t s) {
    const int64_t cmax = nz > 1 && g.one[1].C > g.one[0].C ? g.one[1].C : g.one[0].C;
    // about 512 workgroups: chunks of whole 32-row steps
    const int64_t cols = (cmax + 63) / 64 * nz;
    int64_t chunks = (512 + cols - 1) / cols;
    if (chunks < 1) chunks = 1;
    int64_t chunk = (g.ldt + chunks - 1) / chunks;
    chunk = (chunk + 31) / 32 * 32;
    g.chunk = chunk;
    switch (r) {
        case 8: return grads_r<8>(g, cmax, nz, s);
        case 16: return grads_r<16>(g, cmax, nz, s);
        case 32: return grads_r<32>(g, cmax, nz, s);
        case 64: return grads_r<64>(g, cmax, nz, s);
        default:
            set_error("lora grads: rank %d not served", r);
            return R97Q_EUNSUPPORTED;
    }
}

int launch_transpose2(const uint16_t* B, uint16_t* Bt, int64_t N, const uint16_t* A, uint16_t* At,
                      int64_t K, int r, hipStream_t s) {
    const int rd = down_rank(r);
    const int64_t n = (int64_t)rd * N > (int64_t)r * K ? (int64_t)rd * N : (int64_t)r * K;
    hipLaunchKernelGGL(transpose2_kernel, dim3((unsigned)((n + 255) / 256), 2), dim3(256), 0, s, B, Bt, N, A,
                       At, K, r, rd);
    return launch_status("transpose2_kernel");
}

}  // namespace r97q
