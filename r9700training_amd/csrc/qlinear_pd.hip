// qlinear_pd.hip -- the base products of the quantized linear over a weight decoded once a call,
// for CDNA4 (gfx950):
//
//   qlinear_pd_kernel<true>    Y[T,N]  = X[T,K] . W^T   (+ the adapter's s.t.B^T in the epilogue)
//   qlinear_pd_kernel<false>   dX[T,K] = dY[T,N] . W    (+ the adapter's dt.A in the epilogue)
//
// The reference's rows are gemm_nt_twin / gemm_nt_adjoint over a stored weight
// (src/adjoint/host/linear.cpp:132-243): W(n,k) = code(n,k) * bf16 scale(n, k/128).
//
// The fused kernel (qlinear_rt.hip) decodes each weight tile inside its main loop, once for every
// 512-token panel, so a launch over T tokens decodes the whole weight ceil(T/512) times, and the
// decode's VALU issues between the MFMAs. Here launch_predecode (qlinear_rt.hip) decodes every
// tile once, with the same lanes and arithmetic, into global memory in the LDS tile format and in
// walk order, and this kernel's main loop has no decode at all: each step's 16 KiB tile is loaded
// two steps ahead (2 KiB a wave, one coalesced 1 KiB load a piece) and written into the LDS tile
// the fused kernel would have decoded it into. Everything else is the fused kernel's (rt_core.h): a
// workgroup owns 512 tokens x 128 outputs, its 8 waves 64 tokens each, v_mfma_f32_32x32x16_bf16
// accumulators, the token fragments loaded straight into registers from the activation's tiled
// copy, one barrier a step. The products are the same MFMAs over the same operands in the same
// order, so the results are the fused kernel's bits.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "rt_core.h"

namespace r97q {
namespace rt {
namespace {

constexpr int kPdWaves = 8;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // a native 16-byte vector (registers)

template <bool FWD, int WAVE>
struct PdWave {
    using G = Geo<kPdWaves>;
    static constexpr int kMI = G::kMI;
    static constexpr int kShare = kTileBytes / kPdWaves;  // bytes of a tile this wave copies
    static constexpr int kPieces = kShare / 1024;         // its 16-byte pieces a lane

    const uint16_t* act;
    const uint8_t* wt;  // this output tile's decoded tiles, nsteps x kTileBytes
    int64_t sstride;    // elements between consecutive steps of the tiled operand
    int lane, nsteps;

    // this wave's share of tile s into registers (one coalesced 1 KiB load a piece) ...
    __device__ __forceinline__ void fetch(int s, u32x4 (&r)[kPieces]) const {
        const uint8_t* src = wt + (int64_t)s * kTileBytes + kShare * WAVE + 16 * lane;
#pragma unroll
        for (int q = 0; q < kPieces; ++q) r[q] = *reinterpret_cast<const u32x4*>(src + 1024 * q);
    }
    // ... and from them into the LDS tile at the same offsets (the tile is stored as LDS holds it)
    __device__ __forceinline__ void put(const u32x4 (&r)[kPieces], uint8_t* dst) const {
#pragma unroll
        for (int q = 0; q < kPieces; ++q)
            *reinterpret_cast<u32x4*>(dst + kShare * WAVE + 1024 * q + 16 * lane) = r[q];
    }

    // step s: MFMAs on tile s (LDS `cur`) with the token fragments `t` (each round's reloaded with
    // the next step's once its MFMAs have issued; round 3's at the step's start: they are this
    // step's); tile s+1 (fetched a step ago into `have`) written into `nxt` in round 2 (its last
    // reader was step s-1, which its barrier closed); tile s+2 fetched into `want`. On entry b0
    // holds tile s's round-0 fragments; on exit tile s+1's.
    __device__ __forceinline__ void step(int s, const int64_t (&blk)[kMI], uint4 (&t)[kMI][4], const uint8_t* cur,
                                         uint8_t* nxt, const u32x4 (&have)[kPieces], u32x4 (&want)[kPieces],
                                         bf16x8 (&b0)[kNI], bf16x8 (&b1)[kNI], f32x16 (&acc)[kMI][kNI]) const {
        constexpr int M = kMI * kNI;
        const int sn = s + 1 < nsteps ? s + 1 : nsteps - 1;
        const int sf = s + 2 < nsteps ? s + 2 : nsteps - 1;
        __builtin_amdgcn_sched_barrier(0);
        tokens(act, blk, sstride, s, 3, t);
        fetch(sf, want);
        frags(cur, lane, 1, b1);
        round(t, 0, b0, acc);
        interleave<M, 4, kMI + kPieces, 0, 0>();
        __builtin_amdgcn_sched_barrier(0);
        tokens(act, blk, sstride, sn, 0, t);
        frags(cur, lane, 2, b0);
        round(t, 1, b1, acc);
        interleave<M, 4, kMI, 0, 0>();
        __builtin_amdgcn_sched_barrier(0);
        tokens(act, blk, sstride, sn, 1, t);
        frags(cur, lane, 3, b1);
        round(t, 2, b0, acc);
        put(have, nxt);
        interleave<M, 4, kMI, 0, kPieces>();
        __builtin_amdgcn_sched_barrier(0);
        tile_barrier();
        __builtin_amdgcn_sched_barrier(0);
        tokens(act, blk, sstride, sn, 2, t);
        frags(nxt, lane, 0, b0);
        round(t, 3, b1, acc);
        interleave<M, 4, kMI, 0, 0>();
        __builtin_amdgcn_sched_barrier(0);
    }

    __device__ __forceinline__ void run(int64_t m0, int64_t T, uint8_t* l0, uint8_t* l1, f32x16 (&acc)[kMI][kNI]) const {
        int64_t blk[kMI];
        token_blocks<kMI>(m0, T, lane, blk);
        uint4 t[kMI][4];
        u32x4 ra[kPieces], rb[kPieces];
        bf16x8 b0[kNI], b1[kNI];
        // the loads outstanding at the loop's head are, in order, tile 1's pieces and the token
        // fragments of step 0's rounds 0-2: the order every later step leaves them in
        fetch(0, ra);
        put(ra, l0);
        __builtin_amdgcn_sched_barrier(0);
        fetch(nsteps > 1 ? 1 : 0, rb);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 3; ++j) tokens(act, blk, sstride, 0, j, t);
        __builtin_amdgcn_sched_barrier(0);
        tile_barrier();
        frags(l0, lane, 0, b0);
        // unrolled by two so the LDS tiles and register sets keep fixed names
        for (int s = 0; s < nsteps; s += 2) {
            step(s, blk, t, l0, l1, rb, ra, b0, b1, acc);
            step(s + 1, blk, t, l1, l0, ra, rb, b0, b1, acc);
        }
    }
};

template <bool FWD, int WAVE>
__device__ __forceinline__ void wave_main(const Params& p, uint8_t* l0, uint8_t* l1, int mt, int ot) {
    using G = Geo<kPdWaves>;
    f32x16 acc[G::kMI][kNI];
#pragma unroll
    for (int mi = 0; mi < G::kMI; ++mi)
#pragma unroll
        for (int ni = 0; ni < kNI; ++ni) acc[mi][ni] = (f32x16){};
    const int lane = threadIdx.x & 63;
    const int64_t red = FWD ? p.K : p.N;
    const int nsteps = (int)(red / kStep);
    const int64_t m0 = (int64_t)mt * kBM + G::kWaveM * WAVE, o0 = (int64_t)ot * kBN;
    const PdWave<FWD, WAVE> w{p.act, p.wt + (int64_t)ot * nsteps * kTileBytes, act_tile_blocks(p.T) * kBlock, lane,
                              nsteps};
    w.run(m0, p.T, l0, l1, acc);
    if (p.rank > 0) adapter<G::kMI>(p.P, p.Q, p.rank, m0, o0, p.T, lane, acc);
    store<G::kMI>(acc, p.out, FWD ? p.N : p.K, m0, o0, p.T, lane, p.out_f32, FWD ? 0 : p.accumulate);
    if constexpr (!FWD)
        if (p.sums[0].part || p.sums[1].part) sum_chunks<kPdWaves>(p);
}

template <bool FWD>
__global__ __launch_bounds__(64 * kPdWaves, 1) void qlinear_pd_kernel(const Params p) {
    __shared__ __attribute__((aligned(16))) uint8_t l0[kTileBytes], l1[kTileBytes];
    const int tile = xcd_tile(blockIdx.x, p.mtiles * p.otiles);
    const int mt = tile / p.otiles, ot = tile % p.otiles;
    switch (threadIdx.x >> 6) {
        case 0: wave_main<FWD, 0>(p, l0, l1, mt, ot); break;
        case 1: wave_main<FWD, 1>(p, l0, l1, mt, ot); break;
        case 2: wave_main<FWD, 2>(p, l0, l1, mt, ot); break;
        case 3: wave_main<FWD, 3>(p, l0, l1, mt, ot); break;
        case 4: wave_main<FWD, 4>(p, l0, l1, mt, ot); break;
        case 5: wave_main<FWD, 5>(p, l0, l1, mt, ot); break;
        case 6: wave_main<FWD, 6>(p, l0, l1, mt, ot); break;
        default: wave_main<FWD, 7>(p, l0, l1, mt, ot); break;
    }
}

// The split tiles' partials (part [S][nsplit][kBM][kBN]; slot lt holds tile nfull + lt) added in
// range order, then into the f32 output (accumulate) or written as f32 / bf16; the slots' rows past
// T (never written) are skipped. Four values a thread a pass: kBN is a multiple of 4, so the four
// lie in one row of the tile.
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* part, int S, int nsplit, int nfull,
                                                           int otiles, int64_t T, int64_t ld, void* out, int out_f32,
                                                           int accumulate) {
    const int64_t n = (int64_t)nsplit * kBM * kBN;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x * 4;
    for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; i < n; i += stride) {
        const int tile = nfull + (int)(i / (kBM * kBN));
        const int e = (int)(i % (kBM * kBN));
        const int64_t row = (int64_t)(tile / otiles) * kBM + e / kBN;
        if (row >= T) continue;
        const int64_t o = row * ld + (int64_t)(tile % otiles) * kBN + e % kBN;
        float4 v = *reinterpret_cast<const float4*>(part + i);
        for (int z = 1; z < S; ++z) {
            const float4 u = *reinterpret_cast<const float4*>(part + (int64_t)z * n + i);
            v.x += u.x;
            v.y += u.y;
            v.z += u.z;
            v.w += u.w;
        }
        if (out_f32) {
            float4* d = reinterpret_cast<float4*>(static_cast<float*>(out) + o);
            if (accumulate) {
                const float4 old = *d;
                v = make_float4(old.x + v.x, old.y + v.y, old.z + v.z, old.w + v.w);
            }
            *d = v;
        } else {
            uint16_t* d = static_cast<uint16_t*>(out) + o;
            if (accumulate) {
                v.x += bf16_to_f32(d[0]);
                v.y += bf16_to_f32(d[1]);
                v.z += bf16_to_f32(d[2]);
                v.w += bf16_to_f32(d[3]);
            }
            const uint2 w = {(uint32_t)f32_to_bf16(v.x) | ((uint32_t)f32_to_bf16(v.y) << 16),
                             (uint32_t)f32_to_bf16(v.z) | ((uint32_t)f32_to_bf16(v.w) << 16)};
            *reinterpret_cast<uint2*>(d) = w;
        }
    }
}

}  // namespace

void launch_split_reduce(const Params& p, bool fwd, hipStream_t s) {
    const int nsplit = p.mtiles * p.otiles - p.nfull;
    const int64_t n = (int64_t)nsplit * kBM * kBN;
    const int64_t blocks = (n / 4 + 255) / 256;
    hipLaunchKernelGGL(split_reduce_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, s,
                       (const float*)p.part, p.ksplit, nsplit, p.nfull, p.otiles, p.T, fwd ? p.N : p.K, p.out,
                       p.out_f32, fwd ? 0 : p.accumulate);
}

void launch_pd(const Params& p, bool fwd, hipStream_t s) {
    const dim3 grid((unsigned)(p.mtiles * p.otiles)), block(64 * kPdWaves);
    if (fwd)
        hipLaunchKernelGGL((qlinear_pd_kernel<true>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((qlinear_pd_kernel<false>), grid, block, 0, s, p);
}

}  // namespace rt
}  // namespace r97q
