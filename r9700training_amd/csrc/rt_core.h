// rt_core.h -- the parts the register-fed base products share (qlinear_rt.hip, which decodes the
// weight tile in the main loop, and qlinear_pd.hip, which is fed tiles decoded once a call):
// the LDS tile format, the workgroup's tile order over the XCDs, the token fragments' loads, the
// MFMA rounds and their issue order, and the epilogue (the adapter's up-projection, the store).
//
// The decoded weight tile: 128 rows (outputs: features n in the forward, columns k in dX) x 64
// reduction values, bf16, 128 bytes a row; the row's eight 16-byte chunks XOR-swizzled so 16
// consecutive rows reading one logical chunk land on 16 distinct 16-byte bank groups. Chunk
// 4h + j of a row holds reduction values 32h + 8j .. +8: the order of the token fragments
// (act_tiles.h), so an MFMA's two operands pair up.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "act_tiles.h"
#include "iqr_device.h"
#include "qlinear_rt.h"

namespace r97q {
namespace rt {

typedef __bf16 bf16x8 __attribute__((__vector_size__(16)));
typedef __bf16 bf16x2 __attribute__((__vector_size__(4)));
typedef float f32x16 __attribute__((__vector_size__(64)));

constexpr int kNI = kBN / 32;               // 4 output blocks of 32
constexpr int kTileBytes = kBN * kStep * 2; // one decoded bf16 tile: 128 rows x 128 bytes
constexpr int kBlock = 32 * kStep;          // bf16 elements in one 32 x 64 block of the tiled operand

// the geometry of a workgroup of W waves
template <int W>
struct Geo {
    static constexpr int kWaveM = kBM / W;  // tokens a wave: 128 or 64
    static constexpr int kMI = kWaveM / 32; // its token blocks of 32
    static constexpr int kFRows = 32 / W;   // forward decode: rows a lane takes of each 32-row segment
    static constexpr int kDRows = 64 / W;   // dX decode: rows a lane takes of the step's 64
    static_assert(W == 4 || W == 8, "4 or 8 waves");
};

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    bf16x2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

__device__ __forceinline__ uint8_t* chunk_at(uint8_t* tile, int row, int chunk) {
    return tile + row * 128 + ((chunk ^ swz(row)) << 4);
}

// The end of a tile's production: this wave's LDS writes (and fragment reads) are done, then the
// workgroup barrier. Vector-memory loads (the wave's own token rows, the stream words) are not
// waited for: nothing another wave reads depends on them.
__device__ __forceinline__ void tile_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt not waited
    asm volatile("s_barrier" ::: "memory");
}

// XCD-aware tile order: consecutive workgroup ids are dealt round-robin over the 8 XCDs;
// renumber so each XCD's workgroups take one contiguous run of tiles (tokens outer, outputs
// inner), which keeps a token panel in that XCD's L2.
__device__ __forceinline__ int xcd_tile(int bid, int nwg) {
    const int xcd = bid & 7, local = bid >> 3;
    const int base = nwg >> 3, rem = nwg & 7;
    return xcd * base + (xcd < rem ? xcd : rem) + local;
}

// The fused kernel's work: `full` whole tiles (tiles 0 .. full-1), then `items` split ranges. The
// hardware deals workgroup ids round-robin over the 8 XCDs and starts each XCD's in id order, so
// each XCD's first workgroups take its share of the whole tiles (one contiguous run, as xcd_tile
// deals them) and its later ones its share of the split ranges (contiguous too): the ranges run once
// the whole tiles are done, on every CU. Returns the whole tile's index, full + the range's index,
// or -1 for a workgroup past its XCD's share (work_grid rounds each share up).
__device__ __forceinline__ int xcd_work(int bid, int full, int items) {
    const int xcd = bid & 7, l = bid >> 3;
    const int fb = full >> 3, fr = full & 7, fx = fb + (xcd < fr ? 1 : 0);
    if (l < fx) return xcd * fb + (xcd < fr ? xcd : fr) + l;
    const int ib = items >> 3, ir = items & 7, ix = ib + (xcd < ir ? 1 : 0);
    if (l - fx >= ix) return -1;
    return full + xcd * ib + (xcd < ir ? xcd : ir) + (l - fx);
}

// blk[mi]: element offset of the wave's token block mi at step 0 in the tiled operand of a T-row
// activation (rows past the operand's last block read that block again: their products land in
// rows that are never stored)
template <int MI>
__device__ __forceinline__ void token_blocks(int64_t m0, int64_t T, int lane, int64_t (&blk)[MI]) {
    const int64_t nblk = act_tile_blocks(T);
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
        int64_t rb = (m0 >> 5) + mi;
        if (rb > nblk - 1) rb = nblk - 1;
        blk[mi] = rb * kBlock + 8 * lane;
    }
}

// the token fragments of step s, round j (one 1 KiB load each)
template <int MI>
__device__ __forceinline__ void tokens(const uint16_t* act, const int64_t (&blk)[MI], int64_t sstride, int s, int j,
                                       uint4 (&t)[MI][4]) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
        t[mi][j] = *reinterpret_cast<const uint4*>(act + blk[mi] + (int64_t)s * sstride + 512 * j);
}

// the weight fragments of round j: output block ni's rows, reduction values 32 half + 8j .. +8
__device__ __forceinline__ void frags(const uint8_t* tile, int lane, int j, bf16x8 (&b)[kNI]) {
    const int half = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int ni = 0; ni < kNI; ++ni)
        b[ni] = as_bf16x8(
            *reinterpret_cast<const uint4*>(chunk_at(const_cast<uint8_t*>(tile), 32 * ni + l32, 4 * half + j)));
}

template <int MI>
__device__ __forceinline__ void round(const uint4 (&t)[MI][4], int j, const bf16x8 (&b)[kNI], f32x16 (&acc)[MI][kNI]) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < kNI; ++ni) acc[mi][ni] = mfma32(as_bf16x8(t[mi][j]), b[ni], acc[mi][ni]);
}

// The issue order of one round of M MFMAs: each followed by a share of the round's other work --
// the next round's fragment reads first (they are needed a round later), then the vector-memory
// loads, NVALU VALU operations spread evenly, LDS writes last.
template <int M, int NDSR, int NVMEM, int NVALU, int NDSW>
__device__ __forceinline__ void interleave() {
#pragma unroll
    for (int i = 0; i < M; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        if (i < NDSR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        if (i >= 1 && i - 1 < NVMEM) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
        if (NVALU > 0) __builtin_amdgcn_sched_group_barrier(0x002, (NVALU + M - 1) / M, 0);  // VALU
        if (i >= M - NDSW) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
    }
}

// ---------------------------------------------------------------- epilogue
// acc += [hi | lo](P)[m, :] . [Q | Q][o, :]^T over 2r: P [T, 2r] bf16; Q [outputs, r] bf16
template <int MI>
__device__ __forceinline__ void adapter(const uint16_t* P, const uint16_t* Q, int r, int64_t m0, int64_t o0,
                                        int64_t T, int lane, f32x16 (&acc)[MI][kNI]) {
    const int half = lane >> 5, l32 = lane & 31;
    for (int kk = 0; kk < 2 * r; kk += 16) {
        const int kq = kk + 8 * half;
        bf16x8 pa[MI], qb[kNI];
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) {
            int64_t row = m0 + 32 * mi + l32;
            if (row > T - 1) row = T - 1;
            pa[mi] = as_bf16x8(*reinterpret_cast<const uint4*>(P + row * 2 * r + kq));
        }
#pragma unroll
        for (int ni = 0; ni < kNI; ++ni)
            qb[ni] = as_bf16x8(*reinterpret_cast<const uint4*>(Q + (o0 + 32 * ni + l32) * r + (kq % r)));
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
            for (int ni = 0; ni < kNI; ++ni) acc[mi][ni] = mfma32(pa[mi], qb[ni], acc[mi][ni]);
    }
}

// accumulator element e of tile (mi, ni) is row 32*mi + 8*(e/4) + 4*half + e%4, column 32*ni + l32.
// One instantiation per output mode, so the 64 x MI stores of a lane carry no per-element branch:
// a row pointer a (mi, e) and four stores at immediate offsets 32 ni. FULL: every row of the wave
// is below T (no row check). ACC: a token block's old values are all loaded before any is stored.
template <int MI, bool F32, bool ACC, bool FULL>
__device__ __forceinline__ void store_as(const f32x16 (&acc)[MI][kNI], void* out, int64_t ld, int64_t m0, int64_t o0,
                                         int64_t T, int lane) {
    using E = typename std::conditional<F32, float, uint16_t>::type;
    const int half = lane >> 5, l32 = lane & 31;
    E* base = reinterpret_cast<E*>(out) + (m0 + 4 * half) * ld + o0 + l32;
    const int64_t rows = T - (m0 + 4 * half);  // rows r < rows of this lane's column are stored
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
        float old[16][kNI];
        if constexpr (ACC) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int r = 32 * mi + 8 * (e >> 2) + (e & 3);
                const E* d = base + (int64_t)r * ld;
#pragma unroll
                for (int ni = 0; ni < kNI; ++ni) {
                    if (!FULL && r >= rows) { old[e][ni] = 0.0f; continue; }
                    if constexpr (F32) old[e][ni] = d[32 * ni];
                    else old[e][ni] = bf16_to_f32(d[32 * ni]);
                }
            }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int r = 32 * mi + 8 * (e >> 2) + (e & 3);
            if (!FULL && r >= rows) continue;
            E* d = base + (int64_t)r * ld;
#pragma unroll
            for (int ni = 0; ni < kNI; ++ni) {
                float v = acc[mi][ni][e];
                if constexpr (ACC) v += old[e][ni];
                if constexpr (F32) d[32 * ni] = v;
                else d[32 * ni] = f32_to_bf16(v);
            }
        }
    }
}

template <int MI>
__device__ __forceinline__ void store(const f32x16 (&acc)[MI][kNI], void* out, int64_t ld, int64_t m0, int64_t o0,
                                      int64_t T, int lane, int f32, int accumulate) {
    const bool full = m0 + 32 * MI <= T;  // wave-uniform
    if (f32) {
        if (accumulate) {
            if (full) store_as<MI, true, true, true>(acc, out, ld, m0, o0, T, lane);
            else store_as<MI, true, true, false>(acc, out, ld, m0, o0, T, lane);
        } else {
            if (full) store_as<MI, true, false, true>(acc, out, ld, m0, o0, T, lane);
            else store_as<MI, true, false, false>(acc, out, ld, m0, o0, T, lane);
        }
    } else {
        if (accumulate) store_as<MI, false, true, false>(acc, out, ld, m0, o0, T, lane);
        else store_as<MI, false, false, false>(acc, out, ld, m0, o0, T, lane);
    }
}

// ---------------------------------------------------------------- the factor gradients' sums
// out (+)= the deferred chunk sums of the gradient launch before this one, for dA and dB:
// workgroup b of the launch takes elements [b per, (b+1) per) of each; an element's chunks are
// added in chunk order (the order the gradient launch's own last chunk adds them in), so the
// factor gradients are the same bits either way. Every wave calls it.
template <int W>
__device__ __forceinline__ void sum_chunks(const Params& p) {
    const int64_t nwg = gridDim.x;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const Params::Sums& g = p.sums[q];
        if (!g.part) continue;
        const int64_t n = (int64_t)p.rank * g.cols;
        const int64_t per = (n + nwg - 1) / nwg;
        const int64_t e0 = (int64_t)blockIdx.x * per;
        const int64_t e1 = e0 + per < n ? e0 + per : n;
        for (int64_t e = e0 + threadIdx.x; e < e1; e += 64 * W) {
            const float* src = g.part + e;
            float sum = 0.0f;
            int ch = 0;
            for (; ch + 8 <= g.chunks; ch += 8) {
                float x[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) x[u] = src[(int64_t)(ch + u) * n];
#pragma unroll
                for (int u = 0; u < 8; ++u) sum += x[u];
            }
            for (; ch < g.chunks; ++ch) sum += src[(int64_t)ch * n];
            const int64_t j = e / g.cols, c = e % g.cols;
            g.out[g.transposed ? c * p.rank + j : e] += sum;
        }
    }
}

}  // namespace rt
}  // namespace r97q
