// qlinear_rt.hip -- the register-fed fused IQR-decode + bf16-MFMA base products of the quantized
// linear, for CDNA4 (gfx950). Compiled once per code width (-DR97Q_BITS=3..6, or 8 for the
// int8-code form).
//
//   qlinear_rt_kernel<true>    Y[T,N]  = X[T,K] . W^T   (+ the adapter's s.t.B^T in the epilogue)
//   qlinear_rt_kernel<false>   dX[T,K] = dY[T,N] . W    (+ the adapter's dt.A in the epilogue)
//
// The reference's rows are gemm_nt_twin / gemm_nt_adjoint over a stored weight
// (src/adjoint/host/linear.cpp:132-243): W(n,k) = code(n,k) * bf16 scale(n, k/128).
//
// Shape of a launch. A workgroup owns a 512-token x 128-output tile and has WAVES waves (4: one per
// SIMD, each 128 tokens x 128 outputs, 256 accumulation registers; 8: two per SIMD, each 64 tokens
// x 128 outputs, 128 registers, so one wave's stalls are covered by the other's MFMAs). Each wave
// accumulates in v_mfma_f32_32x32x16_bf16 tiles. The reduction walks in 64-deep steps of four
// rounds (one 16-deep slice each):
//   * the token operand (X, or dY) is loaded straight into registers from its tiled copy
//     (act_tiles.h: every fragment one coalesced 1 KiB load); a round's fragments are reloaded
//     with the next step's once its MFMAs have issued. A wave's token rows are its own, so they
//     never pass through LDS;
//   * the weight tile of the next step (128 x 64 values) is decoded by every lane of the
//     workgroup from the column streams (iqr_device.h) into one half of a double-buffered,
//     XOR-swizzled bf16 LDS tile that all waves read (each decoded value feeds 512 tokens); the
//     decode is spread over the step's first three rounds;
//   * one barrier a step, after the third round: the next tile is complete and no wave still reads
//     the tile it replaces, so the fourth round's MFMAs run while the next tile's first fragments
//     are read.
// LDS holds only the two decoded tiles (32 KiB); per step and CU it takes 16 KiB of decoded writes
// and WAVES x 16 KiB of fragment reads against 256 MFMAs.
//
// Decode of one trellis value (6 VALU ops): the 16-bit state is a bit-field (v_bfe_u32, or
// v_alignbit + mask when it straddles a dword); the codebook hash is v_mad_u32_u24 + mask;
// v_sad_u8 against zero sums its bytes with 1024 in the accumulator, which makes the low half an
// f16 of 1024 + byte-sum; one v_fma_mix_f32 with the exact constant -1150 * scale gives
// (byte-sum - 126) * scale exactly, and v_cvt_pk_bf16_f32 rounds once to bf16: the decoded tile
// is bf16(code * scale), bit for bit. The int8-code form reads (code ^ 0x80) as an unsigned byte
// and applies -128 * scale the same way.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "rt_core.h"

#ifndef R97Q_BITS
#error "compile with -DR97Q_BITS=<code width>"
#endif

#ifndef R97Q_RT_WAVES
#define R97Q_RT_WAVES 8
#endif

namespace r97q {
namespace rt {
namespace {

// (the trellis forms' word access; the int8-code build does not use them)
[[maybe_unused]] __device__ __forceinline__ uint32_t comp(const uint4& v, int c) {
    return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w;
}
[[maybe_unused]] __device__ __forceinline__ uint32_t comp(const uint2& v, int c) { return c == 0 ? v.x : v.y; }

// ---------------------------------------------------------------- one lane's slice of a tile
// ROWS consecutive rows ROWS*SLICE.. of a 32-row segment. Their trellis states are the 16-bit
// windows at bits BITS*(31-i) of the segment's stream; together they span dwords D0..D1 (D1 ==
// BITS is the first dword of the next segment in the stream: the segment below, or the run's top
// one at the seam).
template <int BITS, int ROWS, int SLICE>
struct Span {
    static constexpr int kLo = BITS * (32 - ROWS * (SLICE + 1));
    static constexpr int kHi = BITS * (31 - ROWS * SLICE) + 16;
    static constexpr int D0 = kLo / 32;
    static constexpr int D1 = (kHi - 1) / 32;
    static constexpr int NW = D1 - D0 + 1;
    static_assert(D1 <= BITS, "a window reaches past the next segment's first dword");
};

// The words a lane decodes one tile from: the trellis stream dwords of its COLS columns, or its
// 2*ROWS bytes of int8 codes; and its rows' bf16 scales (two a dword).
template <int BITS, int ROWS, int COLS, int SLICE, bool C8 = (BITS == R97Q_CODES8)>
struct LaneWords {
    using S = Span<BITS, ROWS, SLICE>;
    typename std::conditional<COLS == 4, uint4, uint2>::type w[S::NW];
    uint32_t s[ROWS / 2];
};
template <int BITS, int ROWS, int COLS, int SLICE>
struct LaneWords<BITS, ROWS, COLS, SLICE, true> {
    uint32_t c[ROWS];  // forward: 4 columns x ROWS rows; dX: 2 columns x ROWS rows (COLS * ROWS bytes)
    uint32_t s[ROWS / 2];
};

// n bf16 scales (n = 4, 8 or 16) from 8-byte-aligned `src` into s[n / 2]
template <int N>
__device__ __forceinline__ void load_scales(const uint16_t* src, uint32_t (&s)[N / 2]) {
    if constexpr (N == 4) {
        const uint2 v = *reinterpret_cast<const uint2*>(src);
        s[0] = v.x;
        s[1] = v.y;
    } else {
#pragma unroll
        for (int q = 0; q < N / 8; ++q) {
            const uint4 v = *reinterpret_cast<const uint4*>(src + 8 * q);
            s[4 * q] = v.x;
            s[4 * q + 1] = v.y;
            s[4 * q + 2] = v.z;
            s[4 * q + 3] = v.w;
        }
    }
}

// ---------------------------------------------------------------- one wave
// FWD: decoded tile [128 n][64 k] (k contiguous). Wave w decodes rows FR*w..FR*w+FR-1 of each of
//      the tile's four 32-row segments (FR = 32 / WAVES); lane = (segment lane>>4, 4 columns
//      4*(lane&15)); each lane writes 8 bytes (4 k) a row.
// DX:  decoded tile [128 k][64 n] (n contiguous). Wave w decodes DR = 64 / WAVES rows of the step's
//      64, rows DR*(w % (WAVES/2)) .. of segment w / (WAVES/2); lane = 2 columns 2*lane; each lane
//      writes DR/8 16-byte chunks (8 n each) a column.
// LO (the int8-code form only): with `lo` set, the tile holds the low half of each weight's split,
// bf16(w - bf16(w)) -- exact, since code * bf16 scale has at most 16 significant bits -- so a second
// pass over it completes the exact product of the weight (the vocabulary head's f32-level parity).
// A run-time choice, so both passes share one copy of the loop (two copies spill registers).
template <bool FWD, int WAVES, int WAVE, bool LO = false>
struct Wave {
    using G = Geo<WAVES>;
    static constexpr int kMI = G::kMI;
    static constexpr int BITS = R97Q_BITS;
    static constexpr bool C8 = BITS == R97Q_CODES8;
    static constexpr int ROWS = FWD ? G::kFRows : G::kDRows;
    static constexpr int COLS = FWD ? 4 : 2;
    static constexpr int SLICE = FWD ? WAVE : WAVE % (WAVES / 2);
    static constexpr int SEG = FWD ? 0 : WAVE / (WAVES / 2);  // dX: the wave's segment of the step's two
    using LW = LaneWords<BITS, ROWS, COLS, SLICE>;
    // the pieces of a decode, spread over rounds 0-2: forward rows, dX (column, 8-row chunk) pairs
    static constexpr int kPieces = FWD ? ROWS : 2 * (ROWS / 8);

    const Params& p;
    int64_t red;     // reduction length: K (fwd) or N (dx)
    int64_t m0;      // the wave's first token
    int64_t o0;      // the tile's first output
    int64_t sstride; // elements between consecutive steps of the tiled operand
    int lane;
    int nsteps;      // the walk's end: steps s0 .. nsteps-1 (an even count)
    int s0 = 0;      // the walk's first step (split-K: the range's first)
    bool lo = false; // LO: this pass decodes the weights' low halves
    // forward, trellis forms: the stream offsets of the lane's 32-row segment g and of its halo (the
    // segment below, or the run's top one at the tail-biting seam)
    int64_t fwd_seg = 0, fwd_halo = 0;

    __device__ __forceinline__ void setup() {
        if constexpr (FWD && !C8) {
            const int64_t rs = p.run_rows >> 5, ns = p.N >> 5;
            const int64_t g = (o0 >> 5) + (lane >> 4);
            const int64_t top = (g / rs + 1) * rs;
            const int64_t gh = g % rs != 0 ? g - 1 : (top < ns ? top : ns) - 1;
            fwd_seg = g * BITS * (p.K >> 2) * 4;
            fwd_halo = gh * BITS * (p.K >> 2) * 4;
        }
    }

    // ------------------------------------------------ the weight words of step s
    __device__ __forceinline__ void words(int s, LW& wd) const {
        const int64_t N = p.N, K = p.K;
        if constexpr (C8) {
            const uint8_t* units = reinterpret_cast<const uint8_t*>(p.stream);
            if constexpr (FWD) {
                // rows ROWS*WAVE.. of each segment: one whole 8 x 4 unit (ROWS 8) or one row half
                // of it (ROWS 4: bytes 8h..8h+7 and 16+8h..16+8h+7)
                const int seg = lane >> 4, cg = lane & 15;
                const int64_t srow = o0 + 32 * seg + ROWS * WAVE;
                const uint8_t* u = units + (((srow >> 3) * (K >> 2) + (int64_t)s * (kStep / 4) + cg) * 32);
                if constexpr (ROWS == 8) {
                    const uint4 a = *reinterpret_cast<const uint4*>(u);
                    const uint4 b = *reinterpret_cast<const uint4*>(u + 16);
                    wd.c[0] = a.x; wd.c[1] = a.y; wd.c[2] = a.z; wd.c[3] = a.w;
                    wd.c[4] = b.x; wd.c[5] = b.y; wd.c[6] = b.z; wd.c[7] = b.w;
                } else {
                    const int h = (int)(srow & 7) >> 2;
                    const uint2 a = *reinterpret_cast<const uint2*>(u + 8 * h);
                    const uint2 b = *reinterpret_cast<const uint2*>(u + 16 + 8 * h);
                    wd.c[0] = a.x; wd.c[1] = a.y; wd.c[2] = b.x; wd.c[3] = b.y;
                }
                load_scales<ROWS>(p.scale_t + (((int64_t)s * kStep) >> 7) * N + srow, wd.s);
            } else {
                // the lane's column pair (half lane&1 of each unit) in ROWS/8 units down the rows
                const int64_t srow = (int64_t)s * kStep + 32 * SEG + ROWS * SLICE;
                const int64_t k4 = (o0 >> 2) + (lane >> 1);
                const uint8_t* u = units + ((srow >> 3) * (K >> 2) + k4) * 32 + 16 * (lane & 1);
#pragma unroll
                for (int q = 0; q < ROWS / 8; ++q) {
                    const uint4 a = *reinterpret_cast<const uint4*>(u + q * (K >> 2) * 32);
                    wd.c[4 * q] = a.x; wd.c[4 * q + 1] = a.y; wd.c[4 * q + 2] = a.z; wd.c[4 * q + 3] = a.w;
                }
                load_scales<ROWS>(p.scale_t + (o0 >> 7) * N + srow, wd.s);
            }
        } else {
            using S = Span<BITS, ROWS, SLICE>;
            const int64_t rs = p.run_rows >> 5;  // segments a run
            if constexpr (FWD) {
                // the lane's segment and its halo segment are the same every step: their stream
                // offsets (fwd_seg, fwd_halo) are set up once, before the walk
                (void)rs;
                const int64_t g = (o0 >> 5) + (lane >> 4);
                const int64_t col4 = ((int64_t)s * (kStep / 4) + (lane & 15)) * 4;  // 4-column group
#pragma unroll
                for (int t = 0; t < S::NW; ++t) {
                    const int d = S::D0 + t;
                    const int64_t idx = d < BITS ? fwd_seg + d * (K >> 2) * 4 + col4 : fwd_halo + col4;
                    wd.w[t] = *reinterpret_cast<const uint4*>(p.stream + idx);
                }
                load_scales<ROWS>(p.scale_t + (((int64_t)s * kStep) >> 7) * N + 32 * g + ROWS * SLICE, wd.s);
            } else {
                // the wave's segment is uniform: its halo (needed by the slice whose windows reach
                // the next segment) is computed in scalar registers, without a branch
                const int64_t g = 2 * (int64_t)s + SEG;
                int64_t gh = 0;
                if constexpr (S::D1 == BITS) {
                    const int gi = __builtin_amdgcn_readfirstlane((int)g);
                    const int rsi = (int)rs, ns = (int)(N >> 5);
                    const int q = gi / rsi;
                    const int top = (q + 1) * rsi;
                    gh = gi - q * rsi != 0 ? gi - 1 : (top < ns ? top : ns) - 1;
                }
                const int64_t col = o0 + 2 * lane;
#pragma unroll
                for (int t = 0; t < S::NW; ++t) {
                    const int d = S::D0 + t;
                    const int64_t idx = d < BITS ? (g * BITS + d) * K + col : gh * BITS * K + col;
                    wd.w[t] = *reinterpret_cast<const uint2*>(p.stream + idx);
                }
                load_scales<ROWS>(p.scale_t + (o0 >> 7) * N + 32 * g + ROWS * SLICE, wd.s);
            }
        }
    }

    // ------------------------------------------------ the value of the lane's row i, column c
    __device__ __forceinline__ float value(const LW& wd, int c, int i, float sc, float off) const {
        if constexpr (C8) {
            // forward: byte 2*ROWS*(c>>1) + 2*i + (c&1) of the lane's codes; dX: byte 2*(i&7) + c
            // of its unit i>>3
            const int byte = FWD ? 2 * ROWS * (c >> 1) + 2 * i + (c & 1) : 16 * (i >> 3) + 2 * (i & 7) + c;
            const uint32_t w = wd.c[byte >> 2] ^ 0x80808080u;
            const float v = __builtin_fmaf((float)((w >> (8 * (byte & 3))) & 0xFFu), sc, off);
            // the high half rounded by the hardware's RNE conversion (the one that packs the high
            // tile), so the two halves are exactly the split of v
            if constexpr (LO) return lo ? v - (float)(__bf16)v : v;
            return v;
        } else {
            using S = Span<BITS, ROWS, SLICE>;
            const int o = BITS * (31 - (ROWS * SLICE + i)) - 32 * S::D0;
            const int w = o >> 5, sh = o & 31;
            uint32_t st;
            if (sh + 16 <= 32) st = (comp(wd.w[w], c) >> sh) & 0xFFFFu;
            else st = __builtin_amdgcn_alignbit(comp(wd.w[w + 1], c), comp(wd.w[w], c), sh) & 0xFFFFu;
            const uint32_t h = (st * (p.a24 & 0xFFFFFFu) + p.b) & 0x3F3F3F3Fu;
            const uint32_t d = __builtin_amdgcn_sad_u8(h, 0u, 0x6400u);  // f16(1024 + sum)
            const _Float16 hv = __builtin_bit_cast(_Float16, (uint16_t)d);
            return __builtin_fmaf((float)hv, sc, off);  // (sum - 126) * scale, exact
        }
    }

    __device__ __forceinline__ void scale_of(const LW& wd, int i, float& sc, float& off) const {
        const uint32_t w = wd.s[i >> 1];
        sc = __builtin_bit_cast(float, (i & 1) ? (w & 0xFFFF0000u) : (w << 16));
        off = (C8 ? -128.0f : -1150.0f) * sc;
    }

    // ------------------------------------------------ part PART (0..2) of the decode into `tile`
    template <int PART>
    __device__ __forceinline__ void decode(const LW& wd, uint8_t* tile) const {
        constexpr int q0 = PART * kPieces / 3, q1 = (PART + 1) * kPieces / 3;
        if constexpr (FWD) {
            const int seg = lane >> 4, cg = lane & 15;
#pragma unroll
            for (int i = q0; i < q1; ++i) {
                float sc, off;
                scale_of(wd, i, sc, off);
                const float v0 = value(wd, 0, i, sc, off);
                const float v1 = value(wd, 1, i, sc, off);
                const float v2 = value(wd, 2, i, sc, off);
                const float v3 = value(wd, 3, i, sc, off);
                const int row = 32 * seg + ROWS * WAVE + i;
                const uint2 o = {pack_bf16(v0, v1), pack_bf16(v2, v3)};
                *reinterpret_cast<uint2*>(chunk_at(tile, row, cg >> 1) + ((cg & 1) << 3)) = o;
            }
        } else {
#pragma unroll
            for (int q = q0; q < q1; ++q) {
                const int c = q / (ROWS / 8), hh = q % (ROWS / 8);
                float v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    float sc, off;
                    scale_of(wd, 8 * hh + i, sc, off);
                    v[i] = value(wd, c, 8 * hh + i, sc, off);
                }
                const uint4 o = {pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]),
                                 pack_bf16(v[6], v[7])};
                // rows n = 32*SEG + ROWS*SLICE + 8*hh .. +8 of column 2*lane + c
                *reinterpret_cast<uint4*>(chunk_at(tile, 2 * lane + c, 4 * SEG + (ROWS / 8) * SLICE + hh)) = o;
            }
        }
    }

    static constexpr int kWordLoads = C8 ? (FWD ? 2 : ROWS / 8) + (ROWS + 7) / 8
                                         : Span<C8 ? 5 : BITS, ROWS, SLICE>::NW + (ROWS + 7) / 8;
    static constexpr int kValuPart = (FWD ? 4 * ROWS : 2 * ROWS) * 7 / 3 + 8;  // decode operations of a part
    static constexpr int kWrites(int part) { return (part + 1) * kPieces / 3 - part * kPieces / 3; }

    // step s: MFMAs on tile s (LDS `cur`) with the token fragments `t`; each round's fragments are
    // reloaded with the next step's one round after their MFMAs issued (round 3's at the start of
    // the step: they are this step's); tile s+1 decoded from `dec` into `nxt` over rounds 0-2; the
    // words of step s+2 into `fetch`. On entry b0 holds tile s's round-0 fragments; on exit tile
    // s+1's. Each round is its own scheduling region.
    __device__ __forceinline__ void step(int s, const uint16_t* act, const int64_t (&blk)[kMI], uint4 (&t)[kMI][4],
                                         const uint8_t* cur, uint8_t* nxt, const LW& dec, LW& fetch,
                                         bf16x8 (&b0)[kNI], bf16x8 (&b1)[kNI], f32x16 (&acc)[kMI][kNI]) const {
        const int sn = s + 1 < nsteps ? s + 1 : nsteps - 1;
        const int sf = s + 2 < nsteps ? s + 2 : nsteps - 1;
        __builtin_amdgcn_sched_barrier(0);
        constexpr int M = kMI * kNI;
        tokens(act, blk, sstride, s, 3, t);
        words(sf, fetch);
        frags(cur, lane, 1, b1);
        round(t, 0, b0, acc);
        decode<0>(dec, nxt);
        interleave<M, 4, kMI + kWordLoads, kValuPart, kWrites(0)>();
        __builtin_amdgcn_sched_barrier(0);
        tokens(act, blk, sstride, sn, 0, t);
        frags(cur, lane, 2, b0);
        round(t, 1, b1, acc);
        decode<1>(dec, nxt);
        interleave<M, 4, kMI, kValuPart, kWrites(1)>();
        __builtin_amdgcn_sched_barrier(0);
        tokens(act, blk, sstride, sn, 1, t);
        frags(cur, lane, 3, b1);
        round(t, 2, b0, acc);
        decode<2>(dec, nxt);
        interleave<M, 4, kMI, kValuPart, kWrites(2)>();
        __builtin_amdgcn_sched_barrier(0);
        tile_barrier();
        __builtin_amdgcn_sched_barrier(0);
        tokens(act, blk, sstride, sn, 2, t);
        frags(nxt, lane, 0, b0);
        round(t, 3, b1, acc);
        interleave<M, 4, kMI, 0, 0>();
        __builtin_amdgcn_sched_barrier(0);
    }

    __device__ __forceinline__ void run(const uint16_t* act, uint8_t* t0, uint8_t* t1, f32x16 (&acc)[kMI][kNI]) const {
        int64_t blk[kMI];
        token_blocks<kMI>(m0, p.T, lane, blk);
        uint4 t[kMI][4];
        LW wa, wb;
        bf16x8 b0[kNI], b1[kNI];
        // the loads outstanding at the loop's head are, in order, the words of step 1 and the
        // token fragments of step 0's rounds 0-2: the order every later step leaves them in
        words(s0, wa);
        decode<0>(wa, t0);
        decode<1>(wa, t0);
        decode<2>(wa, t0);
        __builtin_amdgcn_sched_barrier(0);
        words(s0 + 1 < nsteps ? s0 + 1 : s0, wb);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 3; ++j) tokens(act, blk, sstride, s0, j, t);
        __builtin_amdgcn_sched_barrier(0);
        tile_barrier();
        frags(t0, lane, 0, b0);
        // step s decodes tile s+1 from the words of step s+1 and fetches those of step s+2 into
        // the set step s+1 decoded from; unrolled by two so the sets keep fixed names
        for (int s = s0; s < nsteps; s += 2) {
            step(s, act, blk, t, t0, t1, wb, wa, b0, b1, acc);
            step(s + 1, act, blk, t, t1, t0, wa, wb, b0, b1, acc);
        }
    }
};

// The wave's part of one work item: tile (mt, ot), range z of S over the reduction (S = 1: the whole
// reduction, the product into `out`; S > 1: a split tile's range, its partial into the tile's slot
// `sp` of the split partials). mt < 0: no tile (a workgroup past its XCD's share), only the
// factor gradients' sums.
template <bool FWD, int WAVES, int WAVE>
__device__ __forceinline__ void wave_main(const Params& p, uint8_t* t0, uint8_t* t1, int mt, int ot, int z, int S,
                                          float* sp) {
    using G = Geo<WAVES>;
    if (mt >= 0) {
        f32x16 acc[G::kMI][kNI];
#pragma unroll
        for (int mi = 0; mi < G::kMI; ++mi)
#pragma unroll
            for (int ni = 0; ni < kNI; ++ni) acc[mi][ni] = (f32x16){};
        const int lane = threadIdx.x & 63;
        const int64_t red = FWD ? p.K : p.N;
        const int pairs = (int)(red / kStep) / 2;  // the steps go in pairs: a range holds whole pairs
        Wave<FWD, WAVES, WAVE> w{p, red, (int64_t)mt * kBM + G::kWaveM * WAVE, (int64_t)ot * kBN,
                                 act_tile_blocks(p.T) * kBlock, lane, 2 * (int)((int64_t)(z + 1) * pairs / S)};
        w.s0 = 2 * (int)((int64_t)z * pairs / S);
        w.setup();
        w.run(p.act, t0, t1, acc);
        const int64_t ld = FWD ? p.N : p.K;
        if (p.rank > 0 && z == 0) adapter<G::kMI>(p.P, p.Q, p.rank, w.m0, w.o0, p.T, lane, acc);
        if (S > 1)  // the tile's [kBM][kBN] slot, its rows past T left unwritten
            store<G::kMI>(acc, sp, kBN, G::kWaveM * WAVE, 0, p.T - (int64_t)mt * kBM, lane, 1, 0);
        else
            store<G::kMI>(acc, p.out, ld, w.m0, w.o0, p.T, lane, p.out_f32, FWD ? 0 : p.accumulate);
    }
    if constexpr (!FWD)
        if (p.sums[0].part || p.sums[1].part) sum_chunks<WAVES>(p);
}

template <bool FWD, int WAVES>
__global__ __launch_bounds__(64 * WAVES, 1) void qlinear_rt_kernel(const Params p) {
    __shared__ __attribute__((aligned(16))) uint8_t t0[kTileBytes], t1[kTileBytes];
    // the work: tiles 0 .. nfull-1 whole, then ksplit ranges of each later tile (the tiles inner)
    const int ntiles = p.mtiles * p.otiles;
    const int nfull = p.ksplit > 1 ? p.nfull : ntiles;
    const int nsplit = ntiles - nfull;
    const int w = xcd_work(blockIdx.x, nfull, p.ksplit > 1 ? p.ksplit * nsplit : 0);
    int tile = -1, z = 0, S = 1;
    float* sp = nullptr;
    if (w >= 0 && w < nfull) {
        tile = w;
    } else if (w >= nfull) {
        const int q = w - nfull;
        z = q / nsplit;
        tile = nfull + q % nsplit;
        S = p.ksplit;
        sp = p.part + ((int64_t)z * nsplit + (tile - nfull)) * kBM * kBN;
    }
    const int mt = tile >= 0 ? tile / p.otiles : -1, ot = tile >= 0 ? tile % p.otiles : 0;
    switch (threadIdx.x >> 6) {
        case 0: wave_main<FWD, WAVES, 0>(p, t0, t1, mt, ot, z, S, sp); break;
        case 1: wave_main<FWD, WAVES, 1>(p, t0, t1, mt, ot, z, S, sp); break;
        case 2: wave_main<FWD, WAVES, 2>(p, t0, t1, mt, ot, z, S, sp); break;
        case 3: wave_main<FWD, WAVES, 3>(p, t0, t1, mt, ot, z, S, sp); break;
        default:
            if constexpr (WAVES == 8) {
                switch (threadIdx.x >> 6) {
                    case 4: wave_main<FWD, WAVES, 4>(p, t0, t1, mt, ot, z, S, sp); break;
                    case 5: wave_main<FWD, WAVES, 5>(p, t0, t1, mt, ot, z, S, sp); break;
                    case 6: wave_main<FWD, WAVES, 6>(p, t0, t1, mt, ot, z, S, sp); break;
                    default: wave_main<FWD, WAVES, 7>(p, t0, t1, mt, ot, z, S, sp); break;
                }
            }
            break;
    }
}

#if R97Q_BITS == R97Q_CODES8
// ---------------------------------------------------------------- the vocabulary head's products
// The vocabulary head's dX products over the int8-code form: grid (tiles, slices); a workgroup
// takes its tile of each range of its slice in turn, each a plain dX product (the token operand the
// range's gathered cotangent columns, tiled) over the weights' high halves and then over their low
// halves (w = hi + lo exactly, bf16 each), all into one f32 accumulator; the sum times the tile's
// scale.col factor is written in f32 into the slice's partial.
template <int WAVES, int WAVE>
__device__ __forceinline__ void vocab_wave(const VocabRtParams& v, uint8_t* t0, uint8_t* t1, int sl, int mt, int ot) {
    using G = Geo<WAVES>;
    f32x16 acc[G::kMI][kNI];
#pragma unroll
    for (int mi = 0; mi < G::kMI; ++mi)
#pragma unroll
        for (int ni = 0; ni < kNI; ++ni) acc[mi][ni] = (f32x16){};
    const int lane = threadIdx.x & 63;
    const int64_t m0 = (int64_t)mt * kBM + G::kWaveM * WAVE, o0 = (int64_t)ot * kBN;
#pragma clang loop unroll(disable)
    for (int it = 2 * v.first[sl]; it < 2 * v.first[sl + 1]; ++it) {
        const int64_t y = it >> 1;
        Params p = v.p;
        p.act += y * v.z_act;
        p.stream += y * v.z_w;
        p.scale_t += y * v.z_scale;
        // the lane index made opaque each pass, so the lane's addresses are derived inside the pass
        // and not held across passes (which spills registers)
        int ln = lane;
        asm volatile("" : "+v"(ln));
        Wave<false, WAVES, WAVE, true> w{p, p.N, m0, o0, act_tile_blocks(p.T) * kBlock, ln, (int)(p.N / kStep)};
        w.lo = (it & 1) != 0;
        w.setup();
        w.run(p.act, t0, t1, acc);
        // every wave past its last reads of the LDS tiles before the next pass decodes into them
        __syncthreads();
    }
    const float f = v.cf[v.cls[sl] * v.cf_ld + ot];
#pragma unroll
    for (int mi = 0; mi < G::kMI; ++mi)
#pragma unroll
        for (int ni = 0; ni < kNI; ++ni)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[mi][ni][e] *= f;
    store<G::kMI>(acc, static_cast<float*>(v.p.out) + (int64_t)sl * v.p.T * v.p.K, v.p.K, m0, o0, v.p.T, lane, 1, 0);
}

template <int WAVES>
__global__ __launch_bounds__(64 * WAVES, 1) void qlinear_rt_vocab_kernel(const VocabRtParams v) {
    __shared__ __attribute__((aligned(16))) uint8_t t0[kTileBytes], t1[kTileBytes];
    const int tile = xcd_tile(blockIdx.x, v.p.mtiles * v.p.otiles);
    const int mt = tile / v.p.otiles, ot = tile % v.p.otiles;
    const int sl = blockIdx.y;
#define R97Q_VOCAB_WAVE(W)                             \
    case W:                                            \
        vocab_wave<WAVES, W>(v, t0, t1, sl, mt, ot); \
        break;
    switch (threadIdx.x >> 6) {
        R97Q_VOCAB_WAVE(0)
        R97Q_VOCAB_WAVE(1)
        R97Q_VOCAB_WAVE(2)
        R97Q_VOCAB_WAVE(3)
        R97Q_VOCAB_WAVE(4)
        R97Q_VOCAB_WAVE(5)
        R97Q_VOCAB_WAVE(6)
        default: R97Q_VOCAB_WAVE(7)
    }
#undef R97Q_VOCAB_WAVE
}
#endif

// ---------------------------------------------------------------- the weight decoded once a call
// Every tile a product walks, decoded to bf16 in the LDS tile format (rt_core.h) and stored in
// walk order: tile (o, s) -- outputs 128o.. (features n, or columns k for dX), reduction values
// 64s.. -- at byte (o * nsteps + s) * kTileBytes of `out`. The lanes and the arithmetic are the
// main loop's (Wave::words, Wave::decode): a tile is decoded into LDS exactly as the fused kernel
// decodes it, then copied out whole, each wave a contiguous 2 KiB (one 1 KiB store a piece), so a
// tile holds the bits the fused kernel multiplies. A workgroup takes one output tile and kPreSteps
// consecutive steps, two LDS tiles in turn, the next step's words in flight while it decodes one.
constexpr int kPreSteps = 8;

template <int WAVES, int WAVE>
__device__ __forceinline__ void copy_out(const uint8_t* tile, uint8_t* g, int lane) {
    constexpr int kShare = kTileBytes / WAVES;
#pragma unroll
    for (int q = 0; q < kShare / 1024; ++q) {
        const int off = kShare * WAVE + 1024 * q + 16 * lane;
        *reinterpret_cast<uint4*>(g + off) = *reinterpret_cast<const uint4*>(tile + off);
    }
}

template <bool FWD, int WAVES, int WAVE>
__device__ __forceinline__ void wave_predecode(const Params& p, uint8_t* out, uint8_t* t0, uint8_t* t1, int ot,
                                               int s0) {
    using WV = Wave<FWD, WAVES, WAVE>;
    const int lane = threadIdx.x & 63;
    const int64_t red = FWD ? p.K : p.N;
    const int nsteps = (int)(red / kStep);
    WV w{p, red, 0, (int64_t)ot * kBN, 0, lane, nsteps};
    w.setup();
    const int s1 = s0 + kPreSteps < nsteps ? s0 + kPreSteps : nsteps;
    uint8_t* base = out + (int64_t)ot * nsteps * kTileBytes;
    typename WV::LW wa, wb;
    w.words(s0, wa);
    for (int s = s0; s < s1; s += 2) {
        w.words(s + 1 < s1 ? s + 1 : s, wb);
        w.template decode<0>(wa, t0);
        w.template decode<1>(wa, t0);
        w.template decode<2>(wa, t0);
        __syncthreads();
        copy_out<WAVES, WAVE>(t0, base + (int64_t)s * kTileBytes, lane);
        if (s + 1 >= s1) break;
        w.words(s + 2 < s1 ? s + 2 : s + 1, wa);
        w.template decode<0>(wb, t1);
        w.template decode<1>(wb, t1);
        w.template decode<2>(wb, t1);
        __syncthreads();
        copy_out<WAVES, WAVE>(t1, base + (int64_t)(s + 1) * kTileBytes, lane);
    }
}

template <bool FWD, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void predecode_kernel(const Params p, uint8_t* out) {
    __shared__ __attribute__((aligned(16))) uint8_t t0[kTileBytes], t1[kTileBytes];
    const int ot = blockIdx.x, s0 = blockIdx.y * kPreSteps;
    switch (threadIdx.x >> 6) {
        case 0: wave_predecode<FWD, WAVES, 0>(p, out, t0, t1, ot, s0); break;
        case 1: wave_predecode<FWD, WAVES, 1>(p, out, t0, t1, ot, s0); break;
        case 2: wave_predecode<FWD, WAVES, 2>(p, out, t0, t1, ot, s0); break;
        case 3: wave_predecode<FWD, WAVES, 3>(p, out, t0, t1, ot, s0); break;
        default:
            if constexpr (WAVES == 8) {
                switch (threadIdx.x >> 6) {
                    case 4: wave_predecode<FWD, WAVES, 4>(p, out, t0, t1, ot, s0); break;
                    case 5: wave_predecode<FWD, WAVES, 5>(p, out, t0, t1, ot, s0); break;
                    case 6: wave_predecode<FWD, WAVES, 6>(p, out, t0, t1, ot, s0); break;
                    default: wave_predecode<FWD, WAVES, 7>(p, out, t0, t1, ot, s0); break;
                }
            }
            break;
    }
}

}  // namespace

template <>
void launch_predecode<R97Q_BITS>(const Params& p, bool fwd, uint8_t* out, hipStream_t s) {
    const int64_t nsteps = (fwd ? p.K : p.N) / kStep;
    const dim3 grid((unsigned)p.otiles, (unsigned)((nsteps + kPreSteps - 1) / kPreSteps));
    if (fwd)
        hipLaunchKernelGGL((predecode_kernel<true, R97Q_RT_WAVES>), grid, dim3(64 * R97Q_RT_WAVES), 0, s, p, out);
    else
        hipLaunchKernelGGL((predecode_kernel<false, R97Q_RT_WAVES>), grid, dim3(64 * R97Q_RT_WAVES), 0, s, p, out);
}

template <>
void launch_fwd<R97Q_BITS>(const Params& p, hipStream_t s) {
    const int ntiles = p.mtiles * p.otiles;
    const int grid = p.ksplit > 1 ? work_grid(p.nfull, p.ksplit * (ntiles - p.nfull)) : ntiles;
    hipLaunchKernelGGL((qlinear_rt_kernel<true, R97Q_RT_WAVES>), dim3((unsigned)grid), dim3(64 * R97Q_RT_WAVES), 0, s, p);
}

#if R97Q_BITS == R97Q_CODES8
void launch_vocab(const VocabRtParams& v, hipStream_t s) {
    static_assert(R97Q_RT_WAVES == 8, "the vocabulary head's kernel takes 8 waves");
    hipLaunchKernelGGL(qlinear_rt_vocab_kernel<R97Q_RT_WAVES>, dim3((unsigned)(v.p.mtiles * v.p.otiles), (unsigned)v.slices),
                       dim3(64 * R97Q_RT_WAVES), 0, s, v);
}
#endif

template <>
void launch_dx<R97Q_BITS>(const Params& p, hipStream_t s) {
    const int ntiles = p.mtiles * p.otiles;
    const int grid = p.ksplit > 1 ? work_grid(p.nfull, p.ksplit * (ntiles - p.nfull)) : ntiles;
    hipLaunchKernelGGL((qlinear_rt_kernel<false, R97Q_RT_WAVES>), dim3((unsigned)grid), dim3(64 * R97Q_RT_WAVES), 0, s, p);
}

}  // namespace rt
}  // namespace r97q
