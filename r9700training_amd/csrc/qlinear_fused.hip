// qlinear_fused.hip -- the fused IQR-decode + bf16-MFMA base products of the quantized linear, for
// CDNA4 (gfx950). Compiled once per code width (-DR97Q_BITS=3..6).
//
//   qlinear_fwd_kernel   Y[T,N]  = X[T,K] . W^T     (+ the adapter's s.t.B^T in the epilogue)
//   qlinear_dx_kernel    dX[T,K] = dY[T,N] . W      (+ the adapter's dt.A in the epilogue)
//
// The reference's rows are gemm_nt_twin / gemm_nt_adjoint over a stored weight
// (src/adjoint/host/linear.cpp:132-243): W(n,k) = code(n,k) * bf16 scale(n, k/128).
//
// Shape of a launch. A 512-thread workgroup (8 waves, two per SIMD) owns a 512-token x 128 output
// tile; wave w owns tokens [64w, 64w+64) and a 64x128 f32 accumulator of eight
// v_mfma_f32_32x32x16_bf16 tiles (128 registers, so two waves share a SIMD and one's decode VALU
// runs under the other's MFMA). The reduction walks in 64-deep steps:
//   * the token operand (X or dY) of the next step streams global -> LDS with direct
//     global_load_lds_dwordx4 (no registers; 8 lanes cover a row's 128 bytes, so every load is
//     fully coalesced and the XOR swizzle is chosen by the address each lane reads); a wave's 64
//     rows are loaded and read by that wave only, so they need no barrier, only its own vmcnt;
//   * the weight tile of the step (128 x 64 values) is decoded by all 512 lanes from the column
//     streams (iqr_device.h), 16 values a lane (4 columns x 4 rows: one 4-row slice of a 32-row
//     segment per wave, so every bit offset is a compile-time constant), into one half of a
//     double-buffered, XOR-swizzled bf16 LDS tile that all eight waves read. Stream words are
//     fetched two steps ahead. Each decoded value feeds 512 tokens of MFMA.
// LDS: two 64 KiB token tiles + two 16 KiB weight tiles = the whole 160 KiB of a gfx950 CU.
// One barrier a step orders the decode of step s+1 against the reads of step s.
//
// Decode of one value (6 VALU ops): the 16-bit state is a bit-field (v_bfe_u32, or v_alignbit +
// mask when it straddles a dword); the codebook hash is v_mad_u32_u24 + mask; v_sad_u8 against
// zero sums its bytes with 1024 in the accumulator, which makes the low half an f16 of
// 1024 + byte-sum; one v_fma_mix_f32 with the exact constant -1150 * scale gives
// (byte-sum - 126) * scale exactly (19 significant bits at most, so no rounding), and
// v_cvt_pk_bf16_f32 rounds once to bf16: the decoded tile is bf16(code * scale), bit for bit.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "iqr_device.h"
#include "qlinear_fused.h"

#ifndef R97Q_BITS
#error "compile with -DR97Q_BITS=<code width>"
#endif

namespace r97q {
namespace {

typedef __bf16 bf16x8 __attribute__((__vector_size__(16)));
typedef __bf16 bf16x2 __attribute__((__vector_size__(4)));
typedef float f32x16 __attribute__((__vector_size__(64)));

constexpr int kWaves = kThreads / 64;               // 8
constexpr int kTileBytes = 128 * 128;               // one decoded bf16 tile (128 rows x 64 values)
constexpr int kActBytes = kBM * 128;                // one token tile (512 rows x 64 values)
static_assert(kWaves * 64 == kBM, "one wave per 64 tokens");
static_assert(2 * kActBytes + 2 * kTileBytes == 160 * 1024, "the buffers fill a gfx950 CU's LDS");

// The double-buffered LDS tiles, declared as four separate arrays: the compiler then sees that the
// direct global -> LDS loads into a token buffer do not alias the weight tile a wave reads, and
// does not wait for those loads before every LDS read.
struct Lds {
    uint8_t* w[2];  // decoded weight tiles [128 rows][128 bytes]
    uint8_t* x[2];  // token tiles [512 rows][128 bytes]
};

// The end of a main-loop step: this wave's global loads (token rows into LDS, stream words into
// registers) have landed and its LDS writes are done, then the workgroup barrier. (__syncthreads
// would do the same, written out so the wait is exactly vmcnt(0) lgkmcnt(0) and visible to the
// compiler's own wait insertion.)
__device__ __forceinline__ void step_barrier() {
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) expcnt(7: no wait) lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
}

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    bf16x2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint32_t comp(const uint4& v, int c) {
    return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w;
}

// XOR swizzle of a 128-byte LDS row's eight 16-byte chunks: 16 consecutive rows reading one
// logical chunk land on 16 distinct 16-byte bank groups (for 32 or 64 four-byte banks).
__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

__device__ __forceinline__ uint8_t* chunk_at(uint8_t* tile, int row, int chunk) {
    return tile + row * 128 + ((chunk ^ swz(row)) << 4);
}

// ---------------------------------------------------------------- one lane's slice
// ROWS consecutive rows ROWS*SLICE.. of a 32-row segment, COLS consecutive columns. Their states
// are the 16-bit windows at bits BITS*(31-i) of the segment's stream; together they span dwords
// D0..D1 (D1 == BITS is the first dword of the next segment in the stream: the segment below, or
// the run's top one at the seam).
template <int BITS, int ROWS, int SLICE>
struct Span {
    static constexpr int kLo = BITS * (32 - ROWS * (SLICE + 1));
    static constexpr int kHi = BITS * (31 - ROWS * SLICE) + 16;
    static constexpr int D0 = kLo / 32;
    static constexpr int D1 = (kHi - 1) / 32;
    static constexpr int NW = D1 - D0 + 1;
    static_assert(D1 <= BITS, "a window reaches past the next segment's first dword");
};

template <int COLS>
struct ColWord;  // the stream dwords of COLS consecutive columns
template <>
struct ColWord<4> {
    uint4 v;
    __device__ __forceinline__ uint32_t at(int c) const { return comp(v, c); }
};
template <>
struct ColWord<2> {
    uint2 v;
    __device__ __forceinline__ uint32_t at(int c) const { return c == 0 ? v.x : v.y; }
};

template <int BITS, int ROWS, int COLS, int SLICE>
struct Words {
    ColWord<COLS> w[Span<BITS, ROWS, SLICE>::NW];
    typename std::conditional<ROWS == 4, uint2, uint4>::type s;  // the rows' bf16 scales
};

template <int BITS, int ROWS, int COLS, int SLICE>
__device__ __forceinline__ void load_words(const uint32_t* __restrict__ stream,
                                           const uint16_t* __restrict__ scale_t, int64_t N,
                                           int64_t g, int64_t gh, int64_t cols, int64_t col, int64_t kb,
                                           Words<BITS, ROWS, COLS, SLICE>& out) {
    using S = Span<BITS, ROWS, SLICE>;
#pragma unroll
    for (int t = 0; t < S::NW; ++t) {
        const int d = S::D0 + t;
        const int64_t idx = d < BITS ? stream_index(g, BITS, d, cols, col) : stream_index(gh, BITS, 0, cols, col);
        out.w[t].v = *reinterpret_cast<const decltype(out.w[t].v)*>(stream + idx);
    }
    out.s = *reinterpret_cast<const decltype(out.s)*>(scale_t + kb * N + g * 32 + ROWS * SLICE);
}

// the value of row ROWS*SLICE+i, column c: bf16(code * scale) as an exact f32
template <int BITS, int ROWS, int COLS, int SLICE>
__device__ __forceinline__ float slice_value(const Words<BITS, ROWS, COLS, SLICE>& wd, int c, int i,
                                             uint32_t a24, uint32_t b, float sc, float off) {
    using S = Span<BITS, ROWS, SLICE>;
    const int o = BITS * (31 - (ROWS * SLICE + i)) - 32 * S::D0;
    const int w = o >> 5, sh = o & 31;
    uint32_t st;
    if (sh + 16 <= 32) st = (wd.w[w].at(c) >> sh) & 0xFFFFu;
    else st = __builtin_amdgcn_alignbit(wd.w[w + 1].at(c), wd.w[w].at(c), sh) & 0xFFFFu;
    const uint32_t h = (st * (a24 & 0xFFFFFFu) + b) & 0x3F3F3F3Fu;
    const uint32_t d = __builtin_amdgcn_sad_u8(h, 0u, 0x6400u);  // f16(1024 + sum)
    const _Float16 hv = __builtin_bit_cast(_Float16, (uint16_t)d);
    return __builtin_fmaf((float)hv, sc, off);  // (sum - 126) * scale, exact
}

__device__ __forceinline__ void scales_of(uint32_t w, float& a, float& b) {
    a = __builtin_bit_cast(float, w << 16);
    b = __builtin_bit_cast(float, w & 0xFFFF0000u);
}

// off: the exact product that turns the decoded unsigned value into (value - bias) * scale in one
// fma (trellis: f16(1024 + byte sum), bias 1150; int8 codes: code ^ 0x80, bias 128)
template <int N>
__device__ __forceinline__ void slice_scales(const uint32_t* w, float (&sc)[N], float (&off)[N], float bias) {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) scales_of(w[i], sc[2 * i], sc[2 * i + 1]);
#pragma unroll
    for (int i = 0; i < N; ++i) off[i] = -bias * sc[i];
}

// The int8-code form's words of one lane, 16 bytes of a 32-byte unit (8 rows x 4 columns; byte
// 16*(c>>1) + 2*i + (c&1) is row i, column c): a forward lane's 4 rows x 4 columns (two 8-byte
// pieces, one a column pair), a dX lane's 8 rows x one column pair; and the rows' bf16 scales.
template <bool FWD>
struct Codes8 {
    uint4 c;
    typename std::conditional<FWD, uint2, uint4>::type s;
};

// byte `b` of `w` (code ^ 0x80) as code * sc, exactly: (u - 128) * sc has at most 16 significant bits
[[maybe_unused]] __device__ __forceinline__ float code8_value(uint32_t w, int b, float sc, float off) {
    return __builtin_fmaf((float)((w >> (8 * b)) & 0xFFu), sc, off);
}

// XCD-aware tile order: consecutive workgroup ids are dealt round-robin over the 8 XCDs;
// renumber so each XCD's workgroups take one contiguous run of tiles (tokens outer, outputs
// inner), which keeps a token panel in that XCD's L2.
__device__ __forceinline__ int xcd_tile(int bid, int nwg) {
    const int xcd = bid & 7, local = bid >> 3;
    const int base = nwg >> 3, rem = nwg & 7;
    return xcd * base + (xcd < rem ? xcd : rem) + local;
}

// ---------------------------------------------------------------- the main loop
// FWD: decoded tile [128 n][64 k] (k contiguous). Wave w decodes rows 4w..4w+3 of each of the
//      tile's four 32-row segments; lane = (segment lane>>4, 4 columns 4*(lane&15)); each lane
//      writes 8 bytes (4 k) a row.
// DX:  decoded tile [128 k][64 n] (n contiguous). Wave w decodes rows 8*(w&3)..+8 of segment w>>2
//      of the step's two; lane = 2 columns 2*lane; each lane writes one 16-byte chunk (8 n) a
//      column, so a write instruction's rows are the even (or odd) ones and its chunks cover all
//      eight swizzle positions.
template <bool FWD, int BITS, int WAVE>
struct Loop {
    static constexpr int ROWS = FWD ? 4 : 8;
    static constexpr int COLS = FWD ? 4 : 2;
    static constexpr int SLICE = FWD ? WAVE : (WAVE & 3);
    static constexpr bool kCodes8 = BITS == R97Q_CODES8;
    using W = typename std::conditional<kCodes8, Codes8<FWD>, Words<BITS, ROWS, COLS, SLICE>>::type;

    const uint16_t* act;       // X (fwd) or dY (dx): [T, red]
    int64_t red;               // reduction length: K (fwd) or N (dx)
    int64_t N, K;
    const uint32_t* stream;
    const uint16_t* scale_t;
    uint32_t a24, b;
    int64_t run_rows;
    int64_t m0;                // the wave's first token
    int64_t o0;                // the tile's first output: n (fwd) or k (dx)
    int64_t T;
    int lane;

    __device__ __forceinline__ void run(const Lds& lds, f32x16 (&acc)[2][4]) {
        const int seg = FWD ? lane >> 4 : WAVE >> 2;
        const int cg = FWD ? lane & 15 : lane;
        const int nsteps = (int)(red / kStep);

        // where step s's weight tile comes from
        auto words_for = [&](int s, W& wd) {
            if constexpr (kCodes8) {
                // forward: rows o0 + 32*seg + 4*WAVE .. +4 (row half WAVE&1 of the unit), columns
                // 4*cg.. of the step; dX: rows 64*s + 32*seg + 8*SLICE .. +8, columns o0 + 2*lane,
                // +1 (column pair lane&1 of the unit)
                const int8_t* units = reinterpret_cast<const int8_t*>(stream);
                int64_t srow, k4, kb;
                if (FWD) {
                    srow = o0 + 32 * seg + 4 * WAVE;
                    k4 = (int64_t)s * (kStep / 4) + cg;
                    kb = ((int64_t)s * kStep) >> 7;
                } else {
                    srow = (int64_t)s * kStep + 32 * seg + 8 * SLICE;
                    k4 = (o0 >> 2) + (lane >> 1);
                    kb = o0 >> 7;
                }
                const int8_t* unit = units + ((srow >> 3) * (K >> 2) + k4) * 32;
                if constexpr (FWD) {
                    const uint2 p0 = *reinterpret_cast<const uint2*>(unit + 8 * (WAVE & 1));
                    const uint2 p1 = *reinterpret_cast<const uint2*>(unit + 16 + 8 * (WAVE & 1));
                    wd.c = make_uint4(p0.x, p0.y, p1.x, p1.y);
                } else {
                    wd.c = *reinterpret_cast<const uint4*>(unit + 16 * (lane & 1));
                }
                wd.s = *reinterpret_cast<const decltype(wd.s)*>(scale_t + kb * N + srow);
            } else {
                int64_t g, col, kb;
                if (FWD) {
                    g = (o0 >> 5) + seg;
                    col = (int64_t)s * kStep + 4 * cg;
                    kb = ((int64_t)s * kStep) >> 7;
                } else {
                    g = (((int64_t)s * kStep) >> 5) + seg;
                    col = o0 + 2 * cg;
                    kb = o0 >> 7;
                }
                load_words<BITS, ROWS, COLS, SLICE>(stream, scale_t, N, g, halo_segment(g, run_rows, N), K, col,
                                                    kb, wd);
            }
        };
        auto decode = [&](const W& wd, uint8_t* tile) {
            float sc[ROWS], off[ROWS];
            slice_scales<ROWS>(reinterpret_cast<const uint32_t*>(&wd.s), sc, off, kCodes8 ? 128.0f : 1150.0f);
            // the value of the lane's row i, column c
            auto value = [&](int c, int i) -> float {
                if constexpr (kCodes8) {
                    // forward: column c, row i of the row half: byte 8*(c>>1) + 2*i + (c&1) of the
                    // two pieces; dX: column c of the pair, row i: byte 2*i + c
                    const int byte = FWD ? 8 * (c >> 1) + 2 * i + (c & 1) : 2 * i + c;
                    const uint32_t w = comp(wd.c, byte >> 2) ^ 0x80808080u;
                    return code8_value(w, byte & 3, sc[i], off[i]);
                } else {
                    return slice_value<BITS, ROWS, COLS, SLICE>(wd, c, i, a24, b, sc[i], off[i]);
                }
            };
            if (FWD) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float v0 = value(0, i);
                    const float v1 = value(1, i);
                    const float v2 = value(2, i);
                    const float v3 = value(3, i);
                    const int row = 32 * seg + 4 * SLICE + i;
                    const uint2 o = {pack_bf16(v0, v1), pack_bf16(v2, v3)};
                    *reinterpret_cast<uint2*>(chunk_at(tile, row, cg >> 1) + ((cg & 1) << 3)) = o;
                }
            } else {
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    float v[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) v[i] = value(c, i);
                    const uint4 o = {pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]),
                                     pack_bf16(v[6], v[7])};
                    // rows n = 32*seg + 8*SLICE .. +8 of column 2*cg + c: chunk 4*seg + SLICE
                    *reinterpret_cast<uint4*>(chunk_at(tile, 2 * cg + c, 4 * seg + SLICE)) = o;
                }
            }
        };

        // this wave's 64 token rows of a tile sit at rows 64*WAVE.. of the tile: 8 rows of 128
        // bytes a load instruction, lane i writing LDS bytes 16*i of the instruction's 1 KiB (the
        // chunk swizzle is applied by the global address each lane reads)
        const uint16_t* gr[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int r = 8 * q + (lane >> 3);  // row within the wave's 64
            const int pc = lane & 7;            // physical chunk the lane fills
            int64_t row = m0 + r;
            if (row > T - 1) row = T - 1;
            gr[q] = act + row * red + 8 * (pc ^ swz(64 * WAVE + r));
        }
        uint8_t* x0 = lds.x[0] + (64 * WAVE) * 128;  // this wave's rows of the two token buffers
        uint8_t* x1 = lds.x[1] + (64 * WAVE) * 128;

        W wa, wb;
        words_for(0, wa);
        load_act(gr, x0, 0);
        decode(wa, lds.w[0]);
        words_for(nsteps > 1 ? 1 : 0, wa);
        step_barrier();

        // step s: the MFMAs run on buffers s%2 while the words of step s+2 and the token tile of
        // step s+1 are fetched, tile s+1 is decoded from the words fetched a step ago, and the
        // step ends when this wave's token loads have landed and every wave has decoded.
        for (int s = 0; s < nsteps; s += 2) {
            step(s, nsteps, gr, x0, x1, acc, lds.w[0], lds.w[1], wa, wb, words_for, decode);
            step(s + 1, nsteps, gr, x1, x0, acc, lds.w[1], lds.w[0], wb, wa, words_for, decode);
        }
    }

    // rows [8*Q0, 8*Q1) of the wave's 64 x 64 values of step k0 into `dst` (one direct
    // global -> LDS load of 8 rows each)
    template <int Q0 = 0, int Q1 = 8>
    __device__ __forceinline__ void load_act(const uint16_t* const (&gr)[8], uint8_t* dst, int64_t k0) {
#pragma unroll
        for (int q = Q0; q < Q1; ++q)
            __builtin_amdgcn_global_load_lds(static_cast<const void*>(gr[q] + k0),
                                             (__attribute__((address_space(3))) void*)(dst + q * 1024), 16, 0, 0);
    }

    template <class WF, class DF>
    __device__ __forceinline__ void step(int s, int nsteps, const uint16_t* const (&gr)[8],
                                         const uint8_t* xc, uint8_t* xn, f32x16 (&acc)[2][4],
                                         const uint8_t* cur, uint8_t* nxt, W& dec, W& fetch,
                                         WF& words_for, DF& decode) {
        const int half = lane >> 5, l32 = lane & 31;
        const int64_t kn = (int64_t)(s + 1 < nsteps ? s + 1 : nsteps - 1) * kStep;
        // The token tile of step s+1 is issued inside the rounds: the forward half in each of
        // rounds 1 and 2, dX all in round 0 after its fragment reads (measured against issuing it
        // here at the step's start: 12% faster for the forward, 1% for dX).
        // The two waves that share a SIMD (w and w+4) work in opposite phases: wave w+4 decodes
        // the next tile before this step's MFMAs, wave w after them, so each one's decode VALU
        // issues while the other one's MFMAs keep the matrix core busy. (The next tile's buffer
        // was last read in step s-1, which the barrier that ended it closed.)
        if (WAVE >= 4) decode(dec, nxt);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bf16x8 af[2], bf[4];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) {
                const int row = 32 * mi + l32;  // within the wave's rows; swizzle by the tile row
                af[mi] = as_bf16x8(*reinterpret_cast<const uint4*>(
                    const_cast<uint8_t*>(xc) + row * 128 + (((4 * half + j) ^ swz(64 * WAVE + row)) << 4)));
            }
#pragma unroll
            for (int ni = 0; ni < 4; ++ni)
                bf[ni] = as_bf16x8(*reinterpret_cast<const uint4*>(
                    chunk_at(const_cast<uint8_t*>(cur), 32 * ni + l32, 4 * half + j)));
            // the stream words of step s+2, issued in round 1 (measured 1% faster for dX than at
            // the step's start, no change for the forward; round 2 is slower)
            if (j == 1) words_for(s + 2 < nsteps ? s + 2 : nsteps - 1, fetch);
            if constexpr (FWD) {
                if (j == 1) load_act<0, 4>(gr, xn, kn);
                if (j == 2) load_act<4, 8>(gr, xn, kn);
            } else {
                if (j == 0) load_act(gr, xn, kn);
            }
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma32(af[mi], bf[ni], acc[mi][ni]);
        }
        if (WAVE < 4) decode(dec, nxt);
        step_barrier();
    }
};

// ---------------------------------------------------------------- epilogue and kernels
template <bool FWD>
__device__ __forceinline__ void adapter(const uint16_t* P, const uint16_t* Q, int r, int64_t m0,
                                        int64_t o0, int64_t T, int lane, f32x16 (&acc)[2][4]) {
    // acc += [hi | lo](P)[m, :] . [Q | Q][o, :]^T over 2r: P [T, 2r] bf16; Q [outputs, r] bf16
    // (B for the forward, A^T for dX)
    const int half = lane >> 5, l32 = lane & 31;
    for (int kk = 0; kk < 2 * r; kk += 16) {
        const int kq = kk + 8 * half;
        bf16x8 pa[2], qb[4];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
            int64_t row = m0 + 32 * mi + l32;
            if (row > T - 1) row = T - 1;
            pa[mi] = as_bf16x8(*reinterpret_cast<const uint4*>(P + row * 2 * r + kq));
        }
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
            qb[ni] = as_bf16x8(*reinterpret_cast<const uint4*>(Q + (o0 + 32 * ni + l32) * r + (kq % r)));
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma32(pa[mi], qb[ni], acc[mi][ni]);
    }
}

// accumulator element e of tile (mi, ni) is row 32*mi + 8*(e/4) + 4*half + e%4, column 32*ni + l32;
// SCALED: a factor a row, rs[row * rs_ld], applied before the write (a compile-time choice: the
// plain kernels keep the register allocation and schedule they have without it)
template <bool SCALED = false>
__device__ __forceinline__ void store(const f32x16 (&acc)[2][4], void* out, int64_t ld, int64_t m0,
                                      int64_t o0, int64_t T, int lane, int f32, int accumulate,
                                      const float* rs = nullptr, int64_t rs_ld = 0) {
    const int half = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int64_t row = m0 + 32 * mi + 8 * (e >> 2) + 4 * half + (e & 3);
            if (row >= T) continue;
            const float f = SCALED ? rs[row * rs_ld] : 1.0f;
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                const int64_t col = o0 + 32 * ni + l32;
                float v = SCALED ? acc[mi][ni][e] * f : acc[mi][ni][e];
                if (f32) {
                    float* d = reinterpret_cast<float*>(out) + row * ld + col;
                    *d = accumulate ? *d + v : v;
                } else {
                    uint16_t* d = reinterpret_cast<uint16_t*>(out) + row * ld + col;
                    if (accumulate) v += bf16_to_f32(*d);
                    *d = f32_to_bf16(v);
                }
            }
        }
}

template <int BITS, int SLICE>
__device__ __forceinline__ void fwd_wave(const FwdParams& p, const Lds& lds, int lane, int mt, int nt) {
    f32x16 acc[2][4];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = (f32x16){};
    Loop<true, BITS, SLICE> L{p.X, p.K, p.N, p.K, p.stream, p.scale_t, p.a24, p.b, p.run_rows,
                              (int64_t)mt * kBM + 64 * SLICE, (int64_t)nt * kBN, p.T, lane};
    L.run(lds, acc);
    if (p.rank > 0) adapter<true>(p.P, p.B, p.rank, L.m0, L.o0, p.T, lane, acc);
    store(acc, p.Y, p.N, L.m0, L.o0, p.T, lane, p.y_f32, 0);
}

template <int BITS, int SLICE, bool SCALED>
__device__ __forceinline__ void dx_wave(const DxParams& p, const Lds& lds, int lane, int mt, int kt) {
    f32x16 acc[2][4];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = (f32x16){};
    Loop<false, BITS, SLICE> L{p.dY, p.N, p.N, p.K, p.stream, p.scale_t, p.a24, p.b, p.run_rows,
                               (int64_t)mt * kBM + 64 * SLICE, (int64_t)kt * kBN, p.T, lane};
    L.run(lds, acc);
    if (p.rank > 0) adapter<false>(p.P, p.At, p.rank, L.m0, L.o0, p.T, lane, acc);
    // the coded trunk's code basis: the tile's 128 columns are one activation-scale group
    if constexpr (SCALED)
        store<true>(acc, p.dX, p.K, L.m0, L.o0, p.T, lane, p.dx_f32, p.accumulate, p.a_scale + kt, p.a_scale_ld);
    else
        store(acc, p.dX, p.K, L.m0, L.o0, p.T, lane, p.dx_f32, p.accumulate);
}

// X: further template arguments after the slice (", SCALED"), or empty
#define R97Q_WAVE_SWITCH(fn, X, ...)                    \
    switch (threadIdx.x >> 6) {                         \
        case 0: fn<R97Q_BITS, 0 X>(__VA_ARGS__); break;    \
        case 1: fn<R97Q_BITS, 1 X>(__VA_ARGS__); break;    \
        case 2: fn<R97Q_BITS, 2 X>(__VA_ARGS__); break;    \
        case 3: fn<R97Q_BITS, 3 X>(__VA_ARGS__); break;    \
        case 4: fn<R97Q_BITS, 4 X>(__VA_ARGS__); break;    \
        case 5: fn<R97Q_BITS, 5 X>(__VA_ARGS__); break;    \
        case 6: fn<R97Q_BITS, 6 X>(__VA_ARGS__); break;    \
        default: fn<R97Q_BITS, 7 X>(__VA_ARGS__); break;   \
    }
#define R97Q_COMMA_SCALED , SCALED

__global__ __launch_bounds__(kThreads, 1) void qlinear_fwd_kernel(const FwdParams p) {
    __shared__ __attribute__((aligned(16))) uint8_t w0[kTileBytes], w1[kTileBytes], x0[kActBytes], x1[kActBytes];
    const Lds lds{{w0, w1}, {x0, x1}};
    const int tile = xcd_tile(blockIdx.x, p.mtiles * p.ntiles);
    const int mt = tile / p.ntiles, nt = tile % p.ntiles;
    const int lane = threadIdx.x & 63;
    R97Q_WAVE_SWITCH(fwd_wave, , p, lds, lane, mt, nt)
}

// SCALED: dX in the code basis of an i8a8h activation (p.a_scale set)
template <bool SCALED>
__global__ __launch_bounds__(kThreads, 1) void qlinear_dx_kernel(const DxParams p) {
    __shared__ __attribute__((aligned(16))) uint8_t w0[kTileBytes], w1[kTileBytes], x0[kActBytes], x1[kActBytes];
    const Lds lds{{w0, w1}, {x0, x1}};
    const int tile = xcd_tile(blockIdx.x, p.mtiles * p.ktiles);
    const int mt = tile / p.ktiles, kt = tile % p.ktiles;
    const int lane = threadIdx.x & 63;
    R97Q_WAVE_SWITCH(dx_wave, R97Q_COMMA_SCALED, p, lds, lane, mt, kt)
}

}  // namespace

template <>
void launch_fwd<R97Q_BITS>(const FwdParams& p, hipStream_t s) {
    hipLaunchKernelGGL(qlinear_fwd_kernel, dim3((unsigned)(p.mtiles * p.ntiles)), dim3(kThreads), 0, s, p);
}

template <>
void launch_dx<R97Q_BITS>(const DxParams& p, hipStream_t s) {
    const dim3 grid((unsigned)(p.mtiles * p.ktiles));
    if (p.a_scale)
        hipLaunchKernelGGL(qlinear_dx_kernel<true>, grid, dim3(kThreads), 0, s, p);
    else
        hipLaunchKernelGGL(qlinear_dx_kernel<false>, grid, dim3(kThreads), 0, s, p);
}

}  // namespace r97q
