// lora.hip -- the adapter's skinny kernels on gfx950: the rank-r down products t = X.A^T and
// dt = s.dY.B, and the factor gradients dA += dt^T.X and dB += s.dY^T.t.
//
// The reference rows are the float lora_shrink / lora_expand twins and adjoints
// (src/adjoint/host/lora.cpp:226-244, 260-328, 416-441, 451-521); their f64 sums are carried here
// in f32 MFMA accumulators over exact bf16 products, with the f32 adapter activations split into a
// [hi | lo] pair of bf16 (hi = bf16(v), lo = bf16(v - hi)) wherever they enter an MFMA, so the
// adapter path keeps ~16 significant bits.
//
//   lora_down_kernel   one workgroup = 16 token rows (32 at ranks 32 and 64 on long runs) x the whole
//                      reduction, its 8 (or 4) waves an
//                      eighth (quarter) each (v_mfma_f32_16x16x32_bf16), reduced through LDS in a
//                      fixed order; the token rows are read whole-row (coalesced) and turned into
//                      MFMA fragments through the wave's LDS region; it writes the f32 result and
//                      its [hi | lo] splits for the fused kernels' epilogues (row-major) and for the
//                      gradient kernel (transposed).
//   lora_grads_kernel  dA and dB in one launch: a workgroup = 256 output columns x a token
//                      chunk; the token tile (X or dY) and the Pt rows stream through registers
//                      into two LDS slots, loaded three tiles ahead; the token tile is read back
//                      transposed with ds_read_b64_tr_b16, the [hi | lo] split of dt or s.t is
//                      the other operand; each chunk writes its own partial sums, and the last
//                      chunk of a column block to finish adds them into dA or dB in chunk order
//                      (deterministic; the leaves are added into, as the reference's rows add
//                      into the step's f32 gradients).
//   split_kernel       an f32 [T, r] operand (a cotangent handed in) -> its [hi | lo] splits.
//   lora_up_kernel     the up-projection t_cot . A of the shrink's adjoint, on its own (the fused
//                      dX kernel carries it in its epilogue when the base product runs too).
//   transpose2_kernel  B [N, r] -> B^T [rd, N] (zero rows up to the 16-wide rank) and
//                      A [r, K] -> A^T [K, r], in one launch.
//   coded_cot_kernel   the coded shrink's two cotangents from the value-space one g = t_cot . A:
//                      the code's g * scale and the scale's sum over its group of g * code.
//   coded_x_kernel     the coded activation's values x = code * scale as a [hi | lo] bf16 pair (the
//                      token operand of its dA).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "act_tiles.h"
#include "iqr_device.h"
#include "lora.h"
#include "status.h"

namespace r97q {
namespace {

typedef __bf16 bf16x8 __attribute__((__vector_size__(16)));
typedef float f32x4 __attribute__((__vector_size__(16)));
typedef short s16x4 __attribute__((__vector_size__(4 * sizeof(short))));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // a native 16-byte vector (registers)

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// hi = bf16(v), lo = bf16(v - hi): v == hi + lo to ~2^-16 relative
__device__ __forceinline__ void split(float v, uint16_t& hi, uint16_t& lo) {
    hi = f32_to_bf16(v);
    lo = f32_to_bf16(v - bf16_to_f32(hi));
}

// the two transposing reads of a B operand (k = 8g..8g+3, then 8g+4..8g+7) as one bf16x8
__device__ __forceinline__ bf16x8 tr_pair(s16x4 lo4, s16x4 hi4) {
    const uint4 w = {(uint32_t)(uint16_t)lo4[0] | ((uint32_t)(uint16_t)lo4[1] << 16),
                     (uint32_t)(uint16_t)lo4[2] | ((uint32_t)(uint16_t)lo4[3] << 16),
                     (uint32_t)(uint16_t)hi4[0] | ((uint32_t)(uint16_t)hi4[1] << 16),
                     (uint32_t)(uint16_t)hi4[2] | ((uint32_t)(uint16_t)hi4[3] << 16)};
    return as_bf16x8(w);
}

// ---------------------------------------------------------------- down
// One workgroup = 16 token rows (two blocks of 16 at ranks 32 and 64 when that still gives 256
// workgroups); its nw waves (8, or 4 when Kin is not a multiple of 256) each reduce a contiguous
// nw-th of Kin, then the partial sums are added in wave order through LDS. A 16-row block's
// products are the same whatever the workgroup's other block, so the results do not depend on
// the blocking.
//
// KM (the factor k-major, W [Kin, r] row-major: the backward's B as the caller holds it): the MFMA's
// B operand needs 8 consecutive k of one factor column, which that layout keeps r apart. Each wave
// stages its chunk of factor rows -- contiguous in memory, one coalesced 16-byte piece a lane a
// load -- into its own LDS region (rows padded to RD columns, the columns past r zero), then reads
// the operand back transposed with ds_read_b64_tr_b16, as the gradient kernel reads its token
// tile. The chunk's loads are issued with the token rows', a chunk ahead; no transpose launch.
constexpr int kDownWavesMax = 8;

// A chunk is U 32-deep slices: 128 values at rank 16, and at rank 32 with one token block; 64 at
// rank 32 with two and at rank 64 (the token rows' and the factor's registers of two chunks in
// flight stay within the wave's budget)
template <int RD, int MB>
struct DownStage {
    static constexpr int S = 2 * RD + 16;              // LDS bytes a staged factor row (16-aligned)
    static constexpr int NB = RD / 16;
    static constexpr int U = RD == 16 || (RD == 32 && MB == 1) ? 4 : 2;
    static constexpr int CH = 32 * U;                  // values (factor rows) a chunk
    static constexpr int BYTES = CH * S;               // a wave's stage
};

// The token rows of a chunk (16 MB rows x CH values) reach the MFMA layout through the wave's own
// LDS region: each load instruction reads whole row segments (RPI rows of RB bytes, 16 bytes a
// lane, every row's bytes contiguous), the wave writes them into its region and reads back the
// A-operand fragments (16 rows x 4 16-byte pieces). A row's 16-byte chunk c sits at chunk
// c ^ (row & 7): the 8 lanes an LDS cycle serves touch 8 distinct 16-byte bank groups on both
// sides. After the loop the region holds the wave's partial sums for the cross-wave reduction.
template <int RD, int MB>
struct DownTok {
    static constexpr int CH = DownStage<RD, MB>::CH;
    static constexpr int RB = 2 * CH;                  // bytes a staged row
    static constexpr int CPR = RB / 16;                // 16-byte chunks a row (32, 16 or 8)
    static constexpr int RPI = 64 / CPR;               // rows one load instruction covers
    static constexpr int NLD = 16 * MB / RPI;          // load instructions a chunk
    static constexpr int TOK = 16 * MB * RB;           // a wave's staged rows
    static constexpr int RED = 16 * MB * RD * 4;       // a wave's partial sums
    static constexpr int BYTES = TOK > RED ? TOK : RED;
    static_assert(CPR >= 8, "a staged row holds at least 8 chunks");
};

// MB token blocks of 16 rows a workgroup: two at the larger ranks when that still gives a workgroup
// to every CU (down_r), so each factor value a wave loads feeds 32 token rows (at rank 64 the
// factor is four times the token rows' bytes a chunk)
template <int RD, bool KM, int MB>
__global__ __launch_bounds__(512) void lora_down_kernel(DownArgs a) {
    using Tk = DownTok<RD, MB>;
    __shared__ __attribute__((aligned(16))) uint8_t tok_lds[kDownWavesMax * Tk::BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t stage_lds[KM ? kDownWavesMax * DownStage<RD, MB>::BYTES : 16];
    const int nw = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row16 = lane & 15, grp = lane >> 4;
    const int64_t m0 = (int64_t)blockIdx.x * 16 * MB;
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < a.nzero; i += blockDim.x) a.zero[i] = 0;
    if (a.tr_out) {
        // this workgroup's share of the side transpose: columns [c0, c1) of tr_in
        const int64_t per = (a.tr_cols + gridDim.x - 1) / gridDim.x;
        const int64_t c0 = (int64_t)blockIdx.x * per, c1 = c0 + per < a.tr_cols ? c0 + per : a.tr_cols;
        for (int64_t i = threadIdx.x; i < (c1 - c0) * a.r; i += blockDim.x) {
            const int64_t c = c0 + i / a.r;
            const int j = (int)(i % a.r);
            a.tr_out[c * a.r + j] = a.tr_in[(int64_t)j * a.tr_cols + c];
        }
    }
    const int64_t kq = a.Kin / nw;  // a multiple of 32
    const uint16_t* ap[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b) {
        int64_t row = m0 + 16 * b + row16;
        if (row > a.T - 1) row = a.T - 1;
        ap[b] = a.In + row * a.Kin + wave * kq + 8 * grp;
    }
    // the chunk loads: instruction i reads rows RPI i + lrow (clamped to T - 1), chunk lch
    uint8_t* tok = tok_lds + wave * Tk::BYTES;
    const int lrow = lane / Tk::CPR, lch = lane % Tk::CPR;
    const uint16_t* cbase = a.In + wave * kq + 8 * lch;
    auto crow = [&](int i) {
        int64_t row = m0 + Tk::RPI * i + lrow;
        return row > a.T - 1 ? a.T - 1 : row;
    };
    const uint16_t* wp = a.W + (int64_t)row16 * a.Kin + wave * kq + 8 * grp;
    constexpr int NB = RD / 16;
    // KM: the wave's stage, its factor rows from wave * kq on, and the pieces of a full chunk
    using St = DownStage<RD, MB>;
    uint8_t* stage = stage_lds + (KM ? wave * St::BYTES : 0);
    const uint16_t* wk = a.W + (int64_t)wave * kq * a.r;
    const int rb = 2 * a.r;                             // bytes a factor row in memory
    if constexpr (KM) {
        // the columns past r stay zero (never written again)
        if (a.r < RD)
            for (int i = lane; i < St::BYTES / 16; i += 64) reinterpret_cast<u32x4*>(stage)[i] = u32x4{0u, 0u, 0u, 0u};
    }
    f32x4 acc[MB][NB];
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[b][nb] = (f32x4){};
    // Chunks of U 32-deep slices (the chunk's token rows, read whole-row, and U*NB factor loads a
    // lane), two register sets: the loads of chunk c+1 are in flight while chunk c is staged and
    // multiplies.
    constexpr int U = St::U;
    constexpr int CH = St::CH;
    const int64_t nch = kq / CH;
    // the tiled copy: every value this lane loads, at the lane's true row (a row past T, up to the
    // copy's 32-row padding, is written as zeros)
    auto tile = [&](int b, int64_t k, const u32x4& v) {
        const int64_t mt = m0 + 16 * b + row16;
        if (a.tiled != nullptr && mt < (a.T + 31) / 32 * 32)
            *reinterpret_cast<u32x4*>(a.tiled + act_tile_index(mt, wave * kq + 8 * grp + k, a.T)) =
                mt < a.T ? v : u32x4{0u, 0u, 0u, 0u};
    };
    u32x4 rv[2][Tk::NLD], fv[2][U][NB];
    // KM: piece q of a lane (16 bytes) is piece lane + 64 q of the chunk's rows k .. k + rows, in
    // f's flattened slots; it lands at row (16 p) / rb, byte (16 p) % rb of the stage
    // (pieces past the chunk's rows load piece 0 again and are not stored: no predicated loads,
    // so the registers stay registers)
    auto km_load = [&](int64_t k, int rows, u32x4 (&f)[U][NB]) {
        const uint8_t* src = reinterpret_cast<const uint8_t*>(wk + k * a.r);
#pragma unroll
        for (int q = 0; q < U * NB; ++q) {
            const int p = lane + 64 * q;
            f[q / NB][q % NB] = *reinterpret_cast<const u32x4*>(src + (16 * p < rows * rb ? 16 * p : 0));
        }
    };
    auto km_store = [&](int rows, const u32x4 (&f)[U][NB]) {
#pragma unroll
        for (int q = 0; q < U * NB; ++q) {
            const int p = lane + 64 * q;
            if (16 * p < rows * rb)
                *reinterpret_cast<u32x4*>(stage + (16 * p) / rb * St::S + (16 * p) % rb) = f[q / NB][q % NB];
        }
    };
    // KM: the B operand of slice u, column block nb: rows 32u + 8grp .. +8 of the stage at column
    // 16nb + row16, read transposed
    auto km_frag = [&](int u, int nb) {
        const int e = row16 >> 2, q = row16 & 3;
        const int r0 = 32 * u + 8 * grp + e;
        const s16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(stage + r0 * St::S + (16 * nb + 4 * q) * 2));
        const s16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(stage + (r0 + 4) * St::S + (16 * nb + 4 * q) * 2));
        return tr_pair(lo4, hi4);
    };
    auto load = [&](int64_t k, u32x4 (&x)[Tk::NLD], u32x4 (&f)[U][NB]) {
#pragma unroll
        for (int i = 0; i < Tk::NLD; ++i) x[i] = *reinterpret_cast<const u32x4*>(cbase + crow(i) * a.Kin + k);
        if constexpr (KM) {
            km_load(k, CH, f);
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    f[u][nb] = *reinterpret_cast<const u32x4*>(wp + (int64_t)16 * nb * a.Kin + k + 32 * u);
        }
    };
    auto mult = [&](int64_t k, const u32x4 (&raw)[Tk::NLD], const u32x4 (&f)[U][NB]) {
        // the chunk's rows into the wave's region, then the A-operand fragments out of it
#pragma unroll
        for (int i = 0; i < Tk::NLD; ++i) {
            const int row = Tk::RPI * i + lrow;
            *reinterpret_cast<u32x4*>(tok + row * Tk::RB + ((lch ^ (row & 7)) << 4)) = raw[i];
        }
        u32x4 x[MB][U];
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int row = 16 * b + row16;
                x[b][u] = *reinterpret_cast<const u32x4*>(tok + row * Tk::RB + (((4 * u + grp) ^ (row & 7)) << 4));
            }
        if constexpr (KM) km_store(CH, f);
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const bf16x8 bv = KM ? km_frag(u, nb) : __builtin_bit_cast(bf16x8, f[u][nb]);
#pragma unroll
                for (int b = 0; b < MB; ++b) acc[b][nb] = mfma16(__builtin_bit_cast(bf16x8, x[b][u]), bv, acc[b][nb]);
            }
#pragma unroll
            for (int b = 0; b < MB; ++b) tile(b, k + 32 * u, x[b][u]);
        }
    };
    int64_t c = 0;
    if (nch > 0) load(0, rv[0], fv[0]);
    for (; c + 2 <= nch; c += 2) {
        load((c + 1) * CH, rv[1], fv[1]);
        mult(c * CH, rv[0], fv[0]);
        if (c + 2 < nch) load((c + 2) * CH, rv[0], fv[0]);
        mult((c + 1) * CH, rv[1], fv[1]);
    }
    if (c < nch) mult(c * CH, rv[0], fv[0]);  // an odd chunk count: the last one sits in set 0
    for (int64_t k = nch * CH; k < kq; k += 32) {
        bf16x8 av[MB];
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            const u32x4 xr = *reinterpret_cast<const u32x4*>(ap[b] + k);
            tile(b, k, xr);
            av[b] = __builtin_bit_cast(bf16x8, xr);
        }
        if constexpr (KM) {
            km_load(k, 32, fv[0]);
            km_store(32, fv[0]);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const bf16x8 bv = km_frag(0, nb);
#pragma unroll
                for (int b = 0; b < MB; ++b) acc[b][nb] = mfma16(av[b], bv, acc[b][nb]);
            }
        } else {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const bf16x8 bv =
                    __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(wp + (int64_t)16 * nb * a.Kin + k));
#pragma unroll
                for (int b = 0; b < MB; ++b) acc[b][nb] = mfma16(av[b], bv, acc[b][nb]);
            }
        }
    }
    // 16x16 accumulator: element e is row 4*grp + e, column row16. The partial sums go into the
    // wave's own region: its last reads of staged rows were issued before these writes (one wave's
    // LDS operations run in order), and no other wave touches the region
    auto red = [&](int w, int ml, int j) -> float& {
        return reinterpret_cast<float*>(tok_lds + w * Tk::BYTES)[ml * RD + j];
    };
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int e = 0; e < 4; ++e) red(wave, 16 * b + 4 * grp + e, 16 * nb + row16) = acc[b][nb][e];
    // The transposed splits (Pt, Pt2) go out through LDS: [2r][the workgroup's 16 MB tokens] each,
    // then a row's tokens as 16-byte stores (stored a value at a time, a wave's 2-byte stores land
    // in as many rows of Pt, ldt apart: at rank 64 that cost the backward launch 12%). They are zero
    // past T: the gradient kernel reduces over whole 32-row steps.
    constexpr int NM = 16 * MB;
    __shared__ __attribute__((aligned(16))) uint16_t tsp[2][2 * RD][NM];
    const bool tr = a.Pt != nullptr || a.Pt2 != nullptr;  // the same for the whole launch
    __syncthreads();
    for (int i = threadIdx.x; i < NM * RD; i += blockDim.x) {
        const int ml = i / RD, j = i % RD;
        const int64_t m = m0 + ml;
        if (j >= a.r) continue;
        uint16_t hi = 0, lo = 0, h2 = 0, l2 = 0;
        if (m < a.T) {
            float v = red(0, ml, j);
            for (int w = 1; w < nw; ++w) v += red(w, ml, j);
            if (a.out) a.out[m * a.r + j] = a.out_add ? a.out[m * a.r + j] + a.sa * v : a.sa * v;
            split(a.sb * v, hi, lo);
            if (a.P) {
                a.P[m * 2 * a.r + j] = hi;
                a.P[m * 2 * a.r + a.r + j] = lo;
            }
            if (a.Pt2) split(a.s2 * a.U2[m * a.r + j], h2, l2);
        }
        if (tr) {
            tsp[0][j][ml] = hi;
            tsp[0][a.r + j][ml] = lo;
            tsp[1][j][ml] = h2;
            tsp[1][a.r + j][ml] = l2;
        }
    }
    if (!tr) return;
    __syncthreads();
    // a 16-byte piece a thread: 8 tokens of one row (ldt is a multiple of 64, so a piece lies wholly
    // below it or wholly past it; rows past ldt are the tiled copy's padding only)
    const int nrow = 2 * a.r;
    for (int i = threadIdx.x; i < 2 * nrow * (NM / 8); i += blockDim.x) {
        const int which = i / (nrow * (NM / 8)), v = (i / (NM / 8)) % nrow, q = i % (NM / 8);
        uint16_t* dst = which ? a.Pt2 : a.Pt;
        const int64_t m = m0 + 8 * q;
        if (dst == nullptr || m >= a.ldt) continue;
        *reinterpret_cast<u32x4*>(dst + (int64_t)v * a.ldt + m) = *reinterpret_cast<const u32x4*>(&tsp[which][v][8 * q]);
    }
}

// ---------------------------------------------------------------- grads
// device-scope (every XCD) store and load of one f32: written through to, and read from, the
// memory all XCDs share, bypassing the XCD's own L2
__device__ __forceinline__ void device_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float device_load(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// part[chunk][j][c] = scale * sum_{m in chunk} (Pt[j][m] + Pt[r+j][m]) V[m][c]   (j < r)
// computed as C[v][c] = sum_m Pt[v][m] V[m][c] over the 2r [hi | lo] rows v; then out (+)= the
// sum of the chunks' parts in chunk order. No atomics on the values, so dA and dB are the same
// bits on every call: each workgroup counts itself done on its column block's counter (after its
// partial sums are visible device-wide), and the last of the block's chunks adds them all.
//
// A workgroup = 256 columns (8 waves x 32) x a token chunk, walked TOK tokens at a time. Tiles
// stream global -> registers -> LDS: each wave loads TOK/8 token rows of a tile (two 512-byte rows
// a load) and NP 1 KiB pieces of the tile's Pt rows (2r rows x TOK tokens); a tile is loaded three
// iterations before it is multiplied (two register sets in flight) and written to one of two LDS
// slots the iteration before. The token tile is read back transposed with ds_read_b64_tr_b16
// (the MFMA's B operand), the Pt rows straight (the A operand). Token rows are padded to 576
// bytes so the transposing reads of four consecutive rows land on distinct banks. A Pt row's
// 16-byte chunks are stored XOR-swizzled by the row (pt_chunk), so the 16 rows that 16 consecutive
// lanes read at one chunk land on all 64 banks (stored in order, rows 128 or 64 bytes apart put
// every 2nd or 4th row on the same banks).
constexpr int kGradCols = 256;
constexpr int kGradRow = 2 * kGradCols + 64;

template <int R>
struct GradShape {
    static constexpr int R2 = 2 * R;
    static constexpr int VB = R2 / 16;                  // 16-row blocks of Pt (R is 8, 16, 32 or 64)
    static constexpr int TOK = R == 64 ? 32 : 64;       // tokens a tile
    static constexpr int ROWS = TOK / 8;                // token rows a wave loads
    static constexpr int LOADS = ROWS / 2;              // two rows a load (32 lanes x 16 bytes each)
    static constexpr int PTB = R2 * TOK * 2;            // Pt bytes a tile
    static constexpr int NP = (PTB / 1024 + 7) / 8;     // 1 KiB Pt pieces a wave loads
    static constexpr int NREG = LOADS + NP;
    static constexpr int VTILE = TOK * kGradRow;
    static constexpr int SLOT = VTILE + PTB;
    static constexpr int CPR = 2 * TOK / 16;            // 16-byte chunks a Pt row (8 or 4)
};

// the LDS byte of chunk c of Pt row v in a tile: the row's chunks permuted by the row, so rows
// v and v + 16/CPR.. differ in chunk where they share banks (a row is CPR * 4 banks of 64)
template <int R>
__device__ __forceinline__ int pt_chunk(int v, int c) {
    using S = GradShape<R>;
    const int f = (v / (16 / S::CPR)) & (S::CPR - 1);
    return v * (2 * S::TOK) + 16 * (c ^ f);
}

// one lane's loads of a gradient tile: its token row halves (16 bytes each) and Pt pieces
struct GradLane {
    const uint16_t* V;
    const uint16_t* Pt;
    int64_t C, T, ldt, mb, gcol;
    int wave, lane, niter;
};

template <int R>
__device__ __forceinline__ void grad_load(const GradLane& L, int it, u32x4 (&r)[GradShape<R>::NREG]) {
    using S = GradShape<R>;
    if (it > L.niter - 1) it = L.niter - 1;  // past the chunk: its last tile again (never multiplied)
#pragma unroll
    for (int q = 0; q < S::LOADS; ++q) {  // token row ROWS*wave + 2q + (lane >= 32)
        int64_t row = L.mb + S::TOK * it + S::ROWS * L.wave + 2 * q + (L.lane >> 5);
        if (row > L.T - 1) row = L.T - 1;  // rows past T meet zero splits
        r[q] = *reinterpret_cast<const u32x4*>(L.V + row * L.C + L.gcol);
    }
    // Pt piece p (1 KiB = 64 lanes x 16 bytes): byte 1024p + 16*lane of the tile's [2r][TOK]
    // block; pieces past the block (waves with nothing to load) reload piece 0 and do not store
#pragma unroll
    for (int u = 0; u < S::NP; ++u) {
        int piece = L.wave + 8 * u;
        if (piece >= S::PTB / 1024) piece = 0;
        const int byte = 1024 * piece + 16 * L.lane;
        const int v = byte / (2 * S::TOK), m = (byte % (2 * S::TOK)) / 2;
        r[S::LOADS + u] = *reinterpret_cast<const u32x4*>(L.Pt + (int64_t)v * L.ldt + L.mb + S::TOK * it + m);
    }
}

template <int R>
__device__ __forceinline__ void grad_store(const GradLane& L, const u32x4 (&r)[GradShape<R>::NREG], uint8_t* st) {
    using S = GradShape<R>;
#pragma unroll
    for (int q = 0; q < S::LOADS; ++q)
        *reinterpret_cast<u32x4*>(st + (S::ROWS * L.wave + 2 * q + (L.lane >> 5)) * kGradRow + 16 * (L.lane & 31)) =
            r[q];
#pragma unroll
    for (int u = 0; u < S::NP; ++u) {
        const int piece = L.wave + 8 * u;
        // the lane's 16 bytes: chunk (byte % (2 TOK)) / 16 of Pt row byte / (2 TOK)
        const int byte = 1024 * piece + 16 * L.lane;
        if (piece < S::PTB / 1024)
            *reinterpret_cast<u32x4*>(st + S::VTILE + pt_chunk<R>(byte / (2 * S::TOK), (byte % (2 * S::TOK)) / 16)) =
                r[S::LOADS + u];
    }
}

template <int R>
__device__ __forceinline__ void grad_multiply(const uint8_t* st, int wave, int i16, int grp,
                                              f32x4 (&acc)[GradShape<R>::VB][2]) {
    using S = GradShape<R>;
#pragma unroll
    for (int ks = 0; ks < S::TOK / 32; ++ks) {
        bf16x8 pa[S::VB];  // lane (i, grp): Pt row 16vb + i, tokens 32ks + 8grp .. +8
#pragma unroll
        for (int vb = 0; vb < S::VB; ++vb)
            pa[vb] = as_bf16x8(
                *reinterpret_cast<const uint4*>(st + S::VTILE + pt_chunk<R>(16 * vb + i16, 4 * ks + grp)));
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const int col = 32 * wave + 16 * cb;
            const int e = i16 >> 2, q = i16 & 3;
            const s16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4*)(st + (32 * ks + 8 * grp + e) * kGradRow + (col + 4 * q) * 2));
            const s16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4*)(st + (32 * ks + 8 * grp + 4 + e) * kGradRow + (col + 4 * q) * 2));
            const bf16x8 bv = tr_pair(lo4, hi4);
#pragma unroll
            for (int vb = 0; vb < S::VB; ++vb) acc[vb][cb] = mfma16(pa[vb], bv, acc[vb][cb]);
        }
    }
}

template <int R>
__global__ __launch_bounds__(512) void lora_grads_kernel(GradArgs ga) {
    using S = GradShape<R>;
    constexpr int VB = S::VB;
    // (the `last` flag below lives in the slots' first bytes once every wave is done with them: at
    // rank 16 the slots are exactly 80 KiB, so two workgroups fit a CU)
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * S::SLOT];
    int& last = *reinterpret_cast<int*>(lds);
    const GradOne& g = ga.one[blockIdx.z];
    const int64_t C = g.C;
    const int64_t c0 = (int64_t)blockIdx.x * kGradCols;
    if (c0 >= C) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int i16 = lane & 15, grp = lane >> 4;
    const int64_t mb = (int64_t)blockIdx.y * ga.chunk;
    int64_t me = mb + ga.chunk;
    if (me > ga.ldt) me = ga.ldt;
    const int niter = (int)((me - mb) / S::TOK);
    // the lane's 8 columns of every row half it loads (columns past C read column c0 instead and
    // their results are never stored)
    const int64_t gcol = c0 + 8 * (lane & 31) < C ? c0 + 8 * (lane & 31) : c0;

    f32x4 acc[VB][2];
#pragma unroll
    for (int vb = 0; vb < VB; ++vb)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) acc[vb][cb] = (f32x4){};
    const GradLane L{g.V, g.Pt, C, ga.T, ga.ldt, mb, gcol, wave, lane, niter};
    // iteration it: multiply slot it&1, write tile it+1 (its registers) into the other slot (a
    // tile past the chunk's end goes into the slot no wave reads again), one barrier, then reload
    // those registers with tile it+3. Unrolled by two so the register sets keep fixed names.
    u32x4 ra[S::NREG], rb[S::NREG];
    grad_load<R>(L, 0, ra);
    grad_load<R>(L, 1, rb);
    grad_store<R>(L, ra, lds);
    grad_load<R>(L, 2, ra);
    __syncthreads();
    for (int it = 0; it < niter; it += 2) {
        grad_multiply<R>(lds, wave, i16, grp, acc);
        grad_store<R>(L, rb, lds + S::SLOT);
        __syncthreads();
        grad_load<R>(L, it + 3, rb);
        if (it + 1 >= niter) break;
        grad_multiply<R>(lds + S::SLOT, wave, i16, grp, acc);
        grad_store<R>(L, ra, lds);
        __syncthreads();
        grad_load<R>(L, it + 4, ra);
    }
    // acc element e of block (vb, cb): row v = 16vb + 4grp + e, column c0 + 32*wave + 16cb + i16.
    // Row j (< R) pairs with row R + j: the same lane and element VB/2 blocks on, or, for R = 8
    // (one block), the lane 32 on. The partial sums are stored at device scope (through to the
    // memory every XCD reads; no cache write-back or invalidation of the whole L2).
    // Deferred (ga.defer): plain stores, which the launch's end makes visible to the next launch.
    float* part = g.part + (int64_t)blockIdx.y * R * C;
    auto put = [&](float* p, float v) {
        if (ga.defer)
            *p = v;
        else
            device_store(p, v);
    };
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        const int64_t c = c0 + 32 * wave + 16 * cb + i16;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if constexpr (R >= 16) {
#pragma unroll
                for (int vb = 0; vb < VB / 2; ++vb) {
                    const int j = 16 * vb + 4 * grp + e;
                    if (c < C) put(part + (int64_t)j * C + c, g.scale * (acc[vb][cb][e] + acc[vb + VB / 2][cb][e]));
                }
            } else {
                const float other = __shfl_xor(acc[0][cb][e], 32);
                const int j = 4 * grp + e;
                if (grp < 2 && c < C) put(part + (int64_t)j * C + c, g.scale * (acc[0][cb][e] + other));
            }
        }
    }
    if (ga.defer) return;
    // every store of the workgroup complete (its device-scope stores acknowledged, then the
    // workgroup barrier), then the chunk counted done by one acquire-release increment at device
    // scope, whose release covers the workgroup's stores ordered before it by the barrier; the last
    // of the column block's chunks acquires the others' sums (a device-scope fence in every thread)
    // before it reads them
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(g.done + blockIdx.x, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
               (int)gridDim.y - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    // out (+)= the chunks' sums in chunk order; out is [r, C] row-major or, `transposed`, [C, r].
    // A thread takes PAIRS (j, c) pairs; their loads are issued U chunks at a time (32 in flight).
    constexpr int PAIRS = R * kGradCols / 512;
    constexpr int U = PAIRS >= 32 ? 1 : 32 / PAIRS;
    const int nch = (int)gridDim.y;
    float sum[PAIRS];
#pragma unroll
    for (int q = 0; q < PAIRS; ++q) sum[q] = 0.0f;
    for (int ch0 = 0; ch0 < nch; ch0 += U) {
        float v[PAIRS][U];
#pragma unroll
        for (int q = 0; q < PAIRS; ++q) {
            const int i = (int)threadIdx.x + 512 * q;
            const int j = i / kGradCols;
            int64_t c = c0 + i % kGradCols;
            if (c >= C) c = c0;
#pragma unroll
            for (int u = 0; u < U; ++u)
                v[q][u] = ch0 + u < nch ? device_load(g.part + ((int64_t)(ch0 + u) * R + j) * C + c) : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < PAIRS; ++q)
#pragma unroll
            for (int u = 0; u < U; ++u) sum[q] += v[q][u];
    }
#pragma unroll
    for (int q = 0; q < PAIRS; ++q) {
        const int i = (int)threadIdx.x + 512 * q;
        const int j = i / kGradCols;
        const int64_t c = c0 + i % kGradCols;
        if (c >= C) continue;
        float* d = g.transposed ? g.out + c * R + j : g.out + (int64_t)j * C + c;
        *d += sum[q];
    }
    if (threadIdx.x == 0) __hip_atomic_store(g.done + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- split and up
// P [T, 2r] = [hi | lo](s * U[m][j]) row-major, Pt [2r, ldt] the same transposed (zero for
// T <= m < ldt). One thread an (m, j), m < ldt.
__global__ __launch_bounds__(256) void split_kernel(const float* __restrict__ U, int64_t T, int r, int64_t ldt,
                                                    float s, uint16_t* __restrict__ P, uint16_t* __restrict__ Pt,
                                                    int* __restrict__ zero, int nzero) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < nzero) zero[i] = 0;
    if (i >= ldt * r) return;
    const int64_t m = i / r;
    const int j = (int)(i % r);
    uint16_t hi = 0, lo = 0;
    if (m < T) split(s * U[m * r + j], hi, lo);
    if (m < T && P) {
        P[m * 2 * r + j] = hi;
        P[m * 2 * r + r + j] = lo;
    }
    if (Pt) {
        Pt[(int64_t)j * ldt + m] = hi;
        Pt[(int64_t)(r + j) * ldt + m] = lo;
    }
}

// out[m][c] (+)= sum_{v < 2r} P[m][v] Q[c][v mod r]: the up-projection of an [hi | lo] split
// through a factor held output-major (Q = A^T [C, r] for dx = t_cot . A). A workgroup = 4 waves =
// 32 token rows x 256 columns; a wave's 32 x 64 tile is 2 x 4 v_mfma_f32_16x16x32_bf16 blocks.
__global__ __launch_bounds__(256) void lora_up_kernel(const uint16_t* __restrict__ P, const uint16_t* __restrict__ Q,
                                                      int64_t T, int64_t C, int r, float* __restrict__ out,
                                                      int accumulate) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int i16 = lane & 15, g = lane >> 4;
    const int64_t m0 = (int64_t)blockIdx.y * 32;
    const int64_t c0 = (int64_t)blockIdx.x * 256 + 64 * wave;
    if (c0 >= C) return;
    f32x4 acc[2][4];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) acc[mb][cb] = (f32x4){};
    for (int kk = 0; kk < 2 * r; kk += 32) {
        const int kq = kk + 8 * g;
        const bool live = kq < 2 * r;  // rank 8: 2r = 16 fills half of the 32-deep slice
        bf16x8 pa[2], qb[4];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            int64_t row = m0 + 16 * mb + i16;
            if (row > T - 1) row = T - 1;
            pa[mb] = as_bf16x8(live ? *reinterpret_cast<const uint4*>(P + row * 2 * r + kq) : uint4{0u, 0u, 0u, 0u});
        }
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            int64_t c = c0 + 16 * cb + i16;
            if (c > C - 1) c = C - 1;
            qb[cb] = as_bf16x8(live ? *reinterpret_cast<const uint4*>(Q + c * r + (kq % r)) : uint4{0u, 0u, 0u, 0u});
        }
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) acc[mb][cb] = mfma16(pa[mb], qb[cb], acc[mb][cb]);
    }
    // element e of block (mb, cb): row 16mb + 4g + e, column 16cb + i16
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t m = m0 + 16 * mb + 4 * g + e;
            if (m >= T) continue;
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                const int64_t c = c0 + 16 * cb + i16;
                if (c >= C) continue;
                float* d = out + m * C + c;
                *d = accumulate ? *d + acc[mb][cb][e] : acc[mb][cb][e];
            }
        }
}

// ---------------------------------------------------------------- the coded activation
// The code values: int8 codes, or f32 values (the fp8 code dtypes, decoded exactly by the caller).
__device__ __forceinline__ float code_value(const int8_t* c, int64_t i) { return (float)c[i]; }
__device__ __forceinline__ float code_value(const float* c, int64_t i) { return c[i]; }

// One workgroup a (row m, scale group q), group width gw (the last group may be short; columns past
// groups * gw, the caller's zero padding, belong to no group):
//   da[m, k] += g[m, k] * s[m, q];   ds[m, q] += sum_{k in q} g[m, k] * code[m, k]
// the sum reduced in a fixed tree order (the same bits on every call).
template <class Code>
__global__ __launch_bounds__(256) void coded_cot_kernel(const float* __restrict__ g, const Code* __restrict__ code,
                                                        const float* __restrict__ s, int64_t K, int64_t groups,
                                                        int64_t gw, float* __restrict__ da, float* __restrict__ ds) {
    __shared__ float red[256];
    const int64_t m = blockIdx.x, q = blockIdx.y;
    const float sc = s[m * groups + q];
    const int64_t k0 = q * gw, k1 = k0 + gw < K ? k0 + gw : K;
    float part = 0.0f;
    for (int64_t k = k0 + threadIdx.x; k < k1; k += blockDim.x) {
        const float gv = g[m * K + k];
        if (da) da[m * K + k] += gv * sc;
        part += gv * code_value(code, m * K + k);
    }
    if (!ds) return;
    red[threadIdx.x] = part;
    __syncthreads();
    for (int w = blockDim.x / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) ds[m * groups + q] += red[0];
}

// x[m, k] = code[m, k] * s[m, k / gw] (exact in f32 for an 8-bit code times an f32 scale: one
// rounding), as hi = bf16(x), lo = bf16(x - hi); a column past the last group takes the last group's
// scale (the caller's zero padding: x = 0)
template <class Code>
__global__ __launch_bounds__(256) void coded_x_kernel(const Code* __restrict__ code, const float* __restrict__ s,
                                                      int64_t T, int64_t K, int64_t groups, int64_t gw,
                                                      uint16_t* __restrict__ xhi, uint16_t* __restrict__ xlo) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= T * K) return;
    const int64_t m = i / K, k = i % K;
    const int64_t q = k / gw < groups ? k / gw : groups - 1;
    const float x = code_value(code, i) * s[m * groups + q];
    uint16_t hi, lo;
    split(x, hi, lo);
    xhi[i] = hi;
    xlo[i] = lo;
}

// ---------------------------------------------------------------- the tiled token operand
// dst = the fused kernels' tiled copy (act_tiles.h) of act [T, R] bf16. One workgroup a 32-row x
// 64-value block: thread t reads row t/8's 16-byte chunk t%8 (128 contiguous bytes a row) and
// writes it to lane 32*(chunk/4) + row of slice chunk%4 (128 contiguous bytes for eight rows);
// rows past T are written as zero.
__global__ __launch_bounds__(256) void act_tile_kernel(const uint16_t* __restrict__ act, int64_t T, int64_t R,
                                                       uint16_t* __restrict__ dst) {
    const int64_t s = blockIdx.x, rb = blockIdx.y;
    const int i = threadIdx.x >> 3, c = threadIdx.x & 7;
    const int64_t m = 32 * rb + i;
    uint4 v = {0u, 0u, 0u, 0u};
    if (m < T) v = *reinterpret_cast<const uint4*>(act + m * R + 64 * s + 8 * c);
    *reinterpret_cast<uint4*>(dst + ((s * (int64_t)gridDim.y + rb) * 4 + (c & 3)) * 512 + (32 * (c >> 2) + i) * 8) = v;
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
    const int nw = a.Kin % 256 == 0 ? kDownWavesMax : 4;
    // the workgroups cover the splits' ldt rows and, when the tiled copy is written, its 32-row padding
    const int64_t rows = a.tiled && (a.T + 31) / 32 * 32 > a.ldt ? (a.T + 31) / 32 * 32 : a.ldt;
    // two 16-row blocks a workgroup at ranks 32 and 64 when that leaves at least 256 workgroups
    // (one a CU; with fewer, the launch is short of memory parallelism)
    const dim3 block(64 * nw);
    if constexpr (RD >= 32) {
        if ((rows + 31) / 32 >= 256) {
            const dim3 grid((unsigned)((rows + 31) / 32));
            if (a.w_kmajor)
                hipLaunchKernelGGL((lora_down_kernel<RD, true, 2>), grid, block, 0, s, a);
            else
                hipLaunchKernelGGL((lora_down_kernel<RD, false, 2>), grid, block, 0, s, a);
            return launch_status("lora_down_kernel");
        }
    }
    const dim3 grid((unsigned)((rows + 15) / 16));
    if (a.w_kmajor)
        hipLaunchKernelGGL((lora_down_kernel<RD, true, 1>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((lora_down_kernel<RD, false, 1>), grid, block, 0, s, a);
    return launch_status("lora_down_kernel");
}

template <int R>
int grads_r(const GradArgs& g, int64_t cmax, int nz, hipStream_t s) {
    const int64_t chunks = (g.ldt + g.chunk - 1) / g.chunk;
    hipLaunchKernelGGL(lora_grads_kernel<R>, dim3((unsigned)((cmax + kGradCols - 1) / kGradCols), (unsigned)chunks,
                                                  (unsigned)nz),
                       dim3(512), 0, s, g);
    return launch_status("lora_grads_kernel");
}

}  // namespace

int down_rank(int r) { return (r + 15) / 16 * 16; }

int64_t grad_ld(int64_t T) { return (T + 63) / 64 * 64; }

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

int64_t grad_blocks(int64_t C) { return (C + kGradCols - 1) / kGradCols; }

int64_t grad_chunks(int64_t T, int64_t K, int64_t N) {
    // about 256 workgroups (one a CU) over dA's and dB's column blocks
    const int64_t cols = grad_blocks(K) + grad_blocks(N);
    int64_t chunks = (256 + cols - 1) / cols;
    const int64_t tiles = grad_ld(T) / 64;  // no chunk smaller than one 64-token tile
    if (chunks > tiles) chunks = tiles;
    return chunks < 1 ? 1 : chunks;
}

int64_t grad_chunk_rows(int64_t T, int64_t K, int64_t N) {
    const int64_t chunks = grad_chunks(T, K, N);
    const int64_t ldt = grad_ld(T);
    return ((ldt + chunks - 1) / chunks + 63) / 64 * 64;  // whole 64-token tiles
}

int launch_lora_grads(int r, const GradArgs& g, int nz, hipStream_t s) {
    const int64_t cmax = nz > 1 && g.one[1].C > g.one[0].C ? g.one[1].C : g.one[0].C;
    if (g.chunk <= 0 || g.chunk % 64 != 0) {
        set_error("lora grads: chunk %lld is not a positive multiple of 64", (long long)g.chunk);
        return R97Q_EINVAL;
    }
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

int launch_split(const float* U, int64_t T, int r, int64_t ldt, float scale, uint16_t* P, uint16_t* Pt,
                 int* zero, int nzero, hipStream_t s) {
    const int64_t n = ldt * r > nzero ? ldt * r : nzero;
    hipLaunchKernelGGL(split_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, U, T, r, ldt, scale, P,
                       Pt, zero, nzero);
    return launch_status("split_kernel");
}

int launch_lora_up(const uint16_t* P, const uint16_t* Q, int64_t T, int64_t C, int r, float* out, int accumulate,
                   hipStream_t s) {
    hipLaunchKernelGGL(lora_up_kernel, dim3((unsigned)((C + 255) / 256), (unsigned)((T + 31) / 32)), dim3(256), 0, s,
                       P, Q, T, C, r, out, accumulate);
    return launch_status("lora_up_kernel");
}

int launch_coded_cot(const float* g, const void* code, int code_f32, const float* a_scale, int64_t T, int64_t K,
                     int64_t groups, int64_t gw, float* da, float* ds, hipStream_t s) {
    const dim3 grid((unsigned)T, (unsigned)groups), block(gw >= 256 ? 256 : 128);
    if (code_f32)
        hipLaunchKernelGGL(coded_cot_kernel<float>, grid, block, 0, s, g, static_cast<const float*>(code), a_scale, K,
                           groups, gw, da, ds);
    else
        hipLaunchKernelGGL(coded_cot_kernel<int8_t>, grid, block, 0, s, g, static_cast<const int8_t*>(code), a_scale,
                           K, groups, gw, da, ds);
    return launch_status("coded_cot_kernel");
}

int launch_coded_x(const void* code, int code_f32, const float* a_scale, int64_t T, int64_t K, int64_t groups,
                   int64_t gw, uint16_t* xhi, uint16_t* xlo, hipStream_t s) {
    const dim3 grid((unsigned)((T * K + 255) / 256));
    if (code_f32)
        hipLaunchKernelGGL(coded_x_kernel<float>, grid, dim3(256), 0, s, static_cast<const float*>(code), a_scale, T,
                           K, groups, gw, xhi, xlo);
    else
        hipLaunchKernelGGL(coded_x_kernel<int8_t>, grid, dim3(256), 0, s, static_cast<const int8_t*>(code), a_scale,
                           T, K, groups, gw, xhi, xlo);
    return launch_status("coded_x_kernel");
}

int launch_act_tile(const uint16_t* act, int64_t T, int64_t R, uint16_t* dst, hipStream_t s) {
    if (R % 64 != 0 || T <= 0) {
        set_error("act tile: T %lld R %lld (R a multiple of 64)", (long long)T, (long long)R);
        return R97Q_EINVAL;
    }
    hipLaunchKernelGGL(act_tile_kernel, dim3((unsigned)(R / 64), (unsigned)((T + 31) / 32)), dim3(256), 0, s, act, T,
                       R, dst);
    return launch_status("act_tile_kernel");
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
