// qlinear_rt.h -- parameters and launchers of the register-fed fused IQR-decode + MFMA kernels
// (qlinear_rt.hip, compiled once per code width with -DR97Q_BITS=3..6, 8).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace r97q {
namespace rt {

constexpr int kBM = 512;      // tokens per workgroup (four waves of 128)
constexpr int kBN = 128;      // outputs per workgroup: features n (forward) or columns k (dX)
constexpr int kStep = 64;     // reduction depth per main-loop step
constexpr int kThreadsMax = 512; // at most 8 waves (two per SIMD)

// One launch of either product. The token operand `act` is the tiled copy (act_tiles.h) of X
// [T, K] (forward) or dY [T, N] (dX).
struct Params {
    const uint16_t* act;
    int64_t T, N, K;           // the weight is [N, K]
    const uint32_t* stream;
    const uint16_t* scale_t;
    uint32_t a24, b;
    int64_t run_rows;
    const uint16_t* P;         // [T, 2r] bf16: hi | lo of s.t (forward) or dt (dX); null when r = 0
    const uint16_t* Q;         // [outputs, r] bf16: B (forward) or A^T (dX)
    int rank;
    void* out;                 // Y [T, N] or dX [T, K]
    int out_f32;
    int accumulate;            // dX only: add into `out`
    int mtiles, otiles;
    // split-K (fused kernel only): tiles 0 .. nfull-1 (tokens outer, outputs inner) run whole; the
    // reduction of each of the others is dealt over `ksplit` ranges, a workgroup each, each writing
    // its f32 partial product into part [ksplit][tiles - nfull][kBM][kBN] (the adapter's epilogue
    // in range 0 only); launch_split_reduce then adds them, in range order, into `out`. ksplit 1:
    // no split (nfull = every tile), the product written into `out` directly.
    int ksplit;
    int nfull;
    float* part;
    const uint8_t* wt;         // the weight decoded once a call (launch_predecode), for launch_pd
    // dX only: the factor gradients' deferred chunk sums of the gradient launch before this one,
    // added into their outputs in chunk order, the elements spread over the launch's workgroups
    struct Sums {
        const float* part;     // [chunks, r, cols] f32; null: none
        int64_t cols;
        int chunks;
        int transposed;        // out is [cols, r] (dB) instead of [r, cols] (dA)
        float* out;
    } sums[2];
};

template <int BITS>
void launch_fwd(const Params& p, hipStream_t s);
template <int BITS>
void launch_dx(const Params& p, hipStream_t s);

// Every weight tile the product (forward when `fwd`, else dX) walks, decoded to bf16 in the LDS
// tile format, into `out` (wt_bytes(N, K) bytes); then launch_pd runs the product over them.
template <int BITS>
void launch_predecode(const Params& p, bool fwd, uint8_t* out, hipStream_t s);
void launch_pd(const Params& p, bool fwd, hipStream_t s);
// out (+)= part[0] + part[1] + ... + part[ksplit-1], in that order, over each split tile (the split
// product's partials)
void launch_split_reduce(const Params& p, bool fwd, hipStream_t s);
inline int64_t wt_bytes(int64_t N, int64_t K) { return N * K * 2; }
// The vocabulary head's dX products over the int8-code form (the int8-code build's
// qlinear_rt_vocab_kernel), grid (tiles, slices): `p` is range 0's dX product (p.act its gathered
// cotangent columns in the tiled layout, p.stream / p.scale_t its int8-code form; p.out the slices'
// f32 partials [slices][T, K]); range y's operands are y * z_act, z_w (uint32 units) and z_scale
// further on. Slice s holds the ranges first[s] .. first[s+1]-1, all of class cls[s]: a workgroup
// reduces its tile over each of them, over the weights' high halves and then their low halves, into
// one f32 accumulator, and writes it times cf[cls[s] * cf_ld + its 128-column tile] into partial s.
constexpr int kVocabSlices = 64;
struct VocabRtParams {
    Params p;
    int64_t z_act, z_w, z_scale;
    const float* cf;
    int64_t cf_ld;
    int slices;
    int first[kVocabSlices + 1];
    int cls[kVocabSlices];
};
void launch_vocab(const VocabRtParams& v, hipStream_t s);

// the fused kernel's grid for `full` whole tiles and `items` split ranges: 8 x the largest share
// of an XCD (each XCD's share of either kind rounded up; the workgroups past its share do no
// product)
inline int work_grid(int full, int items) { return 8 * ((full + 7) / 8 + (items + 7) / 8); }
// bytes of the split partials: ksplit ranges of each of the tiles past nfull
inline int64_t split_bytes(int ksplit, int64_t split_tiles) { return (int64_t)ksplit * split_tiles * kBM * kBN * 4; }

}  // namespace rt
}  // namespace r97q
