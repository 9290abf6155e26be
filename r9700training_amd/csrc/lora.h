// lora.h -- launchers of the adapter's skinny kernels (lora.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace r97q {

// v[m][j] = sum_k In[m][k] W[j][k] for m < T, j < r (W row-major [down_rank(r), Kin], rows past r
// zero; or, with w_kmajor, W row-major [Kin, r]: the factor as B is held; Kin a multiple of 128).
// Writes, each when non-null:
//   tiled              the fused kernels' tiled copy of In (act_tiles.h), rows T..32*ceil(T/32) zero
//   out [T, r] f32    = sa * v   (+= when out_add)
//   P   [T, 2r] bf16  = [hi | lo](sb * v)                    (row-major)
//   Pt  [2r, ldt] bf16 = [hi | lo](sb * v), transposed       (zero for T <= m < ldt)
//   Pt2 [2r, ldt] bf16 = [hi | lo](s2 * U2[m][j]), transposed (U2 f32 [T, r])
//   zero [nzero]      = 0 (a following gradient launch's counters)
struct DownArgs {
    const uint16_t* In;
    const uint16_t* W;
    int64_t T, Kin, ldt;
    int r;
    float sa, sb;
    float* out;
    uint16_t* P;
    uint16_t* Pt;
    const float* U2;
    float s2;
    uint16_t* Pt2;
    int out_add;  // out += (instead of =)
    uint16_t* tiled;
    int* zero;
    int nzero;
    int w_kmajor;  // W is [Kin, r] (k-major) instead of [down_rank(r), Kin]
    // a side job, when tr_out is non-null: tr_out [tr_cols, r] = tr_in^T, tr_in [r, tr_cols] (the
    // dX epilogue's A^T, written by the backward's launch instead of a launch of its own)
    const uint16_t* tr_in;
    uint16_t* tr_out;
    int64_t tr_cols;
};

// out += scale * sum_m (Pt[j][m] + Pt[r+j][m]) V[m][c]: V bf16 [T, C] (C a multiple of 128), out
// [r, C] row-major or, `transposed`, [C, r]; Pt bf16 [2r, ldt]. The token chunks' partial sums go
// to `part` (f32 [grad_chunks, r, C]) and are added into out in chunk order by the last chunk of
// each column block to finish, counted on `done` (grad_blocks(C) counters, zero at the launch --
// the launch before it clears them -- and zero again after it). With GradArgs::defer the launch
// only writes the partial sums: a later launch adds them into out (the fused dX launch does).
struct GradOne {
    const uint16_t* Pt;
    const uint16_t* V;
    int64_t C;
    float* out;
    float scale;
    int transposed;
    float* part;
    int* done;
};
struct GradArgs {
    GradOne one[2];
    int64_t T, ldt;
    int64_t chunk;  // tokens a chunk: grad_chunk_rows(T, K, N), the size the partial buffers assume
    int defer;      // write the chunks' partial sums only (no counters, no sum into out)
};

int down_rank(int r);          // r rounded up to a multiple of 16
int64_t grad_ld(int64_t T);    // the transposed splits' row length: T rounded up to 64
int64_t grad_blocks(int64_t C);  // the gradient launch's column blocks over C columns (its counters)
// the gradient launch's token chunks (at most this many) and their length in tokens, for dA over K
// columns and dB over N
int64_t grad_chunks(int64_t T, int64_t K, int64_t N);
int64_t grad_chunk_rows(int64_t T, int64_t K, int64_t N);

int launch_lora_down(const DownArgs& a, hipStream_t s);
int launch_lora_grads(int r, const GradArgs& g, int nz, hipStream_t s);
// dst = the fused kernels' tiled copy (act_tiles.h) of act [T, R] bf16 (R a multiple of 64)
int launch_act_tile(const uint16_t* act, int64_t T, int64_t R, uint16_t* dst, hipStream_t s);
int launch_transpose2(const uint16_t* B, uint16_t* Bt, int64_t N, const uint16_t* A, uint16_t* At,
                      int64_t K, int r, hipStream_t s);
// P [T, 2r] / Pt [2r, ldt] = [hi | lo](scale * U), U f32 [T, r]; either output may be null;
// zero [nzero] = 0 (a following gradient launch's counters)
int launch_split(const float* U, int64_t T, int r, int64_t ldt, float scale, uint16_t* P, uint16_t* Pt,
                 int* zero, int nzero, hipStream_t s);
// the coded activation (codes [T, K]: int8, or f32 code values when code_f32; f32 scale a_scale
// [T, groups], group width gw):
//   da [T, K] += g * a_scale;  ds [T, groups] += sum over each group of g * code  (g f32 [T, K];
//   da or ds may be null)
int launch_coded_cot(const float* g, const void* code, int code_f32, const float* a_scale, int64_t T, int64_t K,
                     int64_t groups, int64_t gw, float* da, float* ds, hipStream_t s);
//   x = code * a_scale as [hi | lo] bf16 [T, K] each
int launch_coded_x(const void* code, int code_f32, const float* a_scale, int64_t T, int64_t K, int64_t groups,
                   int64_t gw, uint16_t* xhi, uint16_t* xlo, hipStream_t s);
// out [T, C] f32 (+)= [hi | lo](P) . [Q | Q]^T: P [T, 2r] bf16, Q [C, r] bf16 (C a multiple of 128)
int launch_lora_up(const uint16_t* P, const uint16_t* Q, int64_t T, int64_t C, int r, float* out, int accumulate,
                   hipStream_t s);

}  // namespace r97q
