/* oracle/oracle.h -- CPU restatement of the reference's host path for the IQR linear + LoRA.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (r9700training_amd/) links, loads or calls
 * this. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only as
 * the checker / the reported CPU baseline, never as the thing measured or shipped.
 *
 * Every function restates one reference function (file:line in its comment) in plain C with the
 * reference's arithmetic: f64 accumulation in the reference's loop order, f32 accumulation of the
 * dA / dB leaves per term, bf16 RNE with NaN quieting, the same tail-biting seam. Parity status of
 * each function (what pins it) is listed in the header comment of oracle.c.
 */
#ifndef R97_ORACLE_H
#define R97_ORACLE_H

#include <stdint.h>

#include "../include/r97q.h"

#ifdef __cplusplus
extern "C" {
#endif

/* threads the parallel loops use: R97_THREADS when set to an integer >= 1, else min(8, hw).
 * (src/parallel.h:171-181) */
int orc_thread_count(void);
/* force a thread count (0 = back to the environment rule) */
void orc_set_threads(int n);

/* scalar formats (src/iqr_decode.h:118-188) */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t b);
float orc_f16_to_f32(uint16_t h);
float orc_e4m3_to_f32(uint8_t b);

/* the state's value (src/iqr_decode.h:205-212) */
int32_t orc_state_value(const R97IqrDecodeDesc* d, uint32_t st);

/* description rules, host decode, planes fold (src/iqr_decode.h:321-376, src/iqr_form.h:203-216) */
int32_t orc_iqr_validate(const R97IqrDecodeDesc* d);
int32_t orc_iqr_decode(const R97IqrDecodeDesc* d);
/* out_scale[r*nkb+kb] = bf16(row[r] * factor[kb]) with one rounding */
void orc_fold_scale_col(const float* row, const float* factor, int64_t rows, int64_t nkb,
                        uint16_t* out_scale);

/* gemm_nt twin over a stored weight (src/adjoint/host/linear.cpp:132-219):
 * y[m,n] = sum_k x[m,k] * code[n,k] * bf16(scale[n,k/128]), f64. `rows` (optional, n_rows
 * entries) restricts the twin to those rows m of x / y (y keeps its [M,N] shape). */
void orc_gemm_nt_twin(int64_t M, int64_t N, int64_t K, const double* x, const int8_t* codes,
                      const uint16_t* scale, double* y, const int64_t* rows, int64_t n_rows);
/* gemm_nt adjoint (src/adjoint/host/linear.cpp:221-243): dx[m,k] += sum_n dy[m,n]*W(n,k) */
void orc_gemm_nt_adjoint(int64_t M, int64_t N, int64_t K, const double* dy, const int8_t* codes,
                         const uint16_t* scale, double* dx, const int64_t* rows, int64_t n_rows);

/* float lora_shrink twin (src/adjoint/host/lora.cpp:197-244): t[m,j] = sum_k x[m,k]*A[s,j,k],
 * s = slot[m] (a row outside [0,S) is a base row and is left untouched). */
void orc_lora_shrink_twin(int64_t M, int64_t K, int64_t R, int64_t S, const double* x,
                          const double* slot, const double* lora_a, double* t);
/* float lora_shrink adjoint (src/adjoint/host/lora.cpp:260-328):
 * dx[m,k] += sum_j ct[m,j]*A[s,j,k];  dA[(fused? s*R : 0)+j, k] += (float)(ct[m,j]*x[m,k]),
 * f32 per term, rows serial. `da` may be NULL. */
void orc_lora_shrink_adjoint(int64_t M, int64_t K, int64_t R, int64_t S, const double* x,
                             const double* slot, const double* lora_a, const double* ct,
                             double* dx, float* da, int fused);
/* lora_expand twin (src/adjoint/host/lora.cpp:409-441):
 * y[m,n] (+)= scale[s,n] * sum_j t[m,j]*B[s,n,j]; round_t rounds t to bf16 first (the _mm op);
 * `scale` NULL reads 1.0. y holds the base value on entry (a zero buffer for a plain write). */
void orc_lora_expand_twin(int64_t M, int64_t N, int64_t R, int64_t S, const double* t,
                          const double* slot, const double* lora_b, const double* scale,
                          int round_t, double* y);
/* lora_expand adjoint (src/adjoint/host/lora.cpp:451-521):
 * dt[m,j] += sum_n cy[m,n]*scale[s,n]*B[s,n,j];  dB[n, (fused? s*R:0)+j] += (float)(...),
 * f32 per term. `db` may be NULL. */
void orc_lora_expand_adjoint(int64_t M, int64_t N, int64_t R, int64_t S, const double* t,
                             const double* slot, const double* lora_b, const double* scale,
                             const double* cy, double* dt, float* db, int fused);

/* bf16 rounding the _mm twin applies (src/adjoint/host/lora.cpp:127-135): no NaN quieting */
double orc_rounded_bf16(double v);

/* ---- the coded (i8a8h) trunk: int8 activation codes with an f32 scale per (row, group) ---- */

/* the width of one scale group over k columns from the stream's `groups` columns
 * (src/adjoint/host/lora.cpp:70-77): the power of two whose ceiling division gives `groups`
 * (300 over 3 -> 128), else ceil(k / groups); one group spans the row */
int64_t orc_group_width(int64_t k, int64_t groups);
/* gemm_nt_q twin over a stored weight (src/adjoint/host/linear.cpp:245-282), group 128:
 * y[m,n] = sum_g (sum_{k in g} a[m,k] code[n,k]) * a_scale[m,g] * bf16(scale[n,g]), f64 */
void orc_gemm_nt_q_twin(int64_t M, int64_t N, int64_t K, const double* a, const double* a_scale,
                        const int8_t* codes, const uint16_t* scale, double* y);
/* gemm_nt_q adjoint (src/adjoint/host/linear.cpp:284-317), the code basis:
 * da[m,k] += (sum_n dy[m,n] code[n,k] bf16(scale[n,g])) * a_scale[m,g], g = k/128 */
void orc_gemm_nt_q_adjoint(int64_t M, int64_t N, int64_t K, const double* dy, const int8_t* codes,
                           const uint16_t* scale, const double* a_scale, double* da);
/* coded lora_shrink twin (src/adjoint/host/lora.cpp:204-244): x[m,k] = a[m,k] * a_scale[m,
 * k/group], group = orc_group_width(K, groups); t[m,j] = sum_k x[m,k] A[s,j,k] */
void orc_lora_shrink_q_twin(int64_t M, int64_t K, int64_t R, int64_t S, int64_t groups,
                            const double* a, const double* a_scale, const double* slot,
                            const double* lora_a, double* t);
/* coded lora_shrink adjoint (src/adjoint/host/lora.cpp:246-328), with g = ct . A_s:
 * da[m,k] += g[m,k] a_scale[m,g(k)];  ds[m,g(k)] += g[m,k] a[m,k] (k ascending);
 * dA[(fused? s*R : 0)+j, k] += (float)(ct[m,j] x[m,k]), f32 per term, rows serial.
 * `ds` and `dA` may be NULL. */
void orc_lora_shrink_q_adjoint(int64_t M, int64_t K, int64_t R, int64_t S, int64_t groups,
                               const double* a, const double* a_scale, const double* slot,
                               const double* lora_a, const double* ct, double* da, double* ds,
                               float* dA, int fused);

/* ---- AdamW (include/r97/optim.h, src/optim.cpp) ---- */
typedef struct {
    float lr, beta1, beta2, eps, weight_decay, clip_norm, lr_floor_frac;
    int32_t warmup_steps, total_steps, accum_steps;
} OrcAdamWConfig;
/* scheduled_lr (src/optim.cpp:113-126): linear warm-up, cosine to lr*floor_frac, flat beyond */
float orc_scheduled_lr(const OrcAdamWConfig* cfg, int32_t step);
/* clip_global_norm (src/optim.cpp:131-184): the norm over the concatenation of `count` arrays,
 * one double partial per fixed 4096-element chunk summed in chunk order; rescaled in place when
 * max_norm > 0 and the norm exceeds it. Returns the norm before clipping. */
float orc_clip_global_norm(float* const* x, const int64_t* n, int32_t count, float max_norm);
/* Optimiser::step (src/optim.cpp:223-307) over `count` parameters: acc += g; every accum_steps-th
 * call the mean, the clip, the AdamW update (f32, in the reference's operation order), the buffer
 * cleared. *step is the updates done so far, *pending the calls accumulated; both advance. Returns
 * 1 when this call applied an update. decay[i] == 0 excludes parameter i from weight decay. */
int32_t orc_adamw_step(const OrcAdamWConfig* cfg, float* const* w, float* const* m, float* const* v,
                       float* const* acc, const int64_t* n, const int32_t* decay, int32_t count,
                       const float* const* g, int32_t* step, int32_t* pending);

/* quant_act_i8g / had_quant_act_i8g (src/adjoint/host/quant.cpp:150-236): x f64 [rows, n] ->
 * codes f64 [rows, n] (integers in [-127, 127]), scale f64 [rows, ngrp], live [rows, n] (1 where the
 * clamp did not engage; may be NULL). group is the record's parameter (the effective group is
 * derived as the reference does); returns 0, or 1 when the geometry is refused. */
int32_t orc_quant_act_i8g(const double* x, int64_t rows, int64_t n, int64_t group, int32_t rotated, double* codes,
                          double* scale, uint8_t* live);
/* Its straight-through adjoint (src/adjoint/host/quant.cpp:318-372): dx += W^T(live * g / s). Returns
 * 0, 1 for a refused geometry, 2 for a non-positive scale (the reference throws). */
int32_t orc_quant_act_i8g_adjoint(const double* x, int64_t rows, int64_t n, int64_t group, int32_t rotated,
                                  const double* scale, const double* g, double* dx);

/* The elementwise parts of the fused quantiser producers (src/adjoint/host/elementwise.cpp), in f64:
 *   ORC_PART_RMSNORM   x0 = x [rows, n], x1 = w [n] (NULL: no gain; wadd must then be 0):
 *                      y = x * rs * (w + wadd) * mult, rs = 1 / sqrt(mean(x^2) + eps)      (:459-541)
 *   ORC_PART_SILU_MUL  x0 = gate_up [rows, 2n]: y = silu(gate) * up                       (:278-293)
 *   ORC_PART_SIGMOID_MUL x0 = a, x1 = b [rows, n]: y = sigmoid(a) * b (act_mul, act=sigmoid) (:316-327)
 * The adjoint adds dy's cotangent into dx0 (x0's shape) and, for the sigmoid part, dx1 (b's); the
 * norm's gain is frozen (dx1 untouched). Both return 0, or 1 for an argument outside the rules. */
#define ORC_PART_RMSNORM 0
#define ORC_PART_SILU_MUL 1
#define ORC_PART_SIGMOID_MUL 2
int32_t orc_part_twin(int32_t part, int64_t rows, int64_t n, const double* x0, const double* x1, double eps,
                      double wadd, double mult, double* y);
int32_t orc_part_adjoint(int32_t part, int64_t rows, int64_t n, const double* x0, const double* x1, const double* dy,
                         double eps, double wadd, double mult, double* dx0, double* dx1);
/* rmsnorm_had_quant_i8g / gated_had_quant_i8g / gate_had_quant_i8g (src/adjoint/host/quant.cpp:
 * 896-935, 1008-1405): y = part(x) (f64 [rows, n]), then had_quant_act_i8g over y (codes, scale as
 * orc_quant_act_i8g with rotated = 1). The adjoint: e = W^T(live * g_codes / scale) at y with the
 * forward's scale, plus g_out (the output write's cotangent; may be NULL), then the part's adjoint
 * of e into dx0 / dx1. 0, 1 for a refused geometry, 2 for a non-positive scale. */
int32_t orc_fused_quant(int32_t part, int64_t rows, int64_t n, int64_t group, const double* x0, const double* x1,
                        double eps, double wadd, double mult, double* y, double* codes, double* scale);
int32_t orc_fused_quant_adjoint(int32_t part, int64_t rows, int64_t n, int64_t group, const double* x0,
                                const double* x1, double eps, double wadd, double mult, const double* scale,
                                const double* g_codes, const double* g_out, double* dx0, double* dx1);

/* The vocabulary head's transposed product for one class (src/adjoint/device/vocab_head.hip:88-143,
 * the gather and the GEMV; f64 here): for every token row m and column k,
 *   d_x[m, k] += cf[k/128] * sum_n dy[m, ids[n] - vocab_offset] * gscale[n, k/128] * codes[n, k]
 * with dy bf16 [rows, vocab], codes int8 [ns, K], gscale bf16 [ns, K/128], cf [K/128]; an id outside
 * [vocab_offset, vocab_offset + vocab) contributes zero. */
void orc_vocab_class_product(int64_t rows, int64_t K, int64_t ns, int64_t vocab, int64_t vocab_offset,
                             const uint16_t* dy, const int32_t* ids, const int8_t* codes, const uint16_t* gscale,
                             const float* cf, double* d_x);
/* The unnormalised 128-wide Hadamard over each 128 columns of d_x [rows, K], in place
 * (src/adjoint/device/vocab_head.hip:145-163: the seven butterfly stages, no factor). */
void orc_fwht128(int64_t rows, int64_t K, double* d_x);

#ifdef __cplusplus
}
#endif

#endif
