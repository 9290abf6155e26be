/* r97q.h -- C ABI of the MI355X (gfx950) IQR-quantized linear + LoRA path.
 *
 * Plain C: every argument is a pointer, a size or a flag; no C++ or torch type crosses it.
 * All device pointers are HIP device memory on the current device. Every launch is asynchronous
 * on the caller's stream (a hipStream_t passed as `R97IqrStream`, NULL = the null stream); the
 * caller synchronises. Every entry returns 0 on success or one of the R97Q_E* codes below, and
 * `r97q_last_error()` gives a one-line message for the calling thread's last failure.
 *
 * The path:  Y  = X.W^T + s.(X.A^T).B^T            (forward, t = X.A^T kept for the backward)
 *            dX = dY.W + s.(dY.B).A,  dA = s.(dY.B)^T.X,  dB = s.dY^T.t   (backward)
 * with W a frozen IQR weight [N, K] (tail-biting trellis codes down each column plus a block
 * scale), A [r, K] and B [N, r] the LoRA factors, s = alpha / r.
 */
#ifndef R97Q_H
#define R97Q_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ status codes */
#define R97Q_OK 0
#define R97Q_EINVAL 1       /* a description or size outside the rules (the reference's "1") */
#define R97Q_EUNSUPPORTED 2 /* a valid form this entry point has no kernel for */
#define R97Q_ELAUNCH 3      /* the HIP runtime refused a launch or a query */
#define R97Q_EWORKSPACE 4   /* the workspace passed is smaller than the entry point needs */

/* The last failure's message on the calling thread ("" when none). */
const char* r97q_last_error(void);

/* ------------------------------------------------------------------ the stored IQR form
 *
 * Scale element types. Same numbering as the reference's R97IqrScaleType
 * (src/iqr_decode.h:43-48), because the description below is laid out like its
 * R97IqrDecodeDesc and a caller may fill either. */
enum R97IqrScaleType {
    R97_IQR_F32 = 0,
    R97_IQR_BF16 = 1,
    R97_IQR_F8E4M3 = 2,
    R97_IQR_F16 = 3,
};

/* One stored IQR weight and one range of its output rows: field for field the reference's
 * R97IqrDecodeDesc (src/iqr_decode.h:59-114), so the struct a reference caller fills is accepted
 * unchanged. Plane pointers are DEVICE pointers for the device entry points below. `codes`,
 * `scale` (and `zero`) start at row `row0`; `lut` and `scale2` are whole planes. `out_codes` is
 * [rows, cols] int8 and `out_scale` [rows, cols/128] bf16 bits. */
typedef struct R97IqrDecodeDesc {
    int64_t rows_all;
    int64_t cols;
    int64_t row0;
    int64_t rows;

    int32_t bits;
    int32_t state_bits;
    int32_t run_rows;
    int32_t rb;

    int32_t mad;
    int32_t round_mad;
    uint32_t mad_a;
    uint32_t mad_b;
    const int8_t* lut;

    const uint8_t* codes;
    int64_t codes_row_bytes;

    const uint8_t* scale;
    int32_t scale_dtype;
    int64_t scale_block_cols;
    int64_t scale_row_bytes;

    int32_t affine;
    const uint8_t* zero;
    int32_t zero_bits;
    int64_t zero_row_bytes;

    const uint8_t* scale2;
    int32_t scale2_dtype;
    int64_t scale2_row_bytes;
    int64_t scale2_block_rows;
    int64_t scale2_block_cols;

    int8_t* out_codes;
    uint16_t* out_scale;
} R97IqrDecodeDesc;

/* The stream a launch runs on: a hipStream_t. */
typedef void* R97IqrStream;

/* 0 when `desc` is inside the decode's rules, 1 when not. Host-side check of the description
 * only (it reads no plane). Same rules as the reference's r97_iqr_validate
 * (src/iqr_decode.h:321-349). */
int r97q_iqr_validate(const R97IqrDecodeDesc* desc);

/* Decode rows [row0, row0+rows) of a stored IQR weight to the int8 grid and its bf16 scale, on
 * the card. Replaces the reference's device entry `r97_iqr_decode` (src/iqr_decode.h:386,
 * src/adjoint/device/iqr_decode.hip:47-56), same name, signature and contract: asynchronous on
 * `stream`, returns 0, or 1 when the description is outside the rules or the launch failed. */
int r97_iqr_decode(const R97IqrDecodeDesc* desc, R97IqrStream stream);

/* ------------------------------------------------------------------ the stored encoding
 *
 * How a stored weight's planes are named. The reference's tape hands a stored weight to a row as
 * AdValue{raw, enc}, with `enc` radiance's RadEncoding (the container's plane table: each plane's
 * role, kind, dtype, block and extent), and derives the decode's description from the roles
 * (src/iqr_form.h:87-217, `r97_iqr_desc_from_planes`). radiance is not part of this build, so the
 * plane table is stated here with the fields that derivation reads, and this build's rows read
 * AdValue::enc as an R97Encoding and AdValue::raw as the weight's planes joined in one device
 * buffer (each plane at the offset r97_enc_plane_offsets gives, in the encoding's plane order: the
 * canonical planes the container holds, no relayout).
 *
 * Plane dtypes: the unsigned packed code widths (1..12 bits, LSB first along a row) and the
 * element types of scales and tables. */
#define R97_ENC_STR 32
#define R97_ENC_MAX_PLANES 8
enum R97EncDtype {
    R97_DT_U1 = 1, R97_DT_U2, R97_DT_U3, R97_DT_U4, R97_DT_U5, R97_DT_U6, R97_DT_U7, R97_DT_U8,
    R97_DT_U9, R97_DT_U10, R97_DT_U11, R97_DT_U12,
    R97_DT_I8 = 32, R97_DT_U32, R97_DT_F32, R97_DT_BF16, R97_DT_F16, R97_DT_F8E4M3,
};
/* A tiled plane holds one element per block of [block[0] rows x block[1] columns] of the weight (0:
 * the whole extent); a table holds extent[0] x extent[1] elements whatever the weight's shape. */
enum R97EncPlaneKind { R97_PLANE_TILED = 0, R97_PLANE_TABLE = 1 };
typedef struct R97EncPlane {
    char role[R97_ENC_STR];  /* "codes", "scale", "trellis", "trellis.mad", "zero", "scale.1", "scale.col" */
    uint32_t kind;
    uint32_t dtype;
    int64_t block[2];
    int64_t extent[2];
} R97EncPlane;
typedef struct R97Encoding {
    char scheme[R97_ENC_STR];     /* "trellis" or "affine" */
    char transform[R97_ENC_STR];  /* "" or "fwht128" */
    int32_t n_planes;
    R97EncPlane plane[R97_ENC_MAX_PLANES];
} R97Encoding;
/* One plane's bytes as the caller holds them ({NULL, 0} when not held): the reference's
 * R97IqrStoredPlane (src/iqr_form.h:37-40). */
typedef struct R97IqrStoredPlane {
    const uint8_t* data;
    int64_t bytes;
} R97IqrStoredPlane;

/* Bits of one element of a plane dtype (0 for an unknown one). */
int32_t r97_enc_dtype_bits(uint32_t dtype);
/* Bytes of n elements of `dtype` packed along a row. */
int64_t r97_enc_row_bytes(uint32_t dtype, int64_t n);
/* A plane's element grid over a [rows, cols] weight, and its bytes. */
void r97_enc_plane_dims(const R97EncPlane* plane, int64_t rows, int64_t cols, int64_t* prows, int64_t* pcols);
int64_t r97_enc_plane_bytes(const R97EncPlane* plane, int64_t rows, int64_t cols);
/* The joined layout: offsets[i] of plane i (256-byte aligned, in plane order); returns the total
 * bytes, or -1 for an encoding with no planes or too many. */
int64_t r97_enc_plane_offsets(const R97Encoding* enc, int64_t rows, int64_t cols, int64_t* offsets);
/* The description of the whole weight [rows, cols] from `enc`'s planes (`plane[i]` is plane i's
 * bytes; the out_* fields are left NULL): 1, or 0 when the encoding is not a form the decode reads
 * or a plane it needs is missing or short. Restates r97_iqr_desc_from_planes
 * (src/iqr_form.h:87-183) rule for rule. The planes may be device planes, except "trellis.mad",
 * whose two words the description carries by value: that one is read here, so it is a host copy. */
int r97_iqr_desc_from_encoding(const R97Encoding* enc, const R97IqrStoredPlane* plane, int64_t rows, int64_t cols,
                               R97IqrDecodeDesc* out);
/* The scale.col factor the description cannot carry (src/iqr_form.h:199-216): *factor = the f32
 * plane (cols/128 values), or NULL when the encoding has none; 0 when it has one the fold refuses
 * (not f32, short, or beside a scale that is not one f32 a row). */
int r97_iqr_scale_col(const R97Encoding* enc, const R97IqrStoredPlane* plane, int64_t rows, int64_t cols,
                      const float** factor);

/* ------------------------------------------------------------------ the prepared weight
 *
 * The fused kernels read a weight in a GPU layout made once per weight (the weight is frozen):
 *   stream  : for every trellis run and every column, the column's codes in
 *             descending row order, packed LSB first, so that the trellis state of row n is the
 *             `state_bits`-wide bit window that starts at row n's code. Grouped in 32-row
 *             segments of `bits` dwords; dword d of a segment is stored for 4 consecutive columns
 *             together (one 128-bit load); r9700training_amd/csrc/iqr_device.h states the
 *             layout. Same size as the canonical codes plane: no halo is stored.
 *   scale_t : the effective bf16 scale of every (row, 128-column block), transposed to
 *             [cols/128][rows]: the block scale with scale.1 settled (src/iqr_decode.h:223-235) and
 *             the optional scale.col factor folded in with one rounding (src/iqr_form.h:203-216).
 * The trellis decode runs inside the fused kernels for trellis forms with rb = 1, the computed
 * `trellis.mad` codebook, bits 3..6, state_bits 16, any scale dtype with optional scale.1 /
 * scale.col, cols % 128 == 0, rows % 32 == 0 and run_rows % 32 == 0.
 *
 * Every other form the decode reads (a stored-LUT codebook, rb > 1 row blocks, other code widths
 * and state sizes, the affine grid) is decoded once into the int8-code form (bits =
 * R97Q_CODES8): the reference's stored weight (src/stored_weight.h:24-33: int8 codes [rows, cols]
 * and a bf16 scale a (row, 128 columns)) in the fused kernels' tiled layout, the GPU-resident
 * counterpart of the reference's unit-major device form:
 *   stream  : 32-byte units of 8 rows x 4 columns (byte 16*(c>>1) + 2*i + (c&1) is row i,
 *             column c of the unit), ordered [rows/8][cols/4]; rows * cols bytes;
 *   scale_t : as above.
 * The fused kernels multiply code x scale, rounded once to bf16, in both forms. */
#define R97Q_CODES8 8
typedef struct R97qWeight {
    int64_t rows;          /* N */
    int64_t cols;          /* K */
    int32_t bits;
    int32_t state_bits;
    int32_t run_rows;
    int32_t mad;
    uint32_t mad_a;
    uint32_t mad_b;
    const int8_t* lut;     /* device, 2^state_bits int8 values when !mad */
    const uint32_t* stream;   /* device, r97q_weight_stream_bytes() bytes */
    const uint16_t* scale_t;  /* device, (cols/128) * rows bf16 */
} R97qWeight;

/* Bytes of the stream plane for the whole weight `desc` describes (row0 = 0, rows = rows_all): the
 * trellis stream for the forms decoded inside the kernels, rows * cols for the int8-code form;
 * -1 when the description is outside the decode's rules, rows is not a multiple of 8 or cols of
 * 128 (r97q_last_error says why). */
int64_t r97q_weight_stream_bytes(const R97IqrDecodeDesc* desc);

/* Build the prepared weight from the canonical device planes `desc` points at (whole weight:
 * row0 = 0, rows = rows_all; the out_* fields are unused). `scale_col` is the optional
 * scale.col plane (cols/128 f32 on the device, NULL when the form has none). Writes `stream_out`
 * (r97q_weight_stream_bytes bytes) and `scale_t_out` ((cols/128)*rows bf16) and fills `w`: the
 * trellis stream when the kernels decode the form themselves, else the int8-code form. Replaces
 * the stored-weight put of a decoded grid (src/stored_weight.cpp:38-75) on the card. */
int r97q_weight_prepare(const R97IqrDecodeDesc* desc, const float* scale_col, uint32_t* stream_out,
                        uint16_t* scale_t_out, R97qWeight* w, R97IqrStream stream);
/* The int8-code form of any form the decode reads (r97_iqr_decode's values, tiled; the scale.col
 * fold of src/iqr_form.h:203-216 when `scale_col` is given): codes_out rows * cols bytes. */
int r97q_weight_prepare_codes8(const R97IqrDecodeDesc* desc, const float* scale_col, int8_t* codes_out,
                               uint16_t* scale_t_out, R97qWeight* w, R97IqrStream stream);
/* The int8-code form from a weight already decoded (the reference's StoredWeight,
 * src/stored_weight.h:24-33, on the card): codes int8 [rows, cols], scale bf16 [rows, cols/128];
 * rows a multiple of 8, cols of 128. The counterpart of stored_weight_put (src/stored_weight.h:37) for the kernels. */
int r97q_weight_from_decoded(const int8_t* codes, const uint16_t* scale, int64_t rows, int64_t cols,
                             int8_t* codes_out, uint16_t* scale_t_out, R97qWeight* w, R97IqrStream stream);

/* ------------------------------------------------------------------ fused forward / backward
 *
 * dtype codes for the activations the entry points write. */
#define R97Q_BF16 1
#define R97Q_F32 0

/* How the base products meet the weight (no counterpart in the reference, whose rows decode it
 * into their own buffers): R97Q_DECODE_FUSED decodes each weight tile inside the product's main
 * loop, once for every 512-token panel; R97Q_DECODE_ONCE decodes the whole weight once a call into
 * the workspace (N*K*2 more bytes) and runs the product over the decoded tiles, the same values in
 * the same order (the results are the same bits); R97Q_DECODE_AUTO (the default) takes the second
 * from 16384 tokens on, and from 8192 for weights of 8M (2^23) values or more. Process-wide;
 * returns the previous mode, or -1 for an unknown one. The
 * workspace sizes below follow the mode in force when they are asked. */
#define R97Q_DECODE_AUTO 0
#define R97Q_DECODE_ONCE 1
#define R97Q_DECODE_FUSED 2
int32_t r97q_set_decode_once(int32_t mode);

/* Workspace the forward / backward need at this shape (bytes, 256-aligned pieces inside). */
int64_t r97q_fwd_workspace_bytes(int64_t T, int64_t N, int64_t K, int32_t rank);
int64_t r97q_bwd_workspace_bytes(int64_t T, int64_t N, int64_t K, int32_t rank);

/* Forward: Y[T,N] = X[T,K].W^T + scale.t.B^T with t[T,r] = X.A^T.
 *   X bf16 [T,K]; A bf16 [r,K]; B bf16 [N,r]; rank 0 = no adapter (A, B, t_out unused).
 *   Y is written (not added to) in `y_dtype` (R97Q_BF16 or R97Q_F32).
 *   t_out f32 [T,r] receives t (the unscaled shrink), which the backward reads.
 * The base product is the reference's gemm_nt twin (src/adjoint/host/linear.cpp:193-219), the
 * adapter its lora_shrink and lora_expand twins (src/adjoint/host/lora.cpp:226-244,416-441). */
int r97q_qlinear_lora_fwd(const R97qWeight* w, const uint16_t* X, int64_t T, const uint16_t* A,
                          const uint16_t* B, int32_t rank, float scale, void* Y, int32_t y_dtype,
                          float* t_out, void* workspace, int64_t workspace_bytes,
                          R97IqrStream stream);

/* Backward of the forward above, given dY bf16 [T,N] and the forward's X and t:
 *   dX[T,K]  = dY.W + scale.(dY.B).A       written, or added to when dx_accumulate != 0,
 *                                           in `dx_dtype`;
 *   dA[r,K] += scale.(dY.B)^T.X            f32, always added to (a gradient leaf);
 *   dB[N,r] += scale.dY^T.t                f32, always added to.
 * dA and dB may be NULL to skip them. The reference's rows are gemm_nt_adjoint
 * (src/adjoint/host/linear.cpp:221-243), lora_expand_host_adjoint (lora.cpp:451-521) and the
 * float lora_shrink_host_adjoint (lora.cpp:260-328). */
int r97q_qlinear_lora_bwd(const R97qWeight* w, const uint16_t* X, const uint16_t* dY, int64_t T,
                          const uint16_t* A, const uint16_t* B, int32_t rank, float scale,
                          const float* t, void* dX, int32_t dx_dtype, int32_t dx_accumulate,
                          float* dA, float* dB, void* workspace, int64_t workspace_bytes,
                          R97IqrStream stream);

/* ------------------------------------------------------------------ the quantizer
 *
 * Quantize W [N, K] (HOST f32, row-major) to the trunk IQR form: trellis.mad codes of `bits` with
 * a `state_bits` state over tail-biting runs of `run_rows`, one f32 scale a row and one f32
 * scale.col factor a 128-column block. Outputs are host buffers: codes [N, ceil(K*bits/8)] packed
 * LSB first, row_scale [N], col_factor [K/128]; rel_err (optional) receives the decoded weight's
 * relative RMS error. threads <= 0 uses every hardware thread. The reference's quantizer
 * (radiance's libquant, absent from the reference tree) has no counterpart here to match: the
 * output is a valid stored weight of the reference's format (src/iqr_decode.h), and its error is
 * reported, not matched. */
int r97q_iqr_encode_trellis(const float* W, int64_t N, int64_t K, int32_t bits, int32_t state_bits,
                            int32_t run_rows, uint32_t mad_a, uint32_t mad_b, uint8_t* codes,
                            float* row_scale, float* col_factor, int32_t threads, double* rel_err);

/* ------------------------------------------------------------------ the stages
 *
 * The two calls above are these stages in order on one stream; a caller may issue them itself
 * (to time, overlap or reorder them). The workspace carries the adapter's activations between the
 * stages of one direction, so every stage of a direction gets the same workspace. Each is the part
 * of the reference rows named beside it.
 *
 * Forward: t = X.A^T (f32 into t_out) and the adapter operand of the fused kernel
 *          (lora_shrink_twin, src/adjoint/host/lora.cpp:226-244), and X's tiled copy in the workspace
 *          (the fused kernel's token operand). rank 0: only the tiled copy of X. */
int r97q_lora_fwd_prep(int64_t T, int64_t N, int64_t K, const uint16_t* X, const uint16_t* A,
                       int32_t rank, float scale, float* t_out, void* workspace,
                       int64_t workspace_bytes, R97IqrStream stream);
/* Forward: the fused decode + MFMA kernel, Y = X.W^T (+ scale.t.B^T read from the workspace)
 * (gemm_nt_twin + lora_expand_twin, src/adjoint/host/linear.cpp:193-219, lora.cpp:416-441). */
int r97q_qlinear_fwd_base(const R97qWeight* w, const uint16_t* X, int64_t T, const uint16_t* B,
                          int32_t rank, void* Y, int32_t y_dtype, void* workspace,
                          int64_t workspace_bytes, R97IqrStream stream);
/* Backward: dt = scale.dY.B (in the workspace, as the adapter operands of the fused dX kernel and of
 * dA) (lora_expand_host_adjoint's dt, src/adjoint/host/lora.cpp:495-506), and scale.t as dB's
 * operand: t (the forward's f32 t) is required when rank > 0 (R97Q_EINVAL without it). rank 0:
 * only the tiled copy of dY. */
int r97q_lora_bwd_prep(int64_t T, int64_t N, int64_t K, const uint16_t* dY, const uint16_t* A,
                       const uint16_t* B, const float* t, int32_t rank, float scale, void* workspace,
                       int64_t workspace_bytes, R97IqrStream stream);
/* Backward: dA += dt^T.X and dB += scale.dY^T.t (the leaves of lora_shrink_host_adjoint and
 * lora_expand_host_adjoint, src/adjoint/host/lora.cpp:316-327, 507-520), after r97q_lora_bwd_prep
 * on the same workspace (dB needs that prep to have had t). Either output may be NULL. The token
 * chunks' partial sums are added in a fixed order: repeated calls give the same bits. */
int r97q_lora_bwd_grads(int64_t T, int64_t N, int64_t K, const uint16_t* X, const uint16_t* dY,
                        int32_t rank, float* dA, float* dB, void* workspace, int64_t workspace_bytes,
                        R97IqrStream stream);
/* Backward: the fused decode + MFMA dX kernel, dX = dY.W (+ dt.A from the workspace)
 * (gemm_nt_adjoint + the shrink's dx, src/adjoint/host/linear.cpp:221-243, lora.cpp:295-315). */
int r97q_qlinear_dx_base(const R97qWeight* w, const uint16_t* dY, int64_t T, int32_t rank, void* dX,
                         int32_t dx_dtype, int32_t dx_accumulate, void* workspace,
                         int64_t workspace_bytes, R97IqrStream stream);

/* The forward with no allocation and no workspace argument. No counterpart in the reference: for
 * callers that cannot allocate or hand over device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same arguments, results and status as
 * r97q_qlinear_lora_fwd without the workspace pair; the workspace is a device array of the
 * library's own, one per GPU, of r97q_qlinear_lora_fwd_noalloc_max_bytes() bytes (48 MiB: T*K*2
 * plus T*r*4 and a little, e.g. T = K = 4096 at rank 16). A larger shape gets R97Q_EWORKSPACE.
 * Calls that overlap on one GPU share that array and race: serialise them (one stream, or events). */
int64_t r97q_qlinear_lora_fwd_noalloc_max_bytes(void);
int r97q_qlinear_lora_fwd_noalloc(const R97qWeight* w, const uint16_t* X, int64_t T, const uint16_t* A,
                                  const uint16_t* B, int32_t rank, float scale, void* Y, int32_t y_dtype,
                                  float* t_out, R97IqrStream stream);

/* ------------------------------------------------------------------ the adapter's rows on their own
 *
 * The shrink's and the expand's adjoints as separate calls, for a caller whose backward walk runs
 * them as separate rows (the reference's device rows lora_shrink_device_adjoint and
 * lora_expand_device_adjoint, src/adjoint/device/lora.hip:439-571, whose host twins are
 * src/adjoint/host/lora.cpp:260-328 and 451-521). One adapter slot, every row served; the caller
 * masks base rows by zeroing their cotangent rows.
 *
 * Shrink: dX (+)= t_cot . A (f32 [T, K]; added into when dx_accumulate) and dA += t_cot^T . X
 * (f32 [r, K]); t_cot f32 [T, r] enters the MFMAs as an [hi | lo] bf16 pair. Either output may be
 * NULL (dA needs X). */
int64_t r97q_lora_shrink_bwd_workspace_bytes(int64_t T, int64_t K, int32_t rank);
int r97q_lora_shrink_bwd(int64_t T, int64_t K, const uint16_t* X, const uint16_t* A, int32_t rank,
                         const float* t_cot, float* dX, int32_t dx_accumulate, float* dA, void* workspace,
                         int64_t workspace_bytes, R97IqrStream stream);
/* Expand: t_cot += scale . dY . B (f32 [T, r]) and dB += scale . dY^T . t (f32 [N, r]). Either
 * output may be NULL (dB needs t). */
int64_t r97q_lora_expand_bwd_workspace_bytes(int64_t T, int64_t N, int32_t rank);
int r97q_lora_expand_bwd(int64_t T, int64_t N, const uint16_t* dY, const uint16_t* B, int32_t rank, float scale,
                         const float* t, float* t_cot, float* dB, void* workspace, int64_t workspace_bytes,
                         R97IqrStream stream);

/* ------------------------------------------------------------------ the coded (i8a8h) trunk
 *
 * The activation arrives as int8 codes a [T, K] with one f32 scale a_scale [T, groups] per (row,
 * group); its value is x = a * a_scale[m, k / group_width(K, groups)] (the reference's width rule,
 * src/adjoint/host/lora.cpp:70-77). The rows differentiate in the code basis.
 *
 * gemm_nt_q's adjoint (the reference's device row gemm_nt_q_device, src/adjoint/device/linear.hip:
 * 744-760, registered for dtype i8a8h with group 128; host form src/adjoint/host/linear.cpp:
 * 284-317): dA[m, k] (+)= a_scale[m, k/128] . sum_n dY[m, n] W(n, k), the fused decode + MFMA dX
 * kernel with the scale in its epilogue (each of its 128-column output tiles is one group).
 * a_scale f32 [T, K/128]; dA f32 or bf16 [T, K], added into when accumulate. No workspace. */
int r97q_gemm_nt_q_dx(const R97qWeight* w, const uint16_t* dY, int64_t T, const float* a_scale, void* dA,
                      int32_t da_dtype, int32_t accumulate, R97IqrStream stream);
/* gemm_nt_q's twin, the coded forward (src/adjoint/host/linear.cpp:245-282, group 128 over a stored
 * weight): Y[m, n] = sum_g (sum_{k in g} a[m, k] codes[n, k]) * a_scale[m, g] * scale[n, g], with
 * a int8 [T, K] activation codes and a_scale f32 [T, K/128], and the stored weight's two grids as
 * the reference keeps them (src/stored_weight.h:24-33; r97_iqr_decode writes them, the scale.col
 * fold applied): codes int8 [N, K] row-major, scale bf16 [N, K/128]. N and K multiples of 128. The
 * group sums are exact (int8 MFMA, int32 accumulation); each group is folded into an f32
 * accumulator. Y f32 or bf16 [T, N]. No workspace. */
int r97q_gemm_nt_q_fwd(const int8_t* codes, const uint16_t* scale, int64_t N, int64_t K, const int8_t* a,
                       const float* a_scale, int64_t T, void* Y, int32_t y_dtype, R97IqrStream stream);
/* The coded lora_shrink's adjoint (the reference's device row for the coded trunk,
 * src/adjoint/device/lora.hip:437-577, registered for a coded activation; host form
 * src/adjoint/host/lora.cpp:246-328), one adapter slot, with g = t_cot . A (f32 [T, K]):
 *   da [T, K]      += g * a_scale        (the code's cotangent)
 *   ds [T, groups] += sum over each group of g * a   (the scale's cotangent)
 *   dA [r, K]      += t_cot^T . x
 * a [T, K] is int8 codes (a_dtype R97Q_I8) or f32 code values (R97Q_F32: the fp8 code dtypes, whose
 * values an f32 holds exactly). Column k belongs to group k / group_width; group_width 0 takes the
 * reference's rule group_width(K, groups). A caller serving a K that is not a multiple of 128 pads
 * a, A and da with zero columns and passes the unpadded K's width: a padded column past the last
 * group adds nothing. t_cot f32 [T, r]; any output may be NULL; K a multiple of 128. */
#define R97Q_I8 2
int64_t r97q_lora_shrink_q_bwd_workspace_bytes(int64_t T, int64_t K, int32_t rank);
int r97q_lora_shrink_q_bwd(int64_t T, int64_t K, const void* a, int32_t a_dtype, const float* a_scale, int64_t groups,
                           int64_t group_width, const uint16_t* A, int32_t rank, const float* t_cot, float* da,
                           float* ds, float* dA, void* workspace, int64_t workspace_bytes, R97IqrStream stream);

/* ------------------------------------------------------------------ the step's far side: AdamW
 *
 * The reference's Optimiser::step (src/optim.cpp:223-307; its config include/r97/optim.h:27-40) on
 * the card, over device f32 master weights, moments and accumulation buffers: each call adds the
 * gradients into the buffers; every accum_steps-th call takes the mean, clips it to clip_norm by
 * the global norm (when clip_norm > 0), applies the AdamW update at scheduled_lr(t), and clears the
 * buffers. The results are the reference host optimiser's bits: the same f32 operations in the
 * same order, the norm's double partials over the same 4096-element chunks added in chunk order.
 * No_decay names become decay = 0 on their parameters; the thread count has no counterpart.
 * An update is one elementwise launch over up to 16 parameters (two more with clipping); nothing
 * is read back to the host. */
typedef struct {
    float lr, beta1, beta2, eps, weight_decay, clip_norm, lr_floor_frac;
    int32_t warmup_steps, total_steps, accum_steps;
} R97qAdamWConfig;
typedef struct {
    float* w;    /* master weights, f32 [n] */
    float* m;    /* first moment */
    float* v;    /* second moment */
    float* acc;  /* the accumulation buffer (zero between updates) */
    uint16_t* w_bf16; /* NULL, or bf16 [n]: the updated weights' bf16 copy (RNE), written by the update */
    int64_t n;
    int32_t decay; /* 0: excluded from weight decay */
} R97qAdamWParam;
/* scheduled_lr (src/optim.cpp:113-126): the learning rate of the step-th update (1-based) */
float r97q_scheduled_lr(const R97qAdamWConfig* cfg, int32_t step);
/* the clip's workspace: its factor, then one double a 4096 elements of the parameters (-1: no
 * parameters); needed only with clip_norm > 0 */
int64_t r97q_adamw_workspace_bytes(const R97qAdamWParam* params, int32_t count);
/* One optimiser call (Optimiser::step, src/optim.cpp:223-307). grads[i]: f32 [params[i].n] on the
 * card, only read unless flags holds R97Q_ADAMW_GRADS_STAGED: then they are the device rows' f32
 * staging buffers (include/r97/grad_stage.h), each value taken as grad_stage_flush leaves it in a
 * zero-filled leaf (rounded once to bf16, src/adjoint/device/grad_stage.cpp:69-73) and the buffers
 * cleared by the call -- the flush, the leaf fill and the step in one pass. *updates (updates
 * applied so far) and *pending (calls accumulated) are the optimiser's counters, kept by the
 * caller; *applied (may be NULL) is set to 1 when this call updated. */
#define R97Q_ADAMW_GRADS_STAGED 1
int r97q_adamw_step(const R97qAdamWConfig* cfg, const R97qAdamWParam* params, float* const* grads,
                    int32_t count, int32_t flags, int32_t* updates, int32_t* pending, int32_t* applied,
                    void* workspace, int64_t workspace_bytes, R97IqrStream stream);
/* y = bf16(x) (RNE, NaN quieted), n elements: the kernels' bf16 operands from the f32 master weights */
int r97q_f32_to_bf16(const float* x, uint16_t* y, int64_t n, R97IqrStream stream);

/* ------------------------------------------------------------------ the activation quantiser
 *
 * quant_act_i8g / had_quant_act_i8g, the coded trunk's activation codes (the reference's host rows
 * src/adjoint/host/quant.cpp:179-236 and the geometry :150-177): per row of x [rows, n] (bf16 or
 * f32) and per group of `group` columns (group <= 0 or > n: one group a row; a short last group
 * when it does not divide n; rotated: the unnormalised Walsh-Hadamard transform of each group
 * first, `group` a power of two dividing n, at most 4096 here), scale = amax / 127 (1 for an
 * all-zero group), codes = clamp(rint(v / scale), -127, 127). codes int8 [rows, n], scale f32
 * [rows, ceil(n / group)]. The host rows' f64 arithmetic, so the same codes and scales. */
int r97q_quant_act_i8g(const void* x, int32_t x_dtype, int64_t rows, int64_t n, int64_t group, int32_t rotated,
                       int8_t* codes, float* scale, R97IqrStream stream);
/* The straight-through adjoint (src/adjoint/host/quant.cpp:318-372): dx f32 [rows, n] += W^T (live
 * * g / scale), g the codes' cotangent f32 [rows, n], live 0 where the clamp engaged (|v / scale| >
 * 127), scale the forward's (positive, as the forward writes it); the scale's cotangent is dropped. */
int r97q_quant_act_i8g_bwd(const void* x, int32_t x_dtype, int64_t rows, int64_t n, int64_t group, int32_t rotated,
                           const float* scale, const float* g, float* dx, R97IqrStream stream);

/* ------------------------------------------------------------------ the fused quantiser producers
 *
 * rmsnorm_had_quant_i8g, gated_had_quant_i8g and gate_had_quant_i8g: an elementwise part, then
 * had_quant_act_i8g (above, rotated) over its output y [rows, n]. The reference composes them on the
 * host (src/adjoint/host/quant.cpp:896-935, fused_twin; its card forward is radiance's, absent from
 * the reference tree) from the parts' rows (src/adjoint/host/elementwise.cpp):
 *   R97Q_PART_RMSNORM     x0 = x [rows, n], x1 = w [n]: y = x * rs * (w + wadd) * mult,
 *                         rs = 1 / sqrt(mean over the row of x^2 + eps)               (:459-541)
 *   R97Q_PART_SILU_MUL    x0 = gate_up [rows, 2n], x1 unused: y = silu(gate) * up     (:278-293)
 *   R97Q_PART_SIGMOID_MUL x0 = a, x1 = b [rows, n]: y = sigmoid(a) * b (act_mul, act=sigmoid) (:316-327)
 * x_dtype (bf16, f32 or f64) is that of x0 and x1. y is formed in f64 as the host twins form it;
 * group is a power of two of at most 1024 dividing n (the reference rows' predicate,
 * src/adjoint/device/quant.hip:129-159). codes int8 [rows, n], scale f32 [rows, n / group]; y_out
 * (may be NULL) receives y rounded to f32 and then to bf16, the output the live records write beside
 * the codes. eps, wadd and mult are the norm's (ignored by the other parts). */
#define R97Q_F64 3
#define R97Q_PART_RMSNORM 0
#define R97Q_PART_SILU_MUL 1
#define R97Q_PART_SIGMOID_MUL 2
int r97q_fused_had_quant_i8g(int32_t part, const void* x0, const void* x1, int32_t x_dtype, int64_t rows, int64_t n,
                             int64_t group, double eps, double wadd, double mult, int8_t* codes, float* scale,
                             uint16_t* y_out, R97IqrStream stream);
/* The adjoint (the reference's device rows src/adjoint/device/quant.hip:959-961, host rows
 * src/adjoint/host/quant.cpp:1008-1405): e = W^T(live * g_codes / scale) at y with the forward's
 * scale (f32 [rows, n / group]), plus g_out (the output write's cotangent f32 [rows, n]; may be
 * NULL), then the part's adjoint of e added into dx0 f32 (x0's shape: [rows, 2n] for silu_mul) and,
 * for the sigmoid part, dx1 f32 [rows, n] (b's). The norm's gain is frozen, as the reference
 * registers it: no gain cotangent. */
int r97q_fused_had_quant_i8g_bwd(int32_t part, const void* x0, const void* x1, int32_t x_dtype, int64_t rows,
                                 int64_t n, int64_t group, double eps, double wadd, double mult, const float* scale,
                                 const float* g_codes, const float* g_out, float* dx0, float* dx1,
                                 R97IqrStream stream);

/* ------------------------------------------------------------------ the vocabulary head
 *
 * The vocabulary head's transposed product (src/vocab_head.h:27-99, its kernels
 * src/adjoint/device/vocab_head.hip:82-238): for classes of IQR-coded rows, each with the
 * vocabulary ids of its rows and a per-128-column factor,
 *   d_x[rows, n_embd] += H . sum over classes c of (dy[:, ids_c] . W_c) * scale.col_c
 * with W_c the class's decoded int8 grid times its settled bf16 scale, H the unnormalised 128-wide
 * Hadamard per 128 columns when transform == 128 (applied to the whole of d_x once the classes are
 * added, as the reference does), and ids outside [vocab_offset, vocab_offset + vocab) contributing
 * zero. The same structs as the reference's VocabHeadClass / VocabHeadPlan. */
typedef struct {
    int64_t rows;
    R97IqrDecodeDesc decode;  /* the class's planes on the card; out_* unused, rows_all == rows */
    const void* ids;          /* device int32 [rows]: each row's vocabulary id */
    const void* scale_col;    /* device [n_embd/128] of scale_col_dtype (required, as the reference) */
    int32_t scale_col_dtype;  /* R97IqrScaleType */
    int64_t scale_col_row_bytes;
} R97qVocabClass;
typedef struct {
    int64_t n_embd;
    int64_t vocab;
    int64_t vocab_offset;
    int64_t transform; /* 128: fwht128, 0: none */
    int32_t classes;
    R97qVocabClass cls[4];
} R97qVocabPlan;
/* Workspace for a call over `rows` token rows (-1 when the plan is outside the rules). */
int64_t r97q_vocab_head_workspace_bytes(const R97qVocabPlan* plan, int64_t rows);
/* d_x f32 [rows, n_embd] (added to) from dy bf16 [rows, vocab]. Unlike the reference's entry it
 * does not drain the stream: its scratch is the caller's workspace. Every class's weights are
 * decoded into the workspace each call (the int8-code form, ranges of about 4096 rows), then every
 * range runs through one launch of the register-fed dX kernel with its class's scale.col in the
 * epilogue, and the launch's partial sums are added into d_x in a fixed order. */
int r97q_vocab_head_transpose(const R97qVocabPlan* plan, const uint16_t* dy, int64_t rows, float* d_x,
                              void* workspace, int64_t workspace_bytes, R97IqrStream stream);
/* dst bf16 <- src f32 (RNE, src/adjoint/device/vocab_head.hip:80-86) */
int r97q_vocab_head_cast(uint16_t* dst, const float* src, int64_t values, R97IqrStream stream);

/* ------------------------------------------------------------------ measurement
 * The card's sustained bf16 MFMA rate with nothing else to do (no counterpart in the reference; for
 * bench.py's roofline): 256 workgroups x 8 waves each issuing `iters` x 32
 * v_mfma_f32_32x32x16_bf16 over operands held in registers, random bf16 values or, with
 * zero_operands, zeros. out: out_count floats, at least 256 * 512 (the sums, so nothing is optimised
 * away); a smaller out_count is refused with R97Q_EINVAL before anything is launched. The FLOPs of
 * one launch: r97q_mfma_probe_flops(iters). */
int64_t r97q_mfma_probe_flops(int32_t iters);
int r97q_mfma_probe(int32_t iters, int32_t zero_operands, float* out, int64_t out_count, R97IqrStream stream);

#ifdef __cplusplus
}
#endif

#endif /* R97Q_H */
