"""r9700training_amd -- MI355X (gfx950) IQR-quantized linear + LoRA, forward and backward.

A thin Python front over libr97q.so's C ABI (include/r97q.h). Device memory and streams come
from torch (plumbing only: every byte of arithmetic happens in the HIP kernels of csrc/). There
is no CPU fallback: when the library is missing or cannot load, every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libr97q.so")

R97Q_F32 = 0
R97Q_BF16 = 1
R97Q_I8 = 2
R97Q_F64 = 3
R97Q_PART_RMSNORM, R97Q_PART_SILU_MUL, R97Q_PART_SIGMOID_MUL = 0, 1, 2  # the fused quantisers' parts
R97Q_CODES8 = 8  # R97qWeight.bits of the int8-code form (include/r97q.h)
R97Q_DECODE_AUTO, R97Q_DECODE_ONCE, R97Q_DECODE_FUSED = 0, 1, 2  # r97q_set_decode_once modes
R97Q_ADAMW_GRADS_STAGED = 1  # r97q_adamw_step flags: the gradients are staging buffers (include/r97q.h)


class R97qError(RuntimeError):
    pass


class Desc(C.Structure):
    """R97IqrDecodeDesc (include/r97q.h), the reference's src/iqr_decode.h:59-114 layout."""

    _fields_ = [
        ("rows_all", C.c_int64), ("cols", C.c_int64), ("row0", C.c_int64), ("rows", C.c_int64),
        ("bits", C.c_int32), ("state_bits", C.c_int32), ("run_rows", C.c_int32), ("rb", C.c_int32),
        ("mad", C.c_int32), ("round_mad", C.c_int32), ("mad_a", C.c_uint32), ("mad_b", C.c_uint32),
        ("lut", C.c_void_p),
        ("codes", C.c_void_p), ("codes_row_bytes", C.c_int64),
        ("scale", C.c_void_p), ("scale_dtype", C.c_int32), ("scale_block_cols", C.c_int64),
        ("scale_row_bytes", C.c_int64),
        ("affine", C.c_int32), ("zero", C.c_void_p), ("zero_bits", C.c_int32), ("zero_row_bytes", C.c_int64),
        ("scale2", C.c_void_p), ("scale2_dtype", C.c_int32), ("scale2_row_bytes", C.c_int64),
        ("scale2_block_rows", C.c_int64), ("scale2_block_cols", C.c_int64),
        ("out_codes", C.c_void_p), ("out_scale", C.c_void_p),
    ]


class Weight(C.Structure):
    """R97qWeight (include/r97q.h): a prepared weight on the device."""

    _fields_ = [
        ("rows", C.c_int64), ("cols", C.c_int64), ("bits", C.c_int32), ("state_bits", C.c_int32),
        ("run_rows", C.c_int32), ("mad", C.c_int32), ("mad_a", C.c_uint32), ("mad_b", C.c_uint32),
        ("lut", C.c_void_p), ("stream", C.c_void_p), ("scale_t", C.c_void_p),
    ]


class AdamWConfig(C.Structure):
    """R97qAdamWConfig (include/r97q.h): the reference's AdamWConfig (include/r97/optim.h:27-40)."""

    _fields_ = [("lr", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float), ("eps", C.c_float),
                ("weight_decay", C.c_float), ("clip_norm", C.c_float), ("lr_floor_frac", C.c_float),
                ("warmup_steps", C.c_int32), ("total_steps", C.c_int32), ("accum_steps", C.c_int32)]


class AdamWParam(C.Structure):
    """R97qAdamWParam (include/r97q.h): one parameter's device buffers."""

    _fields_ = [("w", C.c_void_p), ("m", C.c_void_p), ("v", C.c_void_p), ("acc", C.c_void_p),
                ("w_bf16", C.c_void_p), ("n", C.c_int64), ("decay", C.c_int32)]


class VocabClass(C.Structure):
    """R97qVocabClass (include/r97q.h): the reference's VocabHeadClass (src/vocab_head.h:27-40)."""

    _fields_ = [("rows", C.c_int64), ("decode", Desc), ("ids", C.c_void_p), ("scale_col", C.c_void_p),
                ("scale_col_dtype", C.c_int32), ("scale_col_row_bytes", C.c_int64)]


class VocabPlan(C.Structure):
    """R97qVocabPlan (include/r97q.h): the reference's VocabHeadPlan (src/vocab_head.h:42-50)."""

    _fields_ = [("n_embd", C.c_int64), ("vocab", C.c_int64), ("vocab_offset", C.c_int64),
                ("transform", C.c_int64), ("classes", C.c_int32), ("cls", VocabClass * 4)]


R97_ENC_STR = 32
R97_ENC_MAX_PLANES = 8
# R97EncDtype (include/r97q.h)
R97_DT_U = {b: b for b in range(1, 13)}  # unsigned packed code widths 1..12
R97_DT_I8, R97_DT_U32, R97_DT_F32, R97_DT_BF16, R97_DT_F16, R97_DT_F8E4M3 = 32, 33, 34, 35, 36, 37
R97_PLANE_TILED, R97_PLANE_TABLE = 0, 1


class EncPlane(C.Structure):
    """R97EncPlane (include/r97q.h): one plane of a stored weight's encoding."""

    _fields_ = [("role", C.c_char * R97_ENC_STR), ("kind", C.c_uint32), ("dtype", C.c_uint32),
                ("block", C.c_int64 * 2), ("extent", C.c_int64 * 2)]


class Encoding(C.Structure):
    """R97Encoding (include/r97q.h): a stored weight's plane table (what AdValue::enc points at)."""

    _fields_ = [("scheme", C.c_char * R97_ENC_STR), ("transform", C.c_char * R97_ENC_STR), ("n_planes", C.c_int32),
                ("plane", EncPlane * R97_ENC_MAX_PLANES)]

    def add(self, role: str, kind: int, dtype: int, block=(0, 0), extent=(0, 0)) -> int:
        i = self.n_planes
        p = self.plane[i]
        p.role, p.kind, p.dtype = role.encode(), kind, dtype
        p.block[0], p.block[1] = block
        p.extent[0], p.extent[1] = extent
        self.n_planes = i + 1
        return i


class StoredPlane(C.Structure):
    """R97IqrStoredPlane (include/r97q.h): one plane's bytes."""

    _fields_ = [("data", C.c_void_p), ("bytes", C.c_int64)]


# every symbol include/r97q.h declares, with its ctypes signature
_P, _I, _i = C.c_void_p, C.c_int64, C.c_int32
SIGNATURES = {
    "r97q_last_error": (C.c_char_p, []),
    "r97q_iqr_validate": (C.c_int, [C.POINTER(Desc)]),
    "r97_enc_dtype_bits": (C.c_int32, [C.c_uint32]),
    "r97_enc_row_bytes": (C.c_int64, [C.c_uint32, _I]),
    "r97_enc_plane_dims": (None, [C.POINTER(EncPlane), _I, _I, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    "r97_enc_plane_bytes": (C.c_int64, [C.POINTER(EncPlane), _I, _I]),
    "r97_enc_plane_offsets": (C.c_int64, [C.POINTER(Encoding), _I, _I, C.POINTER(C.c_int64)]),
    "r97_iqr_desc_from_encoding": (C.c_int, [C.POINTER(Encoding), C.POINTER(StoredPlane), _I, _I, C.POINTER(Desc)]),
    "r97_iqr_scale_col": (C.c_int, [C.POINTER(Encoding), C.POINTER(StoredPlane), _I, _I,
                                    C.POINTER(C.POINTER(C.c_float))]),
    "r97_iqr_decode": (C.c_int, [C.POINTER(Desc), _P]),
    "r97q_weight_stream_bytes": (C.c_int64, [C.POINTER(Desc)]),
    "r97q_weight_prepare": (C.c_int, [C.POINTER(Desc), _P, _P, _P, C.POINTER(Weight), _P]),
    "r97q_weight_prepare_codes8": (C.c_int, [C.POINTER(Desc), _P, _P, _P, C.POINTER(Weight), _P]),
    "r97q_weight_from_decoded": (C.c_int, [_P, _P, _I, _I, _P, _P, C.POINTER(Weight), _P]),
    "r97q_set_decode_once": (C.c_int32, [_i]),
    "r97q_fwd_workspace_bytes": (C.c_int64, [_I, _I, _I, _i]),
    "r97q_bwd_workspace_bytes": (C.c_int64, [_I, _I, _I, _i]),
    "r97q_qlinear_lora_fwd": (C.c_int, [C.POINTER(Weight), _P, _I, _P, _P, _i, C.c_float, _P, _i, _P, _P, _I, _P]),
    "r97q_qlinear_lora_fwd_noalloc_max_bytes": (C.c_int64, []),
    "r97q_qlinear_lora_fwd_noalloc": (C.c_int, [C.POINTER(Weight), _P, _I, _P, _P, _i, C.c_float, _P, _i, _P, _P]),
    "r97q_qlinear_lora_bwd": (C.c_int, [C.POINTER(Weight), _P, _P, _I, _P, _P, _i, C.c_float, _P, _P, _i, _i,
                                        _P, _P, _P, _I, _P]),
    "r97q_iqr_encode_trellis": (C.c_int, [_P, _I, _I, _i, _i, _i, C.c_uint32, C.c_uint32, _P, _P, _P, _i,
                                          C.POINTER(C.c_double)]),
    "r97q_lora_fwd_prep": (C.c_int, [_I, _I, _I, _P, _P, _i, C.c_float, _P, _P, _I, _P]),
    "r97q_qlinear_fwd_base": (C.c_int, [C.POINTER(Weight), _P, _I, _P, _i, _P, _i, _P, _I, _P]),
    "r97q_lora_bwd_prep": (C.c_int, [_I, _I, _I, _P, _P, _P, _P, _i, C.c_float, _P, _I, _P]),
    "r97q_lora_bwd_grads": (C.c_int, [_I, _I, _I, _P, _P, _i, _P, _P, _P, _I, _P]),
    "r97q_lora_shrink_bwd_workspace_bytes": (_I, [_I, _I, _i]),
    "r97q_lora_shrink_bwd": (C.c_int, [_I, _I, _P, _P, _i, _P, _P, _i, _P, _P, _I, _P]),
    "r97q_lora_expand_bwd_workspace_bytes": (_I, [_I, _I, _i]),
    "r97q_lora_expand_bwd": (C.c_int, [_I, _I, _P, _P, _i, C.c_float, _P, _P, _P, _P, _I, _P]),
    "r97q_qlinear_dx_base": (C.c_int, [C.POINTER(Weight), _P, _I, _i, _P, _i, _i, _P, _I, _P]),
    "r97q_gemm_nt_q_dx": (C.c_int, [C.POINTER(Weight), _P, _I, _P, _P, _i, _i, _P]),
    "r97q_gemm_nt_q_fwd": (C.c_int, [_P, _P, _I, _I, _P, _P, _I, _P, _i, _P]),
    "r97q_lora_shrink_q_bwd_workspace_bytes": (_I, [_I, _I, _i]),
    "r97q_lora_shrink_q_bwd": (C.c_int, [_I, _I, _P, _i, _P, _I, _I, _P, _i, _P, _P, _P, _P, _P, _I, _P]),
    "r97q_scheduled_lr": (C.c_float, [C.POINTER(AdamWConfig), _i]),
    "r97q_adamw_workspace_bytes": (_I, [C.POINTER(AdamWParam), _i]),
    "r97q_adamw_step": (C.c_int, [C.POINTER(AdamWConfig), C.POINTER(AdamWParam), C.POINTER(C.c_void_p), _i, _i,
                                  C.POINTER(C.c_int32), C.POINTER(C.c_int32), C.POINTER(C.c_int32), _P, _I, _P]),
    "r97q_f32_to_bf16": (C.c_int, [_P, _P, _I, _P]),
    "r97q_quant_act_i8g": (C.c_int, [_P, _i, _I, _I, _I, _i, _P, _P, _P]),
    "r97q_quant_act_i8g_bwd": (C.c_int, [_P, _i, _I, _I, _I, _i, _P, _P, _P, _P]),
    "r97q_fused_had_quant_i8g": (C.c_int, [_i, _P, _P, _i, _I, _I, _I, C.c_double, C.c_double, C.c_double, _P,
                                           _P, _P, _P]),
    "r97q_fused_had_quant_i8g_bwd": (C.c_int, [_i, _P, _P, _i, _I, _I, _I, C.c_double, C.c_double, C.c_double,
                                               _P, _P, _P, _P, _P, _P]),
    "r97q_vocab_head_workspace_bytes": (_I, [C.POINTER(VocabPlan), _I]),
    "r97q_vocab_head_transpose": (C.c_int, [C.POINTER(VocabPlan), _P, _I, _P, _P, _I, _P]),
    "r97q_vocab_head_cast": (C.c_int, [_P, _P, _I, _P]),
    "r97q_mfma_probe_flops": (_I, [_i]),
    "r97q_mfma_probe": (C.c_int, [_i, _i, _P, _I, _P]),
}

_lib = None


def lib():
    """The loaded libr97q.so (raises R97qError when it is missing or incomplete)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise R97qError(f"libr97q.so is not built ({LIB_PATH}); run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return lib().r97q_last_error().decode()


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise R97qError(f"{what} failed (status {rc}): {last_error()}")


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(stream=None):
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


from .qlinear import QWeight, qlinear_lora_fwd, qlinear_lora_bwd, iqr_decode  # noqa: E402,F401
