"""oracle/oracle.py -- ctypes front of the CPU checker (TEST INFRASTRUCTURE ONLY).

Loads oracle/liboracle.so (this repo's C restatement of the reference host path) and, when it was
built, oracle/_ref/libr97ref.so (the reference's own host rows). Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg import this module; the product never does.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libr97ref.so")


class Desc(C.Structure):
    """R97IqrDecodeDesc (include/r97q.h; the reference's src/iqr_decode.h:59-114), same layout."""

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


_lib = None
_ref = None
_P = C.c_void_p
_I = C.c_int64


class AdamWConfig(C.Structure):
    """AdamWConfig (include/r97/optim.h:27-40) without no_decay (a per-parameter flag here) and threads."""

    _fields_ = [("lr", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float), ("eps", C.c_float),
                ("weight_decay", C.c_float), ("clip_norm", C.c_float), ("lr_floor_frac", C.c_float),
                ("warmup_steps", C.c_int32), ("total_steps", C.c_int32), ("accum_steps", C.c_int32)]

    @staticmethod
    def make(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0, clip_norm=0.0, lr_floor_frac=0.1,
             warmup_steps=0, total_steps=0, accum_steps=1):
        return AdamWConfig(lr, beta1, beta2, eps, weight_decay, clip_norm, lr_floor_frac, warmup_steps, total_steps,
                           accum_steps)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run make -C oracle)")
        L = C.CDLL(LIB_PATH)
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_f32_to_bf16.argtypes = [C.c_float]
        L.orc_bf16_to_f32.restype = C.c_float
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_e4m3_to_f32.restype = C.c_float
        L.orc_e4m3_to_f32.argtypes = [C.c_uint8]
        L.orc_state_value.restype = C.c_int32
        L.orc_state_value.argtypes = [C.POINTER(Desc), C.c_uint32]
        L.orc_iqr_validate.restype = C.c_int32
        L.orc_iqr_validate.argtypes = [C.POINTER(Desc)]
        L.orc_iqr_decode.restype = C.c_int32
        L.orc_iqr_decode.argtypes = [C.POINTER(Desc)]
        L.orc_fold_scale_col.argtypes = [_P, _P, _I, _I, _P]
        L.orc_gemm_nt_twin.argtypes = [_I, _I, _I, _P, _P, _P, _P, _P, _I]
        L.orc_gemm_nt_adjoint.argtypes = [_I, _I, _I, _P, _P, _P, _P, _P, _I]
        L.orc_lora_shrink_twin.argtypes = [_I, _I, _I, _I, _P, _P, _P, _P]
        L.orc_lora_shrink_adjoint.argtypes = [_I, _I, _I, _I, _P, _P, _P, _P, _P, _P, C.c_int]
        L.orc_lora_expand_twin.argtypes = [_I, _I, _I, _I, _P, _P, _P, _P, C.c_int, _P]
        L.orc_lora_expand_adjoint.argtypes = [_I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, C.c_int]
        L.orc_group_width.restype = C.c_int64
        L.orc_group_width.argtypes = [_I, _I]
        L.orc_gemm_nt_q_twin.argtypes = [_I, _I, _I, _P, _P, _P, _P, _P]
        L.orc_gemm_nt_q_adjoint.argtypes = [_I, _I, _I, _P, _P, _P, _P, _P]
        L.orc_lora_shrink_q_twin.argtypes = [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P]
        L.orc_lora_shrink_q_adjoint.argtypes = [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, C.c_int]
        L.orc_scheduled_lr.restype = C.c_float
        L.orc_scheduled_lr.argtypes = [C.POINTER(AdamWConfig), C.c_int32]
        L.orc_clip_global_norm.restype = C.c_float
        L.orc_clip_global_norm.argtypes = [_P, _P, C.c_int32, C.c_float]
        L.orc_adamw_step.restype = C.c_int32
        L.orc_adamw_step.argtypes = [C.POINTER(AdamWConfig), _P, _P, _P, _P, _P, _P, C.c_int32, _P, _P, _P]
        L.orc_vocab_class_product.argtypes = [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P]
        L.orc_fwht128.argtypes = [_I, _I, _P]
        L.orc_quant_act_i8g.restype = C.c_int32
        L.orc_quant_act_i8g.argtypes = [_P, _I, _I, _I, C.c_int32, _P, _P, _P]
        L.orc_quant_act_i8g_adjoint.restype = C.c_int32
        L.orc_quant_act_i8g_adjoint.argtypes = [_P, _I, _I, _I, C.c_int32, _P, _P, _P]
        L.orc_part_twin.restype = C.c_int32
        L.orc_part_twin.argtypes = [C.c_int32, _I, _I, _P, _P, C.c_double, C.c_double, C.c_double, _P]
        L.orc_part_adjoint.restype = C.c_int32
        L.orc_part_adjoint.argtypes = [C.c_int32, _I, _I, _P, _P, _P, C.c_double, C.c_double, C.c_double, _P, _P]
        L.orc_fused_quant.restype = C.c_int32
        L.orc_fused_quant.argtypes = [C.c_int32, _I, _I, _I, _P, _P, C.c_double, C.c_double, C.c_double, _P, _P, _P]
        L.orc_fused_quant_adjoint.restype = C.c_int32
        L.orc_fused_quant_adjoint.argtypes = [C.c_int32, _I, _I, _I, _P, _P, C.c_double, C.c_double, C.c_double,
                                              _P, _P, _P, _P, _P]
        L.orc_rounded_bf16.restype = C.c_double
        L.orc_rounded_bf16.argtypes = [C.c_double]
        L.orc_thread_count.restype = C.c_int
        L.orc_set_threads.argtypes = [C.c_int]
        _lib = L
    return _lib


def ref():
    """The reference's own host rows, or None when oracle/_ref was not built."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        R = C.CDLL(REF_PATH)
        R.ref_last_error.restype = C.c_char_p
        R.ref_iqr_validate.argtypes = [C.POINTER(Desc)]
        R.ref_iqr_decode.argtypes = [C.POINTER(Desc)]
        R.ref_gemm_nt_twin.argtypes = [_I, _I, _I, _P, _P, _P, _P]
        R.ref_gemm_nt_adjoint.argtypes = [_I, _I, _I, _P, _P, _P, _P]
        R.ref_lora_shrink_twin.argtypes = [_I, _I, _I, _I, _P, _P, _P, _P]
        R.ref_lora_shrink_adjoint.argtypes = [_I, _I, _I, _I, _P, _P, _P, _P, _P, _P, C.c_int]
        R.ref_lora_expand_twin.argtypes = [_I, _I, _I, _I, _P, _P, _P, _P, C.c_int, _P]
        R.ref_lora_expand_adjoint.argtypes = [_I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, C.c_int]
        R.ref_gemm_nt_q_twin.argtypes = [_I, _I, _I, _P, _P, _P, _P, _P]
        R.ref_gemm_nt_q_adjoint.argtypes = [_I, _I, _I, _P, _P, _P, _P, _P]
        R.ref_lora_shrink_q_twin.argtypes = [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P]
        R.ref_lora_shrink_q_adjoint.argtypes = [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, C.c_int]
        R.ref_scheduled_lr.restype = C.c_float
        R.ref_scheduled_lr.argtypes = [C.POINTER(AdamWConfig), C.c_int32]
        R.ref_clip_global_norm.restype = C.c_float
        R.ref_clip_global_norm.argtypes = [_P, _I, C.c_float]
        R.ref_part_twin.argtypes = [C.c_int32, _I, _I, _P, _P, C.c_double, C.c_double, C.c_double, _P]
        R.ref_part_adjoint.argtypes = [C.c_int32, _I, _I, _P, _P, _P, C.c_double, C.c_double, C.c_double, _P, _P]
        R.ref_adamw_run.argtypes = [C.POINTER(AdamWConfig), _P, _P, C.c_int32, _P, _P, C.c_int32, _P, _P, _P, _P, _P]
        _ref = R
    return _ref


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def thread_count() -> int:
    return int(lib().orc_thread_count())


# ------------------------------------------------------------------ decode
def decode(desc: Desc, use_ref: bool = False):
    """Decode `desc` (host planes) -> (int8 [rows, cols], uint16 bf16 bits [rows, cols/128]).

    Returns None when the description is refused."""
    rows, cols = int(desc.rows), int(desc.cols)
    oc = np.zeros((rows, cols), np.int8)
    os_ = np.zeros((rows, cols // 128), np.uint16)
    d = Desc.from_buffer_copy(desc)
    d.out_codes = oc.ctypes.data
    d.out_scale = os_.ctypes.data
    L = ref() if use_ref else lib()
    fn = L.ref_iqr_decode if use_ref else L.orc_iqr_decode
    rc = fn(C.byref(d))
    if rc != 0:
        return None
    return oc, os_


def validate(desc: Desc, use_ref: bool = False) -> int:
    """The description rules; unset output pointers are given a placeholder (the rules require
    both outputs, and this call writes nothing)."""
    d = Desc.from_buffer_copy(desc)
    one = np.zeros(1, np.int64)
    if not d.out_codes:
        d.out_codes = one.ctypes.data
    if not d.out_scale:
        d.out_scale = one.ctypes.data
    return int((ref().ref_iqr_validate if use_ref else lib().orc_iqr_validate)(C.byref(d)))


def fold_scale_col(row: np.ndarray, factor: np.ndarray) -> np.ndarray:
    row = np.ascontiguousarray(row, np.float32)
    factor = np.ascontiguousarray(factor, np.float32)
    out = np.zeros((row.size, factor.size), np.uint16)
    lib().orc_fold_scale_col(_ptr(row), _ptr(factor), row.size, factor.size, _ptr(out))
    return out


# ------------------------------------------------------------------ gemm_nt
def _f64(a):
    return np.ascontiguousarray(a, np.float64)


def gemm_nt_twin(x, codes, scale, rows=None, use_ref=False):
    x = _f64(x)
    M, K = x.shape
    N = codes.shape[0]
    codes = np.ascontiguousarray(codes, np.int8)
    scale = np.ascontiguousarray(scale, np.uint16)
    y = np.zeros((M, N), np.float64)
    if use_ref:
        rc = ref().ref_gemm_nt_twin(M, N, K, _ptr(x), _ptr(codes), _ptr(scale), _ptr(y))
        if rc:
            raise RuntimeError(ref().ref_last_error().decode())
        return y
    r = None if rows is None else np.ascontiguousarray(rows, np.int64)
    lib().orc_gemm_nt_twin(M, N, K, _ptr(x), _ptr(codes), _ptr(scale), _ptr(y), _ptr(r),
                           0 if r is None else r.size)
    return y


def gemm_nt_adjoint(dy, codes, scale, dx=None, rows=None, use_ref=False):
    dy = _f64(dy)
    M, N = dy.shape
    K = codes.shape[1]
    codes = np.ascontiguousarray(codes, np.int8)
    scale = np.ascontiguousarray(scale, np.uint16)
    dx = np.zeros((M, K), np.float64) if dx is None else _f64(dx).copy()
    if use_ref:
        rc = ref().ref_gemm_nt_adjoint(M, N, K, _ptr(dy), _ptr(codes), _ptr(scale), _ptr(dx))
        if rc:
            raise RuntimeError(ref().ref_last_error().decode())
        return dx
    r = None if rows is None else np.ascontiguousarray(rows, np.int64)
    lib().orc_gemm_nt_adjoint(M, N, K, _ptr(dy), _ptr(codes), _ptr(scale), _ptr(dx), _ptr(r),
                              0 if r is None else r.size)
    return dx


# ------------------------------------------------------------------ LoRA
def lora_shrink_twin(x, slot, lora_a, use_ref=False):
    """x [M,K], slot [M], lora_a [S,R,K] -> t [M,R] (base rows left zero)."""
    x, slot, la = _f64(x), _f64(slot), _f64(lora_a)
    M, K = x.shape
    S, R, _ = la.shape
    t = np.zeros((M, R), np.float64)
    if use_ref:
        rc = ref().ref_lora_shrink_twin(M, K, R, S, _ptr(x), _ptr(slot), _ptr(la), _ptr(t))
        if rc:
            raise RuntimeError(ref().ref_last_error().decode())
        return t
    lib().orc_lora_shrink_twin(M, K, R, S, _ptr(x), _ptr(slot), _ptr(la), _ptr(t))
    return t


def lora_shrink_adjoint(x, slot, lora_a, ct, dx=None, da=None, fused=False, use_ref=False):
    x, slot, la, ct = _f64(x), _f64(slot), _f64(lora_a), _f64(ct)
    M, K = x.shape
    S, R, _ = la.shape
    dx = np.zeros((M, K), np.float64) if dx is None else _f64(dx).copy()
    rows = S * R if fused else R
    da = np.zeros((rows, K), np.float32) if da is None else np.ascontiguousarray(da, np.float32).copy()
    if use_ref:
        rc = ref().ref_lora_shrink_adjoint(M, K, R, S, _ptr(x), _ptr(slot), _ptr(la), _ptr(ct),
                                           _ptr(dx), _ptr(da), int(fused))
        if rc:
            raise RuntimeError(ref().ref_last_error().decode())
        return dx, da
    lib().orc_lora_shrink_adjoint(M, K, R, S, _ptr(x), _ptr(slot), _ptr(la), _ptr(ct), _ptr(dx),
                                  _ptr(da), int(fused))
    return dx, da


def lora_expand_twin(t, slot, lora_b, scale, y=None, mm=False, use_ref=False):
    """t [M,R], slot [M], lora_b [S,N,R], scale [S,N] -> y [M,N] (+= onto y when given)."""
    t, slot, lb = _f64(t), _f64(slot), _f64(lora_b)
    sc = None if scale is None else _f64(scale)
    M, R = t.shape
    S, N, _ = lb.shape
    out = np.zeros((M, N), np.float64) if y is None else _f64(y).copy()
    if use_ref:
        if y is not None or sc is None:
            raise ValueError("the reference driver serves the 5-operand plain-write record only")
        rc = ref().ref_lora_expand_twin(M, N, R, S, _ptr(t), _ptr(slot), _ptr(lb), _ptr(sc),
                                        int(mm), _ptr(out))
        if rc:
            raise RuntimeError(ref().ref_last_error().decode())
        return out
    lib().orc_lora_expand_twin(M, N, R, S, _ptr(t), _ptr(slot), _ptr(lb), _ptr(sc), int(mm), _ptr(out))
    return out


def lora_expand_adjoint(t, slot, lora_b, scale, cy, dt=None, db=None, fused=False, use_ref=False):
    t, slot, lb, cy = _f64(t), _f64(slot), _f64(lora_b), _f64(cy)
    sc = None if scale is None else _f64(scale)
    M, R = t.shape
    S, N, _ = lb.shape
    dt = np.zeros((M, R), np.float64) if dt is None else _f64(dt).copy()
    cols = S * R if fused else R
    db = np.zeros((N, cols), np.float32) if db is None else np.ascontiguousarray(db, np.float32).copy()
    if use_ref:
        rc = ref().ref_lora_expand_adjoint(M, N, R, S, _ptr(t), _ptr(slot), _ptr(lb), _ptr(sc),
                                           _ptr(cy), _ptr(dt), _ptr(db), int(fused))
        if rc:
            raise RuntimeError(ref().ref_last_error().decode())
        return dt, db
    lib().orc_lora_expand_adjoint(M, N, R, S, _ptr(t), _ptr(slot), _ptr(lb), _ptr(sc), _ptr(cy),
                                  _ptr(dt), _ptr(db), int(fused))
    return dt, db


# ------------------------------------------------------------------ the whole path
def qlinear_lora_reference(x, codes, scale, A, B, s, dy, rows=None):
    """The host path of one adapted linear, composed the way the walk composes its three records
    (src/backward.cpp:556-737, reverse order expand -> shrink -> gemm_nt), single adapter, all rows
    on slot 0. Returns dict(y, t, dx, dA, dB) in f64 (dA, dB f32 leaves).

    `rows` (optional) restricts the row-local outputs (y, t, dx) to those token rows; dA and dB
    need every row and are then None."""
    x = _f64(x)
    M, K = x.shape
    N = codes.shape[0]
    R = A.shape[0]
    slot = np.zeros(M, np.float64)
    scale_n = np.full((1, N), float(s), np.float64)
    la = _f64(A).reshape(1, R, K)
    lb = _f64(B).reshape(1, N, R)
    if rows is not None:
        rows = np.asarray(rows, np.int64)
        xs, dys = x[rows], _f64(dy)[rows]
        sl = np.zeros(rows.size, np.float64)
        y = gemm_nt_twin(xs, codes, scale)
        t = lora_shrink_twin(xs, sl, la)
        y = lora_expand_twin(t, sl, lb, scale_n, y=y)
        dt, _ = lora_expand_adjoint(t, sl, lb, scale_n, dys, db=None)
        dx, _ = lora_shrink_adjoint(xs, sl, la, dt)
        dx = gemm_nt_adjoint(dys, codes, scale, dx=dx)
        return dict(y=y, t=t, dx=dx, dA=None, dB=None)
    y = gemm_nt_twin(x, codes, scale)
    t = lora_shrink_twin(x, slot, la)
    y = lora_expand_twin(t, slot, lb, scale_n, y=y)
    dt, dB = lora_expand_adjoint(t, slot, lb, scale_n, dy)
    dx, dA = lora_shrink_adjoint(x, slot, la, dt)
    dx = gemm_nt_adjoint(dy, codes, scale, dx=dx)
    return dict(y=y, t=t, dx=dx, dA=dA, dB=dB)


# ------------------------------------------------------------------ the coded (i8a8h) trunk
def group_width(k: int, groups: int) -> int:
    return int(lib().orc_group_width(int(k), int(groups)))


def _check_ref(rc):
    if rc:
        raise RuntimeError(ref().ref_last_error().decode())


def gemm_nt_q_twin(a, a_scale, codes, scale, use_ref=False):
    """a [M,K] codes (f64 of integers), a_scale [M, K/128], the stored weight (codes, bf16 scale)
    -> y [M,N] = sum_g (a . code over group g) * a_scale[m,g] * scale[n,g]."""
    a, a_scale = _f64(a), _f64(a_scale)
    M, K = a.shape
    N = codes.shape[0]
    codes = np.ascontiguousarray(codes, np.int8)
    scale = np.ascontiguousarray(scale, np.uint16)
    y = np.zeros((M, N), np.float64)
    if use_ref:
        _check_ref(ref().ref_gemm_nt_q_twin(M, N, K, _ptr(a), _ptr(a_scale), _ptr(codes), _ptr(scale), _ptr(y)))
        return y
    lib().orc_gemm_nt_q_twin(M, N, K, _ptr(a), _ptr(a_scale), _ptr(codes), _ptr(scale), _ptr(y))
    return y


def gemm_nt_q_adjoint(dy, codes, scale, a_scale, da=None, use_ref=False):
    """da [M,K] += (dy . W)[m,k] * a_scale[m, k/128] (the code basis)."""
    dy, a_scale = _f64(dy), _f64(a_scale)
    M, N = dy.shape
    K = codes.shape[1]
    codes = np.ascontiguousarray(codes, np.int8)
    scale = np.ascontiguousarray(scale, np.uint16)
    da = np.zeros((M, K), np.float64) if da is None else _f64(da).copy()
    if use_ref:
        _check_ref(ref().ref_gemm_nt_q_adjoint(M, N, K, _ptr(dy), _ptr(codes), _ptr(scale), _ptr(a_scale), _ptr(da)))
        return da
    lib().orc_gemm_nt_q_adjoint(M, N, K, _ptr(dy), _ptr(codes), _ptr(scale), _ptr(a_scale), _ptr(da))
    return da


def lora_shrink_q_twin(a, a_scale, slot, lora_a, use_ref=False):
    """The coded shrink: x = a * a_scale[m, k / group_width(K, groups)]; t = x . A_s^T."""
    a, a_scale, slot, la = _f64(a), _f64(a_scale), _f64(slot), _f64(lora_a)
    M, K = a.shape
    groups = a_scale.shape[1]
    S, R, _ = la.shape
    t = np.zeros((M, R), np.float64)
    if use_ref:
        _check_ref(ref().ref_lora_shrink_q_twin(M, K, R, S, group_width(K, groups), _ptr(a), _ptr(a_scale),
                                                _ptr(slot), _ptr(la), _ptr(t)))
        return t
    lib().orc_lora_shrink_q_twin(M, K, R, S, groups, _ptr(a), _ptr(a_scale), _ptr(slot), _ptr(la), _ptr(t))
    return t


def lora_shrink_q_adjoint(a, a_scale, slot, lora_a, ct, da=None, ds=None, dA=None, fused=False, use_ref=False):
    """-> (da [M,K] code cotangent, ds [M,groups] scale cotangent, dA f32 leaf), each added into
    what is passed."""
    a, a_scale, slot, la, ct = _f64(a), _f64(a_scale), _f64(slot), _f64(lora_a), _f64(ct)
    M, K = a.shape
    groups = a_scale.shape[1]
    S, R, _ = la.shape
    da = np.zeros((M, K), np.float64) if da is None else _f64(da).copy()
    ds = np.zeros((M, groups), np.float64) if ds is None else _f64(ds).copy()
    rows = S * R if fused else R
    dA = np.zeros((rows, K), np.float32) if dA is None else np.ascontiguousarray(dA, np.float32).copy()
    if use_ref:
        _check_ref(ref().ref_lora_shrink_q_adjoint(M, K, R, S, group_width(K, groups), _ptr(a), _ptr(a_scale),
                                                   _ptr(slot), _ptr(la), _ptr(ct), _ptr(da), _ptr(ds), _ptr(dA),
                                                   int(fused)))
        return da, ds, dA
    lib().orc_lora_shrink_q_adjoint(M, K, R, S, groups, _ptr(a), _ptr(a_scale), _ptr(slot), _ptr(la), _ptr(ct),
                                    _ptr(da), _ptr(ds), _ptr(dA), int(fused))
    return da, ds, dA


# ------------------------------------------------------------------ AdamW
def _ptrs(arrays):
    return (C.c_void_p * len(arrays))(*[a.ctypes.data for a in arrays])


def scheduled_lr(cfg: AdamWConfig, step: int, use_ref=False) -> float:
    if use_ref:
        return float(ref().ref_scheduled_lr(C.byref(cfg), int(step)))
    return float(lib().orc_scheduled_lr(C.byref(cfg), int(step)))


def clip_global_norm(arrays, max_norm: float, use_ref=False):
    """-> norm; the float32 arrays are rescaled in place (the reference takes one array here)."""
    if use_ref:
        assert len(arrays) == 1
        return float(ref().ref_clip_global_norm(arrays[0].ctypes.data, arrays[0].size, float(max_norm)))
    n = np.array([a.size for a in arrays], np.int64)
    return float(lib().orc_clip_global_norm(_ptrs(arrays), _ptr(n), len(arrays), float(max_norm)))


class AdamW:
    """The oracle's Optimiser over host float32 arrays (parameters updated in place)."""

    def __init__(self, cfg: AdamWConfig, params, decay=None):
        self.cfg = cfg
        self.w = params
        self.m = [np.zeros_like(p) for p in params]
        self.v = [np.zeros_like(p) for p in params]
        self.acc = [np.zeros_like(p) for p in params]
        self.n = np.array([p.size for p in params], np.int64)
        self.decay = np.array([1] * len(params) if decay is None else decay, np.int32)
        self.step_count = C.c_int32(0)
        self.pending = C.c_int32(0)

    def step(self, grads) -> bool:
        grads = [np.ascontiguousarray(g, np.float32) for g in grads]
        return bool(lib().orc_adamw_step(C.byref(self.cfg), _ptrs(self.w), _ptrs(self.m), _ptrs(self.v),
                                         _ptrs(self.acc), _ptr(self.n), _ptr(self.decay), len(self.w), _ptrs(grads),
                                         C.byref(self.step_count), C.byref(self.pending)))


def adamw_run_ref(cfg: AdamWConfig, params, grads_per_step, decay=None):
    """The reference's Optimiser over `params` (float32 arrays, not modified) for each gradient set;
    -> (w, m, v, acc) lists and (updates, pending)."""
    n = np.array([p.size for p in params], np.int64)
    decay = np.array([1] * len(params) if decay is None else decay, np.int32)
    w = np.concatenate([p.ravel() for p in params]).astype(np.float32)
    g = np.concatenate([np.concatenate([x.ravel() for x in gs]) for gs in grads_per_step]).astype(np.float32)
    m, v, acc = np.zeros_like(w), np.zeros_like(w), np.zeros_like(w)
    upd, pend = C.c_int32(0), C.c_int32(0)
    _check_ref(ref().ref_adamw_run(C.byref(cfg), _ptr(n), _ptr(decay), len(params), _ptr(w), _ptr(g),
                                   len(grads_per_step), _ptr(m), _ptr(v), _ptr(acc), C.byref(upd), C.byref(pend)))
    split = np.cumsum(n)[:-1]
    return ([a.reshape(p.shape) for a, p in zip(np.split(w, split), params)],
            [a.reshape(p.shape) for a, p in zip(np.split(m, split), params)],
            [a.reshape(p.shape) for a, p in zip(np.split(v, split), params)],
            [a.reshape(p.shape) for a, p in zip(np.split(acc, split), params)], (upd.value, pend.value))


def vocab_head_transpose(dy_bits, classes, vocab_offset=0, transform=0, d_x=None):
    """The vocabulary head's transposed product (src/adjoint/device/vocab_head.hip:169-238) in f64:
    dy_bits uint16 bf16 bits [rows, vocab]; classes: (codes int8 [ns, K], gscale uint16 [ns, K/128],
    ids int32 [ns], cf f32 [K/128]) each; d_x f64 [rows, K] added to (zeros when None), then the
    unnormalised Hadamard over the whole of d_x when transform == 128."""
    dy_bits = np.ascontiguousarray(dy_bits, np.uint16)
    rows, vocab = dy_bits.shape
    K = classes[0][0].shape[1]
    out = np.zeros((rows, K)) if d_x is None else np.array(d_x, np.float64, copy=True, order="C")
    for codes, gscale, ids, cf in classes:
        codes = np.ascontiguousarray(codes, np.int8)
        lib().orc_vocab_class_product(rows, K, codes.shape[0], vocab, vocab_offset, _ptr(dy_bits),
                                      _ptr(np.ascontiguousarray(ids, np.int32)), _ptr(codes),
                                      _ptr(np.ascontiguousarray(gscale, np.uint16)),
                                      _ptr(np.ascontiguousarray(cf, np.float32)), _ptr(out))
    if transform == 128:
        lib().orc_fwht128(rows, K, _ptr(out))
    return out


def fwht128(x):
    """The unnormalised 128-wide Hadamard over each 128 values of the rows of x (f64 copy)."""
    out = np.array(x, np.float64, copy=True, order="C")
    lib().orc_fwht128(out.shape[0], out.shape[1], _ptr(out))
    return out


def quant_act_i8g(x, group, rotated=False):
    """quant_act_i8g / had_quant_act_i8g (src/adjoint/host/quant.cpp:208-236) on x f64 [rows, n]
    -> (codes f64, scale f64 [rows, ngrp], live uint8); None when the geometry is refused."""
    x = np.ascontiguousarray(x, np.float64)
    rows, n = x.shape
    t = group if rotated else (n if group <= 0 or group > n else group)
    ngrp = (n + t - 1) // max(t, 1)
    codes, scale = np.zeros((rows, n)), np.zeros((rows, ngrp))
    live = np.zeros((rows, n), np.uint8)
    if lib().orc_quant_act_i8g(_ptr(x), rows, n, group, int(rotated), _ptr(codes), _ptr(scale), _ptr(live)):
        return None
    return codes, scale, live


def quant_act_i8g_adjoint(x, scale, g, group, rotated=False, dx=None):
    """The straight-through adjoint (src/adjoint/host/quant.cpp:318-372): dx + W^T(live g / s)."""
    x = np.ascontiguousarray(x, np.float64)
    rows, n = x.shape
    out = np.zeros((rows, n)) if dx is None else np.array(dx, np.float64, copy=True, order="C")
    rc = lib().orc_quant_act_i8g_adjoint(_ptr(x), rows, n, group, int(rotated),
                                         _ptr(np.ascontiguousarray(scale, np.float64)),
                                         _ptr(np.ascontiguousarray(g, np.float64)), _ptr(out))
    if rc:
        raise ValueError("quant adjoint: geometry refused" if rc == 1 else "quant adjoint: non-positive scale")
    return out


# The fused quantiser producers' elementwise parts (src/adjoint/host/elementwise.cpp) and the
# producers themselves (src/adjoint/host/quant.cpp:896-1405). part: "rmsnorm" (x0 = x [rows, n],
# x1 = w [n] or None), "silu_mul" (x0 = gate_up [rows, 2n]), "sigmoid_mul" (x0 = a, x1 = b [rows, n]).
PARTS = {"rmsnorm": 0, "silu_mul": 1, "sigmoid_mul": 2}


def _part_args(part, x0, x1):
    x0 = np.ascontiguousarray(x0, np.float64)
    x1 = None if x1 is None else np.ascontiguousarray(x1, np.float64)
    rows = x0.shape[0]
    n = x0.shape[1] // 2 if part == "silu_mul" else x0.shape[1]
    return PARTS[part], rows, n, x0, x1


def _opt(a):
    return None if a is None else _ptr(a)


def part_twin(part, x0, x1=None, eps=1e-6, wadd=0.0, mult=1.0, use_ref=False):
    """y [rows, n] = the part over its inputs (f64)."""
    k, rows, n, x0, x1 = _part_args(part, x0, x1)
    y = np.zeros((rows, n))
    if use_ref:
        _check_ref(ref().ref_part_twin(k, rows, n, _ptr(x0), _opt(x1), eps, wadd, mult, _ptr(y)))
    elif lib().orc_part_twin(k, rows, n, _ptr(x0), _opt(x1), eps, wadd, mult, _ptr(y)):
        raise ValueError(f"{part}: arguments refused")
    return y


def part_adjoint(part, x0, x1, dy, eps=1e-6, wadd=0.0, mult=1.0, use_ref=False):
    """(dx0, dx1): the part's adjoint of dy [rows, n] (dx1 None unless sigmoid_mul)."""
    k, rows, n, x0, x1 = _part_args(part, x0, x1)
    dy = np.ascontiguousarray(dy, np.float64)
    dx0 = np.zeros(x0.shape)
    dx1 = np.zeros((rows, n)) if part == "sigmoid_mul" else None
    if use_ref:
        _check_ref(ref().ref_part_adjoint(k, rows, n, _ptr(x0), _opt(x1), _ptr(dy), eps, wadd, mult, _ptr(dx0),
                                          _opt(dx1)))
    elif lib().orc_part_adjoint(k, rows, n, _ptr(x0), _opt(x1), _ptr(dy), eps, wadd, mult, _ptr(dx0), _opt(dx1)):
        raise ValueError(f"{part}: arguments refused")
    return dx0, dx1


def fused_quant(part, x0, x1, group, eps=1e-6, wadd=0.0, mult=1.0):
    """(y f64 [rows, n], codes f64, scale f64 [rows, n/group]) of the fused producer."""
    k, rows, n, x0, x1 = _part_args(part, x0, x1)
    y, codes, scale = np.zeros((rows, n)), np.zeros((rows, n)), np.zeros((rows, n // max(group, 1)))
    if lib().orc_fused_quant(k, rows, n, group, _ptr(x0), _opt(x1), eps, wadd, mult, _ptr(y), _ptr(codes),
                             _ptr(scale)):
        raise ValueError(f"fused {part}: geometry refused")
    return y, codes, scale


def fused_quant_adjoint(part, x0, x1, group, scale, g_codes, g_out=None, eps=1e-6, wadd=0.0, mult=1.0):
    """(dx0, dx1) of the fused producer: the codes' cotangent through the quantiser at part(x) with
    the forward's scale, plus the output write's cotangent, then through the part."""
    k, rows, n, x0, x1 = _part_args(part, x0, x1)
    dx0 = np.zeros(x0.shape)
    dx1 = np.zeros((rows, n)) if part == "sigmoid_mul" else None
    g_out = None if g_out is None else np.ascontiguousarray(g_out, np.float64)
    rc = lib().orc_fused_quant_adjoint(k, rows, n, group, _ptr(x0), _opt(x1), eps, wadd, mult,
                                       _ptr(np.ascontiguousarray(scale, np.float64)),
                                       _ptr(np.ascontiguousarray(g_codes, np.float64)), _opt(g_out), _ptr(dx0),
                                       _opt(dx1))
    if rc:
        raise ValueError(f"fused {part} adjoint: " + ("geometry refused" if rc == 1 else "non-positive scale"))
    return dx0, dx1
