"""This repo's IQR quantizer (r97q_iqr_encode_trellis, host C++) from Python: W -> trunk-form planes."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import R97qError, lib

# a trellis.mad codebook (A odd, 24 bits; B any 32 bits): any pair gives a valid stored weight
DEFAULT_MAD = (0x5A3C2B | 1, 0x8E2A7C15)


def quantize_trellis(W: np.ndarray, bits: int = 5, state_bits: int = 16, run_rows: int = 256,
                     mad=DEFAULT_MAD, threads: int = 0):
    """Quantize host f32 W [N, K] to the trunk IQR form. Returns dict(codes uint8 [N, row_bytes],
    row_scale f32 [N], col_factor f32 [K/128], mad_a, mad_b, bits, state_bits, run_rows, rel_err)."""
    W = np.ascontiguousarray(W, np.float32)
    N, K = W.shape
    row_bytes = (K * bits + 7) // 8
    codes = np.zeros((N, row_bytes), np.uint8)
    row_scale = np.zeros(N, np.float32)
    col_factor = np.zeros(K // 128, np.float32)
    err = C.c_double(0.0)
    rc = lib().r97q_iqr_encode_trellis(
        W.ctypes.data_as(C.c_void_p), N, K, bits, state_bits, run_rows, mad[0], mad[1],
        codes.ctypes.data_as(C.c_void_p), row_scale.ctypes.data_as(C.c_void_p),
        col_factor.ctypes.data_as(C.c_void_p), threads, C.byref(err))
    if rc != 0:
        raise R97qError(f"r97q_iqr_encode_trellis failed (status {rc}) for W {W.shape}, bits {bits}")
    return dict(codes=codes, row_scale=row_scale, col_factor=col_factor, mad_a=mad[0], mad_b=mad[1],
                bits=bits, state_bits=state_bits, run_rows=run_rows, rel_err=float(err.value))
