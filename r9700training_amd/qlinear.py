"""The fused IQR-linear + LoRA path on device tensors (a front over include/r97q.h).

Shapes and dtypes follow the C ABI: X, dY bf16 [T, K] / [T, N]; A bf16 [r, K]; B bf16 [N, r];
t f32 [T, r]; dA f32 [r, K]; dB f32 [N, r]. Planes are uint8 device tensors.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import Desc, R97Q_BF16, R97Q_F32, R97Q_I8, Weight, _ptr, _stream, check, lib


def device_desc(planes: dict, rows: int, cols: int, fields: dict) -> Desc:
    """A description over device planes. `planes` maps codes / scale / lut / scale2 / zero to
    uint8 (or int8) device tensors; `fields` holds the scalar fields (bits, state_bits, ...)."""
    d = Desc()
    d.rows_all, d.cols, d.row0, d.rows = rows, cols, 0, rows
    for k, v in fields.items():
        setattr(d, k, v)
    for k in ("codes", "scale", "lut", "scale2", "zero"):
        t = planes.get(k)
        if t is not None:
            setattr(d, k, t.data_ptr())
    return d


def iqr_decode(desc: Desc, out_codes: torch.Tensor, out_scale: torch.Tensor, stream=None) -> None:
    """r97_iqr_decode over `desc` (device planes) into out_codes int8 [rows, cols] and out_scale
    int16 (bf16 bits) [rows, cols/128]."""
    d = Desc.from_buffer_copy(desc)
    d.out_codes = out_codes.data_ptr()
    d.out_scale = out_scale.data_ptr()
    rc = lib().r97_iqr_decode(C.byref(d), _stream(stream))
    check(rc, "r97_iqr_decode")


class QWeight:
    """A prepared IQR weight on the device (made once: the base weight is frozen): the column
    streams for the forms the kernels decode themselves, else the int8-code form (codes8=True asks
    for the int8-code form whatever the form), and the transposed effective scale."""

    def __init__(self, desc: Desc, scale_col: torch.Tensor | None = None, device="cuda", stream=None,
                 codes8=False):
        L = lib()
        d = Desc.from_buffer_copy(desc)
        self.rows, self.cols = int(d.rows_all), int(d.cols)
        nbytes = self.rows * self.cols if codes8 else L.r97q_weight_stream_bytes(C.byref(d))
        if nbytes < 0:
            check(2, "r97q_weight_stream_bytes")
        self.stream_plane = torch.empty((nbytes + 3) // 4, dtype=torch.int32, device=device)
        self.scale_t = torch.empty((self.cols // 128) * self.rows, dtype=torch.int16, device=device)
        self.w = Weight()
        self._scale_col = scale_col
        entry = "r97q_weight_prepare_codes8" if codes8 else "r97q_weight_prepare"
        rc = getattr(L, entry)(C.byref(d), _ptr(scale_col), _ptr(self.stream_plane), _ptr(self.scale_t),
                               C.byref(self.w), _stream(stream))
        check(rc, entry)

    @classmethod
    def from_decoded(cls, codes: torch.Tensor, scale: torch.Tensor, stream=None) -> "QWeight":
        """The int8-code form of a decoded weight: codes int8 [N, K], scale bf16 bits (int16 or
        uint16 storage) [N, K/128], both on the device (the reference's StoredWeight)."""
        if codes.dtype != torch.int8 or codes.dim() != 2 or not codes.is_contiguous():
            raise ValueError("QWeight.from_decoded: codes are a contiguous int8 [N, K] tensor")
        N, K = codes.shape
        if scale.element_size() != 2 or scale.numel() != N * (K // 128) or not scale.is_contiguous():
            raise ValueError("QWeight.from_decoded: scale holds N * K/128 bf16 values")
        self = cls.__new__(cls)
        self.rows, self.cols = int(N), int(K)
        self.stream_plane = torch.empty((N * K + 3) // 4, dtype=torch.int32, device=codes.device)
        self.scale_t = torch.empty((K // 128) * N, dtype=torch.int16, device=codes.device)
        self.w = Weight()
        self._scale_col = None
        check(lib().r97q_weight_from_decoded(_ptr(codes), _ptr(scale), N, K, _ptr(self.stream_plane),
                                             _ptr(self.scale_t), C.byref(self.w), _stream(stream)),
              "r97q_weight_from_decoded")
        return self

    @property
    def codes8(self) -> bool:
        return self.w.bits == 8

    @property
    def N(self):
        return self.rows

    @property
    def K(self):
        return self.cols


def fwd_workspace(T, N, K, rank, device="cuda"):
    n = lib().r97q_fwd_workspace_bytes(T, N, K, rank)
    return torch.empty(max(n, 1), dtype=torch.uint8, device=device)


def bwd_workspace(T, N, K, rank, device="cuda"):
    n = lib().r97q_bwd_workspace_bytes(T, N, K, rank)
    return torch.empty(max(n, 1), dtype=torch.uint8, device=device)


def qlinear_lora_fwd(w: QWeight, X, A=None, B=None, scale=1.0, y_dtype=torch.bfloat16, workspace=None,
                     out=None, t_out=None, stream=None):
    """Y = X.W^T + scale.(X.A^T).B^T; returns (Y, t)."""
    T = X.shape[0]
    rank = 0 if A is None else A.shape[0]
    if out is None:
        out = torch.empty((T, w.N), dtype=y_dtype, device=X.device)
    if rank and t_out is None:
        t_out = torch.empty((T, rank), dtype=torch.float32, device=X.device)
    if workspace is None:
        workspace = fwd_workspace(T, w.N, w.K, rank, X.device)
    rc = lib().r97q_qlinear_lora_fwd(
        C.byref(w.w), _ptr(X), T, _ptr(A), _ptr(B), rank, float(scale), _ptr(out),
        R97Q_F32 if out.dtype == torch.float32 else R97Q_BF16, _ptr(t_out), _ptr(workspace),
        workspace.numel(), _stream(stream))
    check(rc, "r97q_qlinear_lora_fwd")
    return out, t_out


def qlinear_lora_bwd(w: QWeight, X, dY, A=None, B=None, t=None, scale=1.0, dx_dtype=torch.bfloat16,
                     dX=None, accumulate=False, dA=None, dB=None, workspace=None, stream=None):
    """dX (written or added to), dA += ..., dB += ...; returns (dX, dA, dB)."""
    T = dY.shape[0]
    rank = 0 if A is None else A.shape[0]
    if dX is None:
        dX = torch.empty((T, w.K), dtype=dx_dtype, device=dY.device)
    if rank and dA is None:
        dA = torch.zeros((rank, w.K), dtype=torch.float32, device=dY.device)
    if rank and dB is None:
        dB = torch.zeros((w.N, rank), dtype=torch.float32, device=dY.device)
    if workspace is None:
        workspace = bwd_workspace(T, w.N, w.K, rank, dY.device)
    rc = lib().r97q_qlinear_lora_bwd(
        C.byref(w.w), _ptr(X), _ptr(dY), T, _ptr(A), _ptr(B), rank, float(scale), _ptr(t), _ptr(dX),
        R97Q_F32 if dX.dtype == torch.float32 else R97Q_BF16, int(bool(accumulate)), _ptr(dA),
        _ptr(dB), _ptr(workspace), workspace.numel(), _stream(stream))
    check(rc, "r97q_qlinear_lora_bwd")
    return dX, dA, dB


def _workspace(nbytes: int, device, what: str) -> torch.Tensor:
    if nbytes < 0:
        raise ValueError(f"{what}: shape or rank not served")
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)


def lora_shrink_bwd(X, A, t_cot, dX=None, accumulate=False, dA=None, want_dA=True, workspace=None, stream=None):
    """The shrink's adjoint on its own: dX (+)= t_cot . A (f32 [T, K]), dA += t_cot^T . X (f32 [r, K]).
    X bf16 [T, K] (may be None when no dA is wanted), A bf16 [r, K], t_cot f32 [T, r]. Returns (dX, dA)."""
    T, rank = t_cot.shape
    K = A.shape[1]
    if dX is None:
        dX = torch.zeros((T, K), dtype=torch.float32, device=t_cot.device)
    if want_dA and dA is None:
        dA = torch.zeros((rank, K), dtype=torch.float32, device=t_cot.device)
    if workspace is None:
        workspace = _workspace(lib().r97q_lora_shrink_bwd_workspace_bytes(T, K, rank), t_cot.device, "lora_shrink_bwd")
    rc = lib().r97q_lora_shrink_bwd(T, K, _ptr(X), _ptr(A), rank, _ptr(t_cot), _ptr(dX), int(bool(accumulate)),
                                    _ptr(dA if want_dA else None), _ptr(workspace), workspace.numel(), _stream(stream))
    check(rc, "r97q_lora_shrink_bwd")
    return dX, dA


def lora_expand_bwd(dY, B, scale, t=None, t_cot=None, dB=None, want_dB=True, workspace=None, stream=None):
    """The expand's adjoint on its own: t_cot += scale . dY . B (f32 [T, r]), dB += scale . dY^T . t
    (f32 [N, r]). dY bf16 [T, N], B bf16 [N, r], t f32 [T, r]. Returns (t_cot, dB)."""
    T, N = dY.shape
    rank = B.shape[1]
    if t_cot is None:
        t_cot = torch.zeros((T, rank), dtype=torch.float32, device=dY.device)
    if want_dB and dB is None:
        dB = torch.zeros((N, rank), dtype=torch.float32, device=dY.device)
    if workspace is None:
        workspace = _workspace(lib().r97q_lora_expand_bwd_workspace_bytes(T, N, rank), dY.device, "lora_expand_bwd")
    rc = lib().r97q_lora_expand_bwd(T, N, _ptr(dY), _ptr(B), rank, float(scale), _ptr(t), _ptr(t_cot),
                                    _ptr(dB if want_dB else None), _ptr(workspace), workspace.numel(), _stream(stream))
    check(rc, "r97q_lora_expand_bwd")
    return t_cot, dB


# ------------------------------------------------------------------ the coded (i8a8h) trunk
def gemm_nt_q_dx(w: QWeight, dY, a_scale, dA=None, accumulate=False, da_dtype=torch.float32, stream=None):
    """gemm_nt_q's adjoint in the code basis: dA[m, k] (+)= a_scale[m, k/128] . (dY . W)[m, k].
    dY bf16 [T, N], a_scale f32 [T, K/128]. Returns dA."""
    T = dY.shape[0]
    if dA is None:
        dA = torch.zeros((T, w.K), dtype=da_dtype, device=dY.device)
    rc = lib().r97q_gemm_nt_q_dx(C.byref(w.w), _ptr(dY), T, _ptr(a_scale), _ptr(dA),
                                 R97Q_F32 if dA.dtype == torch.float32 else R97Q_BF16, int(bool(accumulate)),
                                 _stream(stream))
    check(rc, "r97q_gemm_nt_q_dx")
    return dA


def gemm_nt_q_fwd(codes, scale, a, a_scale, Y=None, y_dtype=torch.float32, stream=None):
    """gemm_nt_q's twin, the coded forward: Y[m, n] = sum_g (a . codes over group g)[m, n] *
    a_scale[m, g] * scale[n, g]. The stored weight's grids: codes int8 [N, K], scale bf16 [N, K/128]
    (as uint16 bits or bfloat16); a int8 [T, K], a_scale f32 [T, K/128]. Returns Y [T, N]."""
    T, K = a.shape
    N = codes.shape[0]
    if Y is None:
        Y = torch.empty((T, N), dtype=y_dtype, device=a.device)
    rc = lib().r97q_gemm_nt_q_fwd(_ptr(codes), _ptr(scale), N, K, _ptr(a), _ptr(a_scale), T, _ptr(Y),
                                  R97Q_F32 if Y.dtype == torch.float32 else R97Q_BF16, _stream(stream))
    check(rc, "r97q_gemm_nt_q_fwd")
    return Y


def lora_shrink_q_bwd(a, a_scale, A, t_cot, da=None, ds=None, dA=None, want=("da", "ds", "dA"), workspace=None,
                      stream=None, group_width=0):
    """The coded shrink's adjoint: a [T, K] int8 codes (or f32 code values), a_scale f32 [T, groups],
    A bf16 [r, K], t_cot f32 [T, r]. Adds into (and returns) da f32 [T, K], ds f32 [T, groups], dA f32
    [r, K]. group_width 0: the reference's width rule over (K, groups)."""
    T, K = a.shape
    groups = a_scale.shape[1]
    rank = A.shape[0]
    dev = t_cot.device
    if "da" in want and da is None:
        da = torch.zeros((T, K), dtype=torch.float32, device=dev)
    if "ds" in want and ds is None:
        ds = torch.zeros((T, groups), dtype=torch.float32, device=dev)
    if "dA" in want and dA is None:
        dA = torch.zeros((rank, K), dtype=torch.float32, device=dev)
    if workspace is None:
        workspace = _workspace(lib().r97q_lora_shrink_q_bwd_workspace_bytes(T, K, rank), dev, "lora_shrink_q_bwd")
    a_dtype = R97Q_F32 if a.dtype == torch.float32 else R97Q_I8
    rc = lib().r97q_lora_shrink_q_bwd(T, K, _ptr(a), a_dtype, _ptr(a_scale), groups, group_width, _ptr(A), rank,
                                      _ptr(t_cot),
                                      _ptr(da if "da" in want else None), _ptr(ds if "ds" in want else None),
                                      _ptr(dA if "dA" in want else None), _ptr(workspace), workspace.numel(),
                                      _stream(stream))
    check(rc, "r97q_lora_shrink_q_bwd")
    return da, ds, dA
