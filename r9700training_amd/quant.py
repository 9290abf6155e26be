"""The coded trunk's activation quantiser on the card (a front over r97q_quant_act_i8g and its
straight-through adjoint, include/r97q.h; the reference's quant_act_i8g / had_quant_act_i8g rows)."""
from __future__ import annotations

import torch

from . import R97Q_BF16, R97Q_F32, _ptr, _stream, check, lib


def _geometry(n: int, group: int, rotated: bool) -> int:
    if rotated:
        return group
    return n if group <= 0 or group > n else group


def _dtype(x: torch.Tensor) -> int:
    if x.dtype == torch.bfloat16:
        return R97Q_BF16
    if x.dtype == torch.float32:
        return R97Q_F32
    raise ValueError("quant: the activation is bf16 or f32")


def quant_act_i8g(x: torch.Tensor, group: int, rotated: bool = False, stream=None):
    """x [rows, n] -> (codes int8 [rows, n], scale f32 [rows, ngroups])."""
    if x.dim() != 2 or not x.is_contiguous():
        raise ValueError("quant_act_i8g: x is a contiguous [rows, n] tensor")
    rows, n = x.shape
    g = _geometry(n, group, rotated)
    codes = torch.empty((rows, n), dtype=torch.int8, device=x.device)
    scale = torch.empty((rows, (n + g - 1) // max(g, 1)), dtype=torch.float32, device=x.device)
    check(lib().r97q_quant_act_i8g(_ptr(x), _dtype(x), rows, n, group, int(rotated), _ptr(codes), _ptr(scale),
                                   _stream(stream)), "r97q_quant_act_i8g")
    return codes, scale


def quant_act_i8g_bwd(x: torch.Tensor, scale: torch.Tensor, g: torch.Tensor, group: int, rotated: bool = False,
                      dx: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """dx (f32, zeros when None) += the straight-through adjoint of the codes' cotangent g."""
    rows, n = x.shape
    dx = torch.zeros((rows, n), dtype=torch.float32, device=x.device) if dx is None else dx
    for t in (scale, g, dx):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("quant_act_i8g_bwd: scale, g and dx are contiguous f32 tensors")
    check(lib().r97q_quant_act_i8g_bwd(_ptr(x), _dtype(x), rows, n, group, int(rotated), _ptr(scale), _ptr(g),
                                       _ptr(dx), _stream(stream)), "r97q_quant_act_i8g_bwd")
    return dx
