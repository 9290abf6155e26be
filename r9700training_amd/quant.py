"""The coded trunk's activation quantiser on the card (a front over r97q_quant_act_i8g and its
straight-through adjoint, include/r97q.h; the reference's quant_act_i8g / had_quant_act_i8g rows),
and the fused producers rmsnorm_had_quant_i8g, gated_had_quant_i8g and gate_had_quant_i8g
(r97q_fused_had_quant_i8g; the reference's src/adjoint/host/quant.cpp:896-1405)."""
from __future__ import annotations

import torch

from . import (R97Q_BF16, R97Q_F32, R97Q_F64, R97Q_PART_RMSNORM, R97Q_PART_SIGMOID_MUL, R97Q_PART_SILU_MUL,
               _ptr, _stream, check, lib)


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


PARTS = {"rmsnorm": R97Q_PART_RMSNORM, "silu_mul": R97Q_PART_SILU_MUL, "sigmoid_mul": R97Q_PART_SIGMOID_MUL}


def _part_inputs(part: str, x0: torch.Tensor, x1):
    if part not in PARTS:
        raise ValueError(f"fused quantiser: part {part!r} is not one of {sorted(PARTS)}")
    dt = {torch.bfloat16: R97Q_BF16, torch.float32: R97Q_F32, torch.float64: R97Q_F64}.get(x0.dtype)
    if dt is None or x0.dim() != 2 or not x0.is_contiguous():
        raise ValueError("fused quantiser: x0 is a contiguous [rows, width] bf16, f32 or f64 tensor")
    rows = x0.shape[0]
    n = x0.shape[1] // 2 if part == "silu_mul" else x0.shape[1]
    if part != "silu_mul":
        want = (n,) if part == "rmsnorm" else (rows, n)
        if x1 is None or tuple(x1.shape) != want or x1.dtype != x0.dtype or not x1.is_contiguous():
            raise ValueError(f"fused quantiser: {part} takes a contiguous second input of shape {want} in x0's dtype")
    return PARTS[part], dt, rows, n


def fused_had_quant_i8g(part: str, x0: torch.Tensor, x1: torch.Tensor | None, group: int, eps: float = 1e-6,
                        wadd: float = 0.0, mult: float = 1.0, want_y: bool = False, stream=None):
    """(codes int8 [rows, n], scale f32 [rows, n / group], y bf16 [rows, n] or None) of the fused
    producer: part "rmsnorm" (x0 = x, x1 = w [n]), "silu_mul" (x0 = gate_up [rows, 2n]) or
    "sigmoid_mul" (x0 = a, x1 = b), then the rotated group quantiser."""
    k, dt, rows, n = _part_inputs(part, x0, x1)
    codes = torch.empty((rows, n), dtype=torch.int8, device=x0.device)
    scale = torch.empty((rows, n // max(group, 1)), dtype=torch.float32, device=x0.device)
    y = torch.empty((rows, n), dtype=torch.bfloat16, device=x0.device) if want_y else None
    check(lib().r97q_fused_had_quant_i8g(k, _ptr(x0), _ptr(x1) if x1 is not None else None, dt, rows, n, group,
                                         eps, wadd, mult, _ptr(codes), _ptr(scale),
                                         _ptr(y) if y is not None else None, _stream(stream)),
          "r97q_fused_had_quant_i8g")
    return codes, scale, y


def fused_had_quant_i8g_bwd(part: str, x0: torch.Tensor, x1: torch.Tensor | None, group: int, scale: torch.Tensor,
                            g_codes: torch.Tensor, g_out: torch.Tensor | None = None, eps: float = 1e-6,
                            wadd: float = 0.0, mult: float = 1.0, dx0: torch.Tensor | None = None,
                            dx1: torch.Tensor | None = None, stream=None):
    """(dx0, dx1) (f32, zeros when None; dx1 None unless sigmoid_mul) += the fused producer's adjoint
    of the codes' cotangent g_codes and the output's cotangent g_out."""
    k, dt, rows, n = _part_inputs(part, x0, x1)
    dx0 = torch.zeros(x0.shape, dtype=torch.float32, device=x0.device) if dx0 is None else dx0
    if part == "sigmoid_mul" and dx1 is None:
        dx1 = torch.zeros((rows, n), dtype=torch.float32, device=x0.device)
    for t in (scale, g_codes, g_out, dx0, dx1):
        if t is not None and (t.dtype != torch.float32 or not t.is_contiguous()):
            raise ValueError("fused_had_quant_i8g_bwd: scale, cotangents and dx are contiguous f32 tensors")
    check(lib().r97q_fused_had_quant_i8g_bwd(k, _ptr(x0), _ptr(x1) if x1 is not None else None, dt, rows, n, group,
                                             eps, wadd, mult, _ptr(scale), _ptr(g_codes),
                                             _ptr(g_out) if g_out is not None else None, _ptr(dx0),
                                             _ptr(dx1) if dx1 is not None else None, _stream(stream)),
          "r97q_fused_had_quant_i8g_bwd")
    return dx0, dx1
