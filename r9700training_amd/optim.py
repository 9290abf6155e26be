"""AdamW for the adapter's factors on the card (a front over r97q_adamw_step, include/r97q.h).

The reference's optimiser (include/r97/optim.h, src/optim.cpp) keeps f32 master weights, moments and
an accumulation buffer per parameter and updates them on the host; this one keeps the same four
buffers as device tensors and produces the same bits. An update is one launch over all the
parameters, which can also write the kernels' next bf16 operands (`bf16_out`) and take the device
rows' staged f32 gradients directly (`staged=True`: the reference's grad_stage flush into zero-filled
leaves, fused into the step).
"""
from __future__ import annotations

import ctypes as C

import torch

from . import R97Q_ADAMW_GRADS_STAGED, AdamWConfig, AdamWParam, _ptr, _stream, check, lib


def config(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0, clip_norm=0.0, lr_floor_frac=0.1,
           warmup_steps=0, total_steps=0, accum_steps=1) -> AdamWConfig:
    """The reference's AdamWConfig defaults (include/r97/optim.h:27-40)."""
    return AdamWConfig(lr, beta1, beta2, eps, weight_decay, clip_norm, lr_floor_frac, warmup_steps, total_steps,
                       accum_steps)


def scheduled_lr(cfg: AdamWConfig, step: int) -> float:
    return float(lib().r97q_scheduled_lr(C.byref(cfg), int(step)))


class DeviceAdamW:
    """Optimiser over f32 device tensors (updated in place). decay[i] = 0 excludes parameter i from
    weight decay (the reference's no_decay names). bf16_out[i] (optional): a bf16 tensor shaped
    like parameter i that every update refreshes with the new weights (RNE)."""

    def __init__(self, params, cfg: AdamWConfig, decay=None, bf16_out=None):
        if not params:
            raise ValueError("DeviceAdamW: empty parameter set")
        for p in params:
            if p.dtype != torch.float32 or not p.is_cuda or not p.is_contiguous():
                raise ValueError("DeviceAdamW: parameters are contiguous f32 device tensors")
        if bf16_out is not None:
            if len(bf16_out) != len(params):
                raise ValueError("DeviceAdamW: one bf16_out tensor a parameter")
            for o, p in zip(bf16_out, params):
                if o.dtype != torch.bfloat16 or o.shape != p.shape or not o.is_contiguous() or o.device != p.device:
                    raise ValueError("DeviceAdamW: bf16_out tensors are contiguous bf16, shaped as the parameters")
        self.params = list(params)
        self.bf16_out = list(bf16_out) if bf16_out is not None else None
        self.cfg = cfg
        self.m = [torch.zeros_like(p) for p in params]
        self.v = [torch.zeros_like(p) for p in params]
        self.acc = [torch.zeros_like(p) for p in params]
        decay = [1] * len(params) if decay is None else list(decay)
        outs = self.bf16_out or [None] * len(params)
        self._table = (AdamWParam * len(params))(*[
            AdamWParam(p.data_ptr(), m.data_ptr(), v.data_ptr(), a.data_ptr(), o.data_ptr() if o is not None else None,
                       p.numel(), int(d))
            for p, m, v, a, o, d in zip(self.params, self.m, self.v, self.acc, outs, decay)])
        nbytes = lib().r97q_adamw_workspace_bytes(self._table, len(params))
        self.workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=params[0].device)
        self.updates = C.c_int32(0)
        self.pending = C.c_int32(0)

    def step(self, grads, stream=None, staged=False) -> bool:
        """Accumulate `grads` (f32 device tensors shaped like the parameters); every accum_steps-th
        call apply one update. staged: `grads` are f32 staging buffers, each value rounded once to
        bf16 (the flush) and the buffers cleared by the call. Returns True when this call updated."""
        if len(grads) != len(self.params):
            raise ValueError("DeviceAdamW.step: grads do not match the parameter set")
        for g, p in zip(grads, self.params):
            if g.shape != p.shape or g.dtype != torch.float32 or not g.is_contiguous() or g.device != p.device:
                raise ValueError("DeviceAdamW.step: grads do not match the parameter set")
        ptrs = (C.c_void_p * len(grads))(*[g.data_ptr() for g in grads])
        applied = C.c_int32(0)
        rc = lib().r97q_adamw_step(C.byref(self.cfg), self._table, ptrs, len(grads),
                                   R97Q_ADAMW_GRADS_STAGED if staged else 0, C.byref(self.updates),
                                   C.byref(self.pending), C.byref(applied), _ptr(self.workspace),
                                   self.workspace.numel(), _stream(stream))
        check(rc, "r97q_adamw_step")
        return bool(applied.value)


def bf16_copies(params, out=None, stream=None):
    """bf16 copies of f32 device tensors (RNE), into `out` when given."""
    out = [torch.empty(p.shape, dtype=torch.bfloat16, device=p.device) for p in params] if out is None else out
    for p, o in zip(params, out):
        check(lib().r97q_f32_to_bf16(_ptr(p), _ptr(o), p.numel(), _stream(stream)), "r97q_f32_to_bf16")
    return out
