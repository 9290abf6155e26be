"""The vocabulary head's transposed product on the card (a front over r97q_vocab_head_transpose,
include/r97q.h; the reference's src/vocab_head.h).

A plan holds up to four classes of IQR-coded rows: each class's planes on the card (an
R97IqrDecodeDesc with rows_all == the class's rows), the vocabulary id of each of its rows, and its
per-128-column scale.col. `transpose` adds H . sum_c (dy[:, ids_c] . W_c) * scale.col_c into d_x.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import Desc, VocabClass, VocabPlan, _ptr, _stream, check, lib

R97_IQR_F32 = 0


class VocabHead:
    def __init__(self, n_embd: int, vocab: int, classes, vocab_offset: int = 0, transform: int = 0):
        """classes: (desc, ids, scale_col[, scale_col_dtype]) each -- desc a Desc over device planes,
        ids a device int32 tensor [rows], scale_col a device tensor of n_embd/128 values (f32 unless
        the dtype says otherwise). The tensors must outlive the plan."""
        if not 1 <= len(classes) <= 4:
            raise ValueError("VocabHead: one to four classes")
        self.plan = VocabPlan()
        self.plan.n_embd, self.plan.vocab, self.plan.vocab_offset = int(n_embd), int(vocab), int(vocab_offset)
        self.plan.transform, self.plan.classes = int(transform), len(classes)
        self._keep = []
        for i, c in enumerate(classes):
            desc, ids, cf = c[:3]
            dtype = c[3] if len(c) > 3 else R97_IQR_F32
            if ids.dtype != torch.int32 or not ids.is_cuda:
                raise ValueError("VocabHead: ids are a device int32 tensor")
            k = self.plan.cls[i]
            k.rows = int(desc.rows_all)
            k.decode = Desc.from_buffer_copy(desc)
            k.ids = ids.data_ptr()
            k.scale_col = cf.data_ptr()
            k.scale_col_dtype = int(dtype)
            k.scale_col_row_bytes = cf.numel() * cf.element_size()
            self._keep += [ids, cf]

    def workspace_bytes(self, rows: int) -> int:
        n = lib().r97q_vocab_head_workspace_bytes(C.byref(self.plan), int(rows))
        if n < 0:
            check(1, "r97q_vocab_head_workspace_bytes")
        return int(n)

    def transpose(self, dy: torch.Tensor, d_x: torch.Tensor, workspace: torch.Tensor | None = None, stream=None):
        """d_x f32 [rows, n_embd] += the head's transposed product of dy bf16 [rows, vocab]."""
        rows = dy.shape[0]
        if dy.dtype != torch.bfloat16 or tuple(dy.shape) != (rows, self.plan.vocab) or not dy.is_contiguous():
            raise ValueError("VocabHead.transpose: dy is a contiguous bf16 [rows, vocab] tensor")
        if d_x.dtype != torch.float32 or tuple(d_x.shape) != (rows, self.plan.n_embd) or not d_x.is_contiguous():
            raise ValueError("VocabHead.transpose: d_x is a contiguous f32 [rows, n_embd] tensor")
        need = self.workspace_bytes(rows)
        if workspace is None:
            workspace = torch.empty(need, dtype=torch.uint8, device=dy.device)
        check(lib().r97q_vocab_head_transpose(C.byref(self.plan), _ptr(dy), rows, _ptr(d_x), _ptr(workspace),
                                              workspace.numel(), _stream(stream)), "r97q_vocab_head_transpose")
        return d_x


def cast(src: torch.Tensor, dst: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """bf16 <- f32, round to nearest even (the CE loop's fill)."""
    if src.dtype != torch.float32 or not src.is_contiguous():
        raise ValueError("cast: src is a contiguous f32 tensor")
    dst = torch.empty(src.shape, dtype=torch.bfloat16, device=src.device) if dst is None else dst
    check(lib().r97q_vocab_head_cast(_ptr(dst), _ptr(src), src.numel(), _stream(stream)), "r97q_vocab_head_cast")
    return dst
