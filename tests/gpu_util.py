"""Helpers for the GPU tests: planes to the device, rel-L2, the oracle's inputs from device tensors."""
from __future__ import annotations

import numpy as np
import torch

import iqr_synth as S
from r9700training_amd import Desc
from r9700training_amd.qlinear import QWeight


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def device_desc(p: S.Planes, keep: list, row0: int = 0, rows: int | None = None) -> Desc:
    """The planes of `p` on the device and their description (tensors appended to `keep`)."""
    rows = p.rows - row0 if rows is None else rows
    codes = dev(p.codes)
    scale = dev(p.scale)
    keep += [codes, scale]
    d = Desc()
    d.rows_all, d.cols, d.row0, d.rows = p.rows, p.cols, row0, rows
    d.bits, d.state_bits, d.run_rows, d.rb = p.bits, p.state_bits, p.run_rows, p.rb
    d.mad, d.round_mad, d.mad_a, d.mad_b = p.mad, p.round_mad, p.mad_a, p.mad_b
    if p.lut is not None:
        lut = dev(p.lut)
        keep.append(lut)
        d.lut = lut.data_ptr()
    d.codes = codes.data_ptr() + row0 * p.codes_row_bytes
    d.codes_row_bytes = p.codes_row_bytes
    d.scale = scale.data_ptr() + row0 * p.scale_row_bytes
    d.scale_dtype, d.scale_block_cols, d.scale_row_bytes = p.scale_dtype, p.scale_block_cols, p.scale_row_bytes
    d.affine = p.affine
    if p.affine:
        zero = dev(p.zero)
        keep.append(zero)
        d.zero = zero.data_ptr() + row0 * p.zero.shape[1]
        d.zero_bits = p.zero_bits
        d.zero_row_bytes = p.zero.shape[1]
    if p.scale2 is not None:
        s2 = dev(p.scale2)
        keep.append(s2)
        d.scale2 = s2.data_ptr()
        d.scale2_dtype = p.scale2_dtype
        d.scale2_row_bytes = p.scale2_row_bytes
    return d


def prepared(p: S.Planes, keep: list) -> QWeight:
    d = device_desc(p, keep)
    sc = None
    if p.scale_col is not None:
        sc = dev(p.scale_col)
        keep.append(sc)
    return QWeight(d, scale_col=sc)


def host_weight(p: S.Planes):
    """The oracle's stored weight for `p`: int8 codes and the (folded) bf16 scale."""
    from oracle import oracle as O

    codes, scale = O.decode(p.desc())
    if p.scale_col is not None:
        scale = O.fold_scale_col(p.scale.view(np.float32).reshape(-1), p.scale_col)
    return codes, scale


def bf16_tensor(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).cuda()


def f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def rel_l2(got: np.ndarray, want: np.ndarray) -> float:
    num = np.linalg.norm((np.asarray(got, np.float64) - np.asarray(want, np.float64)).ravel())
    den = np.linalg.norm(np.asarray(want, np.float64).ravel())
    return float(num / den) if den > 0 else float(num)


def stored_operand(p: S.Planes, keep: list):
    """The stored operand the rows read for `p`: (its R97Encoding, the joined planes on the device)."""
    e, buf = S.joined(p)
    d = dev(buf)
    keep.append(d)
    return e, d
