"""The forward entry that allocates nothing (r97q_qlinear_lora_fwd_noalloc, include/r97q.h) against
the entry it varies (r97q_qlinear_lora_fwd with a caller's workspace), through the C ABI.

Both run the same kernels over the same inputs, so Y and t must be the same bits. Two calls in a row
on the library's one scratch array, the second at a smaller shape and rank (the first call's
contents left in the array must not matter); then a shape past the array is refused by name, before
any launch."""
import ctypes as C

import numpy as np
import pytest
import torch

import iqr_synth as S
from gpu_util import bf16_tensor, prepared
from test_rows import bf16_round

pytestmark = pytest.mark.gpu


def run_pair(L, w, T, r, seed):
    from r9700training_amd import R97Q_F32, _ptr, _stream, check

    rng = np.random.default_rng(seed)
    N, K = w.N, w.K
    X = bf16_tensor(bf16_round(rng.standard_normal((T, K))))
    A = bf16_tensor(bf16_round(0.01 * rng.standard_normal((r, K)))) if r else None
    B = bf16_tensor(bf16_round(0.01 * rng.standard_normal((N, r)))) if r else None
    Y1 = torch.full((T, N), float("nan"), dtype=torch.float32, device="cuda")
    Y2 = torch.full((T, N), float("nan"), dtype=torch.float32, device="cuda")
    t1 = torch.full((T, max(r, 1)), float("nan"), dtype=torch.float32, device="cuda")
    t2 = torch.full((T, max(r, 1)), float("nan"), dtype=torch.float32, device="cuda")
    ws = torch.empty(max(L.r97q_fwd_workspace_bytes(T, N, K, r), 1), dtype=torch.uint8, device="cuda")
    st = _stream()
    check(L.r97q_qlinear_lora_fwd(C.byref(w.w), _ptr(X), T, _ptr(A), _ptr(B), r, 2.0, _ptr(Y1), R97Q_F32,
                                  _ptr(t1) if r else None, _ptr(ws), ws.numel(), st), "r97q_qlinear_lora_fwd")
    check(L.r97q_qlinear_lora_fwd_noalloc(C.byref(w.w), _ptr(X), T, _ptr(A), _ptr(B), r, 2.0, _ptr(Y2), R97Q_F32,
                                          _ptr(t2) if r else None, st), "r97q_qlinear_lora_fwd_noalloc")
    torch.cuda.synchronize()
    return Y1, Y2, t1, t2


def test_noalloc_forward_equals_the_workspace_forward():
    from r9700training_amd import R97Q_F32, lib, _ptr, _stream

    L = lib()
    keep = []
    cases = [(1024, 512, 1024, 16), (300, 256, 512, 8)]  # the second smaller: T, N, K and rank
    for i, (T, N, K, r) in enumerate(cases):
        print(f"case noalloc forward call {i + 1}: T={T} N={N} K={K} rank={r}", flush=True)
        planes = S.trellis(rows=N, cols=K, bits=5, run_rows=128, rowf=True, seed=30 + i,
                           scale_col=(0.75 + 0.5 * np.arange(K // 128) / (K // 128)).astype(np.float32))
        w = prepared(planes, keep)
        Y1, Y2, t1, t2 = run_pair(L, w, T, r, seed=40 + i)
        assert not torch.isnan(Y2).any().item()
        assert torch.equal(Y1, Y2), f"call {i + 1}: Y differs from the workspace entry's"
        assert torch.equal(t1, t2), f"call {i + 1}: t differs from the workspace entry's"
        print(f"  Y and t equal, bit for bit (max |Y| {Y1.abs().max().item():.3f})", flush=True)
    # past the array: refused before any launch
    T, N, K = 8192, 256, 4096
    planes = S.trellis(rows=N, cols=K, bits=5, run_rows=128, rowf=True, seed=50, packed=True)
    w = prepared(planes, keep)
    X = torch.zeros((T, K), dtype=torch.bfloat16, device="cuda")
    Y = torch.zeros((T, N), dtype=torch.float32, device="cuda")
    rc = L.r97q_qlinear_lora_fwd_noalloc(C.byref(w.w), _ptr(X), T, None, None, 0, 1.0, _ptr(Y), R97Q_F32, None,
                                         _stream())
    assert rc != 0 and b"past the" in L.r97q_last_error()
    assert L.r97q_fwd_workspace_bytes(T, N, K, 0) > L.r97q_qlinear_lora_fwd_noalloc_max_bytes()
