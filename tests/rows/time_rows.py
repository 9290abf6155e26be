"""Timing of the adjoint rows at C2 (T = N = K = 4096, rank 16) through the registry, the way the
reference's backward walk calls them: f64 host values in and out, the row stages them to the card,
runs the kernels and brings the result back. Each row's call time is printed beside the C ABI's
time for the same product on resident device operands (HIP events), so the staging cost of the row
contract stands next to the kernels it wraps.

Run on a GPU box from the repo root (after __graft_entry__.build()):
    python tests/rows/time_rows.py
Prints a markdown table."""
import ctypes as C
import os
import statistics
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.dirname(HERE)]

import iqr_synth as S  # noqa: E402
from gpu_util import prepared, stored_operand  # noqa: E402

from r9700training_amd import R97Q_F32, _ptr, _stream, check, lib  # noqa: E402
from r9700training_amd.qlinear import bwd_workspace, fwd_workspace  # noqa: E402

_P = C.c_void_p


def hook():
    L = C.CDLL(os.path.join(HERE, "librowshook.so"))
    L.rh_last_error.restype = C.c_char_p
    L.rh_last_row_ms.restype = C.c_double
    L.rh_gemm_nt.argtypes = [C.c_int64, C.c_int64, C.c_int64, _P, _P, _P, _P, _P]
    L.rh_lora_shrink.argtypes = [C.c_int64] * 4 + [_P] * 6 + [C.c_int]
    L.rh_lora_expand.argtypes = [C.c_int64] * 4 + [_P] * 7 + [C.c_int, C.c_int, _P]
    return L


def timed(fn, H, reps=3):
    """Median wall time (ms) of `fn` over `reps` calls after one warm call, and the median time of
    the row invocation alone inside it (rh_last_row_ms: without the hook building the record's f64
    values and copying the results out, which a walk does not do)."""
    fn()
    out, row = [], []
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        out.append((time.perf_counter() - t0) * 1e3)
        row.append(H.rh_last_row_ms())
    return statistics.median(out), statistics.median(row)


def events(fn, reps=20):
    """Mean GPU time (ms) of `fn` between two HIP events on the current stream."""
    fn()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def main():
    T = N = K = 4096
    r, alpha = 16, 32.0
    s = alpha / r
    H = hook()
    L = lib()
    rng = np.random.default_rng(2001)
    p = S.trellis(rows=N, cols=K, bits=5, run_rows=256, rowf=True, seed=3, packed=True,
                  scale_col=(0.5 + rng.random(K // 128)).astype(np.float32))
    keep = []
    enc, raw = stored_operand(p, keep)
    bf = lambda a: S.bf16_bits_to_f32(S.f32_to_bf16_bits(np.asarray(a, np.float32))).astype(np.float64)
    x = bf(rng.standard_normal((T, K)))
    dy = bf(rng.standard_normal((T, N)))
    la = bf(0.01 * rng.standard_normal((1, r, K)))
    lb = bf(0.01 * rng.standard_normal((1, N, r)))
    slot = np.zeros(T)
    t = rng.standard_normal((T, r))
    t_cot = rng.standard_normal((T, r))
    dx = np.zeros((T, K))
    tc = np.zeros((T, r))
    dA = np.zeros((1, r, K), np.float32)
    dB = np.zeros((1, N, r), np.float32)
    scale = np.full((1, N), s)

    def ck(rc):
        if rc != 0:
            raise RuntimeError(H.rh_last_error().decode())

    rows = {
        "gemm_nt (dX = dY.W, stored IQR weight)": lambda: ck(H.rh_gemm_nt(
            T, N, K, dy.ctypes.data, C.addressof(enc), raw.data_ptr(), None, dx.ctypes.data)),
        "lora_shrink (dX += t_cot.A, dA)": lambda: ck(H.rh_lora_shrink(
            T, K, r, 1, x.ctypes.data, slot.ctypes.data, la.ctypes.data, t_cot.ctypes.data, dx.ctypes.data,
            dA.ctypes.data, 1)),
        "lora_expand (t_cot = s.dY.B, dB)": lambda: ck(H.rh_lora_expand(
            T, N, r, 1, t.ctypes.data, slot.ctypes.data, lb.ctypes.data, scale.ctypes.data, dy.ctypes.data,
            tc.ctypes.data, dB.ctypes.data, 1, 0, None)),
    }
    row_ms = {k: timed(f, H) for k, f in rows.items()}

    # the C ABI on resident operands: the fused dX product, and the whole fwd + bwd step
    dev = torch.device("cuda:0")
    w = prepared(p, keep)
    X = torch.from_numpy(x.astype(np.float32)).to(dev).to(torch.bfloat16)
    dY = torch.from_numpy(dy.astype(np.float32)).to(dev).to(torch.bfloat16)
    A = torch.from_numpy(la[0].astype(np.float32)).to(dev).to(torch.bfloat16)
    B = torch.from_numpy(lb[0].astype(np.float32)).to(dev).to(torch.bfloat16)
    Y = torch.empty((T, N), device=dev)
    dXd = torch.empty((T, K), device=dev)
    tt = torch.empty((T, r), device=dev)
    dAd = torch.zeros((r, K), device=dev)
    dBd = torch.zeros((N, r), device=dev)
    wsf, wsb = fwd_workspace(T, N, K, r, dev), bwd_workspace(T, N, K, r, dev)
    st = _stream(torch.cuda.current_stream())
    P = _ptr

    def dx_base():
        check(L.r97q_lora_bwd_prep(T, N, K, P(dY), P(A), P(B), P(tt), 0, s, P(wsb), wsb.numel(), st), "prep")
        check(L.r97q_qlinear_dx_base(C.byref(w.w), P(dY), T, 0, P(dXd), R97Q_F32, 0, P(wsb), wsb.numel(), st), "dx")

    def step():
        check(L.r97q_lora_fwd_prep(T, N, K, P(X), P(A), r, s, P(tt), P(wsf), wsf.numel(), st), "fwd_prep")
        check(L.r97q_qlinear_fwd_base(C.byref(w.w), P(X), T, P(B), r, P(Y), R97Q_F32, P(wsf), wsf.numel(), st), "fwd")
        check(L.r97q_lora_bwd_prep(T, N, K, P(dY), P(A), P(B), P(tt), r, s, P(wsb), wsb.numel(), st), "bwd_prep")
        check(L.r97q_lora_bwd_grads(T, N, K, P(X), P(dY), r, P(dAd), P(dBd), P(wsb), wsb.numel(), st), "grads")
        check(L.r97q_qlinear_dx_base(C.byref(w.w), P(dY), T, r, P(dXd), R97Q_F32, 0, P(wsb), wsb.numel(), st), "dx")

    abi = {"dX product, C ABI (dY tiled copy + fused kernel)": events(dx_base),
           "whole fwd + bwd step, C ABI (all five entries)": events(step)}

    print("| call at C2 (T = N = K = 4096, rank 16) | ms a call (the row) | ms a call (with the hook's record building) |")
    print("|---|---:|---:|")
    for k, (v, rv) in row_ms.items():
        print(f"| registry row `{k}`, f64 host in / out | {rv:.1f} | {v:.1f} |")
    for k, v in abi.items():
        print(f"| {k}, device-resident | {v:.3f} | |")
    print(f"\nrow calls: median of 3 after a warm call (wall clock, synchronised; the row alone timed inside "
          f"the hook around the registry's function); C ABI: HIP events over 20 calls; torch {torch.__version__}, "
          f"nproc {os.cpu_count()}, host threads {os.environ.get('R97_THREADS', 'min(8, nproc)')}")


if __name__ == "__main__":
    main()
