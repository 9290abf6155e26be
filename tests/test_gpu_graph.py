"""The fwd + bwd step captured in a HIP graph (torch.cuda.CUDAGraph over the five stage entries):
the entry points allocate, set and synchronise nothing, so a capture records their kernels as they
are, and every replay -- with the program's own eager work and synchronisations between replays --
gives the eager step's bits."""
import ctypes as C
import os
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_step_replays_in_a_graph():
    sys.path.insert(0, ROOT)
    import bench
    from r9700training_amd import R97Q_F32, _ptr, _stream, check, lib
    from r9700training_amd.qlinear import bwd_workspace, fwd_workspace

    print("case graph T=1024 N=K=1024 r=16", flush=True)
    dev = torch.device("cuda:0")
    T, N, K, r, s = 1024, 1024, 1024, 16, 2.0
    inp = bench.make_inputs(T, N, K, r, 7, dev)
    w = inp["w"]
    L = lib()
    Y = torch.empty((T, N), device=dev)
    dX = torch.empty((T, K), device=dev)
    t = torch.empty((T, r), device=dev)
    dA = torch.zeros((r, K), device=dev)
    dB = torch.zeros((N, r), device=dev)
    wsf, wsb = fwd_workspace(T, N, K, r, dev), bwd_workspace(T, N, K, r, dev)
    P = _ptr

    def step(stream):
        st = _stream(stream)
        dA.zero_()
        dB.zero_()
        check(L.r97q_lora_fwd_prep(T, N, K, P(inp["X"]), P(inp["A"]), r, s, P(t), P(wsf), wsf.numel(), st), "fwd_prep")
        check(L.r97q_qlinear_fwd_base(C.byref(w.w), P(inp["X"]), T, P(inp["B"]), r, P(Y), R97Q_F32, P(wsf),
                                      wsf.numel(), st), "fwd_base")
        check(L.r97q_lora_bwd_prep(T, N, K, P(inp["dY"]), P(inp["A"]), P(inp["B"]), P(t), r, s, P(wsb),
                                   wsb.numel(), st), "bwd_prep")
        check(L.r97q_lora_bwd_grads(T, N, K, P(inp["X"]), P(inp["dY"]), r, P(dA), P(dB), P(wsb), wsb.numel(), st),
              "bwd_grads")
        check(L.r97q_qlinear_dx_base(C.byref(w.w), P(inp["dY"]), T, r, P(dX), R97Q_F32, 0, P(wsb), wsb.numel(), st),
              "dx_base")

    step(torch.cuda.current_stream())
    torch.cuda.synchronize()
    eager = [x.clone() for x in (Y, t, dX, dA, dB)]
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(side)  # warm the side stream once outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        step(torch.cuda.current_stream())
    for i in range(4):
        for x in (Y, t, dX, dA, dB):
            x.fill_(float("nan"))  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name, x, e in zip(("Y", "t", "dX", "dA", "dB"), (Y, t, dX, dA, dB), eager):
            assert torch.equal(x, e), (i, name)
