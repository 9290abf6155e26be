"""The fused IQR-linear + LoRA path on the card against the oracle (the reference's host rows,
restated in oracle/ and pinned by the golden vectors).

Bars: the fused kernels' own weight decode is bit-exact (an identity operand reads bf16(code*scale)
back element for element); Y and dX (f32 outputs) within relative L2 2e-3 of the f64 host path,
with the same bf16 inputs on both sides -- the weight tile's single bf16 rounding costs ~1.65e-3;
t, dA and dB (the adapter path, carried through [hi | lo] bf16 splits) within 1e-4. bf16 outputs
add a second rounding of the same size (~2.35e-3 in all) and are held to 2.6e-3.
"""
import numpy as np
import pytest
import torch

import iqr_synth as S
from gpu_util import bf16_tensor, f64, host_weight, prepared, rel_l2
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL_BASE = 2e-3     # north star: Y / dX within relative L2 2e-3 of the fp32 host path
TOL_ADAPTER = 1e-4  # t, dA, dB


def bf16_round(a):
    return S.bf16_bits_to_f32(S.f32_to_bf16_bits(np.asarray(a, np.float32))).astype(np.float64)


def weight_planes(N, K, bits=5, run=256, seed=0, factor=True):
    rng = np.random.default_rng(seed + 1)
    sc = (0.75 + 0.5 * rng.random(K // 128)).astype(np.float32) if factor else None
    return S.trellis(rows=N, cols=K, bits=bits, state_bits=16, run_rows=run, rb=1, mad=1,
                     scale_dtype=S.F32, rowf=True, seed=seed, scale_col=sc)


@pytest.mark.parametrize("bits,run,N,K", [(5, 256, 256, 256), (5, 64, 384, 128), (3, 32, 128, 256),
                                          (4, 128, 256, 384), (6, 32, 128, 128)])
def test_fused_decode_is_exact(bits, run, N, K):
    """X = I reads the fused forward's decoded tile back: Y[k, n] = bf16(code[n,k] * scale[n,k/128]);
    dY = I does the same for the dX kernel's tile (the trellis walks the other way there)."""
    print(f"case bits={bits} run={run} N={N} K={K}", flush=True)
    from r9700training_amd.qlinear import qlinear_lora_bwd, qlinear_lora_fwd

    p = weight_planes(N, K, bits, run, seed=bits * 7 + run)
    keep = []
    w = prepared(p, keep)
    codes, scale = host_weight(p)
    Wb = S.bf16_bits_to_f32(S.f32_to_bf16_bits(
        (codes.astype(np.float32) * np.repeat(S.bf16_bits_to_f32(scale), 128, axis=1))))
    eyeK = torch.eye(K, dtype=torch.bfloat16, device="cuda")
    Y, _ = qlinear_lora_fwd(w, eyeK, y_dtype=torch.float32)
    eyeN = torch.eye(N, dtype=torch.bfloat16, device="cuda")
    dX, _, _ = qlinear_lora_bwd(w, None, eyeN, dx_dtype=torch.float32)
    torch.cuda.synchronize()
    assert np.array_equal(Y.cpu().numpy().T.view(np.uint32), Wb.view(np.uint32))
    assert np.array_equal(dX.cpu().numpy().view(np.uint32), Wb.view(np.uint32))


def run_case(T, N, K, r, bits=5, run=256, seed=0, out_dtype=torch.float32, alpha=None):
    from r9700training_amd.qlinear import qlinear_lora_bwd, qlinear_lora_fwd

    rng = np.random.default_rng(seed)
    p = weight_planes(N, K, bits, run, seed=seed + 100)
    keep = []
    w = prepared(p, keep)
    codes, scale = host_weight(p)
    x = bf16_round(rng.standard_normal((T, K)))
    dy = bf16_round(rng.standard_normal((T, N)))
    A = bf16_round(0.01 * rng.standard_normal((max(r, 1), K)))[:r]
    B = bf16_round(0.01 * rng.standard_normal((N, max(r, 1))))[:, :r]
    s = (2.0 * r if alpha is None else alpha) / max(r, 1)
    Xd, dYd = bf16_tensor(x), bf16_tensor(dy)
    Ad = bf16_tensor(A) if r else None
    Bd = bf16_tensor(B) if r else None
    Y, t = qlinear_lora_fwd(w, Xd, Ad, Bd, s, y_dtype=out_dtype)
    dX, dA, dB = qlinear_lora_bwd(w, Xd, dYd, Ad, Bd, t, s, dx_dtype=out_dtype)
    torch.cuda.synchronize()
    if r:
        ref = O.qlinear_lora_reference(x, codes, scale, A, B, s, dy)
    else:
        ref = dict(y=O.gemm_nt_twin(x, codes, scale), dx=O.gemm_nt_adjoint(dy, codes, scale))
    return dict(Y=f64(Y), dX=f64(dX), t=None if t is None else f64(t), dA=None if dA is None else f64(dA),
                dB=None if dB is None else f64(dB)), ref


CASES = [
    # T, N, K, r, bits, run
    (128, 1024, 1024, 8, 5, 256),   # config 1's shape
    (300, 256, 384, 16, 5, 64),     # a token tail (T not a multiple of 512), short runs
    (512, 384, 256, 32, 4, 128),
    (64, 128, 128, 64, 6, 32),
    (700, 256, 256, 0, 5, 256),     # no adapter: the plain stored-weight gemm_nt and its adjoint
]


@pytest.mark.parametrize("T,N,K,r,bits,run", CASES)
def test_fwd_bwd_parity(T, N, K, r, bits, run):
    print(f"case T={T} N={N} K={K} r={r} bits={bits} run={run}", flush=True)
    got, ref = run_case(T, N, K, r, bits, run, seed=T + N + K + r)
    ey, edx = rel_l2(got["Y"], ref["y"]), rel_l2(got["dX"], ref["dx"])
    print(f"  rel L2  Y {ey:.3e}  dX {edx:.3e}", flush=True)
    assert ey <= TOL_BASE and edx <= TOL_BASE
    if r:
        et, eA, eB = rel_l2(got["t"], ref["t"]), rel_l2(got["dA"], ref["dA"]), rel_l2(got["dB"], ref["dB"])
        print(f"  rel L2  t {et:.3e}  dA {eA:.3e}  dB {eB:.3e}", flush=True)
        assert et <= TOL_ADAPTER and eA <= TOL_ADAPTER and eB <= TOL_ADAPTER


def test_bf16_outputs_and_teeth():
    """bf16 outputs: the weight tile's rounding plus the output's, ~2.35e-3 in all; and a wrong
    answer fails the bars (the reference with its adapter scale doubled is far outside them)."""
    got, ref = run_case(256, 512, 256, 16, out_dtype=torch.bfloat16, seed=5)
    ey, edx = rel_l2(got["Y"], ref["y"]), rel_l2(got["dX"], ref["dx"])
    print(f"  bf16 outputs rel L2  Y {ey:.3e}  dX {edx:.3e}", flush=True)
    assert ey <= 2.6e-3 and edx <= 2.6e-3
    assert rel_l2(got["dB"], 2 * ref["dB"]) > 0.1
    assert rel_l2(got["Y"], ref["y"] + 0.02 * np.abs(ref["y"]).mean()) > TOL_BASE


# Weights whose last trellis run is short (rows_all % run_rows != 0): its tail-biting seam wraps to
# that short run's own top segment (src/iqr_decode.h:278-315; the reference pins the case in
# tests/host/iqr_decode.cpp:311-338). The fused kernels read the seam in both walks.
SHORT_RUNS = [
    # bits, run, N, K
    (3, 256, 640, 256),  # runs 256, 256, 128
    (4, 96, 256, 128),   # runs 96, 96, 64
    (5, 256, 384, 256),  # runs 256, 128
    (6, 96, 128, 256),   # runs 96, 32: the shortest run
]


def _decode_mode(mode):
    from r9700training_amd import R97Q_DECODE_AUTO, R97Q_DECODE_FUSED, R97Q_DECODE_ONCE, lib

    return lib(), {"fused": R97Q_DECODE_FUSED, "once": R97Q_DECODE_ONCE}[mode], R97Q_DECODE_AUTO


@pytest.mark.parametrize("mode", ["fused", "once"])
@pytest.mark.parametrize("bits,run,N,K", SHORT_RUNS)
def test_short_last_run_decode_is_exact(bits, run, N, K, mode):
    """The identity read-back of test_fused_decode_is_exact over weights with a short last run, on the
    fused kernels (the decode in the main loop) and on the decode-once path (the same lanes into the
    workspace): both walks give bf16(code * scale) bit for bit, the seam rows included."""
    print(f"case bits={bits} run={run} N={N} K={K} mode={mode}", flush=True)
    from r9700training_amd.qlinear import qlinear_lora_bwd, qlinear_lora_fwd

    L, m, auto = _decode_mode(mode)
    p = weight_planes(N, K, bits, run, seed=bits * 11 + run + N)
    keep = []
    w = prepared(p, keep)
    assert w.w.bits == bits, "the trellis form itself, not the int8-code form"
    codes, scale = host_weight(p)
    Wb = S.bf16_bits_to_f32(S.f32_to_bf16_bits(
        (codes.astype(np.float32) * np.repeat(S.bf16_bits_to_f32(scale), 128, axis=1))))
    L.r97q_set_decode_once(m)
    try:
        Y, _ = qlinear_lora_fwd(w, torch.eye(K, dtype=torch.bfloat16, device="cuda"), y_dtype=torch.float32)
        dX, _, _ = qlinear_lora_bwd(w, None, torch.eye(N, dtype=torch.bfloat16, device="cuda"),
                                    dx_dtype=torch.float32)
        torch.cuda.synchronize()
    finally:
        L.r97q_set_decode_once(auto)
    assert np.array_equal(Y.cpu().numpy().T.view(np.uint32), Wb.view(np.uint32))
    assert np.array_equal(dX.cpu().numpy().view(np.uint32), Wb.view(np.uint32))


@pytest.mark.parametrize("bits,run,N,K", SHORT_RUNS)
def test_short_last_run_parity(bits, run, N, K):
    """Y, dX within 2e-3 and t, dA, dB within 1e-4 of the host rows over the same weights, at a token
    count that is not a multiple of the 512-token tile."""
    T, r = 300, 16
    print(f"case T={T} N={N} K={K} r={r} bits={bits} run={run}", flush=True)
    got, ref = run_case(T, N, K, r, bits, run, seed=N + K + bits)
    ey, edx = rel_l2(got["Y"], ref["y"]), rel_l2(got["dX"], ref["dx"])
    et, eA, eB = rel_l2(got["t"], ref["t"]), rel_l2(got["dA"], ref["dA"]), rel_l2(got["dB"], ref["dB"])
    print(f"  rel L2  Y {ey:.3e}  dX {edx:.3e}  t {et:.3e}  dA {eA:.3e}  dB {eB:.3e}", flush=True)
    assert ey <= TOL_BASE and edx <= TOL_BASE
    assert et <= TOL_ADAPTER and eA <= TOL_ADAPTER and eB <= TOL_ADAPTER


def test_dx_accumulate_and_grad_accumulate():
    from r9700training_amd.qlinear import qlinear_lora_bwd, qlinear_lora_fwd

    rng = np.random.default_rng(1)
    T, N, K, r = 256, 256, 256, 16
    p = weight_planes(N, K, seed=11)
    keep = []
    w = prepared(p, keep)
    X = bf16_tensor(rng.standard_normal((T, K)))
    dY = bf16_tensor(rng.standard_normal((T, N)))
    A = bf16_tensor(0.01 * rng.standard_normal((r, K)))
    B = bf16_tensor(0.01 * rng.standard_normal((N, r)))
    _, t = qlinear_lora_fwd(w, X, A, B, 2.0)
    dX1, dA1, dB1 = qlinear_lora_bwd(w, X, dY, A, B, t, 2.0, dx_dtype=torch.float32)
    base = torch.randn((T, K), dtype=torch.float32, device="cuda")
    dX2 = base.clone()
    dA2, dB2 = dA1.clone(), dB1.clone()
    qlinear_lora_bwd(w, X, dY, A, B, t, 2.0, dX=dX2, accumulate=True, dA=dA2, dB=dB2)
    torch.cuda.synchronize()
    assert torch.allclose(dX2, base + dX1, rtol=1e-6, atol=1e-6)
    # the factor gradients are added into: dA1 + (the same sum again) is 2 * dA1 exactly
    assert torch.equal(dA2, 2 * dA1) and torch.equal(dB2, 2 * dB1)


def test_grads_are_deterministic():
    """dA and dB sum their token chunks in a fixed order: repeated calls give the same bits."""
    from r9700training_amd.qlinear import qlinear_lora_bwd, qlinear_lora_fwd

    rng = np.random.default_rng(4)
    T, N, K, r = 1000, 384, 512, 16
    p = weight_planes(N, K, seed=21)
    keep = []
    w = prepared(p, keep)
    X = bf16_tensor(rng.standard_normal((T, K)))
    dY = bf16_tensor(rng.standard_normal((T, N)))
    A = bf16_tensor(0.01 * rng.standard_normal((r, K)))
    B = bf16_tensor(0.01 * rng.standard_normal((N, r)))
    _, t = qlinear_lora_fwd(w, X, A, B, 2.0)
    runs = [qlinear_lora_bwd(w, X, dY, A, B, t, 2.0, dx_dtype=torch.float32) for _ in range(3)]
    torch.cuda.synchronize()
    for dX, dA, dB in runs[1:]:
        assert torch.equal(dX, runs[0][0]) and torch.equal(dA, runs[0][1]) and torch.equal(dB, runs[0][2])


@pytest.mark.parametrize("T,N,K,r", [(1100, 384, 512, 16), (700, 256, 640, 64), (300, 512, 256, 8)])
def test_fused_backward_equals_stages(T, N, K, r):
    """r97q_qlinear_lora_bwd hands the factor gradients' chunk sums to its dX launch, which adds them
    in chunk order; the stand-alone stages (bwd_prep, bwd_grads adding them in its own launch,
    dx_base) give the same dX, dA and dB bit for bit."""
    import ctypes as C
    from r9700training_amd import R97Q_F32, _ptr, _stream, check, lib
    from r9700training_amd.qlinear import bwd_workspace, qlinear_lora_bwd, qlinear_lora_fwd

    print(f"case fused vs staged T={T} N={N} K={K} r={r}", flush=True)
    rng = np.random.default_rng(T + r)
    keep = []
    w = prepared(weight_planes(N, K, seed=T), keep)
    X = bf16_tensor(rng.standard_normal((T, K)))
    dY = bf16_tensor(rng.standard_normal((T, N)))
    A = bf16_tensor(0.01 * rng.standard_normal((r, K)))
    B = bf16_tensor(0.01 * rng.standard_normal((N, r)))
    _, t = qlinear_lora_fwd(w, X, A, B, 2.0)
    dA0 = torch.randn((r, K), dtype=torch.float32, device="cuda")  # added into, both ways
    dB0 = torch.randn((N, r), dtype=torch.float32, device="cuda")
    dX1, dA1, dB1 = qlinear_lora_bwd(w, X, dY, A, B, t, 2.0, dx_dtype=torch.float32, dA=dA0.clone(), dB=dB0.clone())
    L = lib()
    ws = bwd_workspace(T, N, K, r)
    st = _stream(None)
    dX2 = torch.empty((T, K), dtype=torch.float32, device="cuda")
    dA2, dB2 = dA0.clone(), dB0.clone()
    P = _ptr
    check(L.r97q_lora_bwd_prep(T, N, K, P(dY), P(A), P(B), P(t), r, 2.0, P(ws), ws.numel(), st), "bwd_prep")
    check(L.r97q_lora_bwd_grads(T, N, K, P(X), P(dY), r, P(dA2), P(dB2), P(ws), ws.numel(), st), "bwd_grads")
    check(L.r97q_qlinear_dx_base(C.byref(w.w), P(dY), T, r, P(dX2), R97Q_F32, 0, P(ws), ws.numel(), st), "dx_base")
    torch.cuda.synchronize()
    assert torch.equal(dX1, dX2) and torch.equal(dA1, dA2) and torch.equal(dB1, dB2)
    assert not torch.equal(dA1, dA0) and not torch.equal(dB1, dB0)


@pytest.mark.parametrize("want", ["dA", "dB"])
def test_fused_backward_one_factor(want):
    """The fused backward asked for one factor's gradient (the other pointer null) takes that
    factor's own chunking, as the stand-alone gradient entry does: the same bits as the stages
    called the same way, and the other factor untouched."""
    import ctypes as C
    from r9700training_amd import R97Q_F32, _ptr, _stream, check, lib
    from r9700training_amd.qlinear import bwd_workspace, qlinear_lora_fwd

    T, N, K, r = 1000, 384, 640, 16
    print(f"case fused one factor {want} T={T} N={N} K={K} r={r}", flush=True)
    rng = np.random.default_rng(77)
    keep = []
    w = prepared(weight_planes(N, K, seed=5), keep)
    X = bf16_tensor(rng.standard_normal((T, K)))
    dY = bf16_tensor(rng.standard_normal((T, N)))
    A = bf16_tensor(0.01 * rng.standard_normal((r, K)))
    B = bf16_tensor(0.01 * rng.standard_normal((N, r)))
    _, t = qlinear_lora_fwd(w, X, A, B, 2.0)
    L = lib()
    P = _ptr
    st = _stream(None)
    out = {}
    for path in ("fused", "stages"):
        ws = bwd_workspace(T, N, K, r)
        dX = torch.empty((T, K), dtype=torch.float32, device="cuda")
        g = torch.zeros((r, K) if want == "dA" else (N, r), dtype=torch.float32, device="cuda")
        dA, dB = (g, None) if want == "dA" else (None, g)
        if path == "fused":
            check(L.r97q_qlinear_lora_bwd(C.byref(w.w), P(X), P(dY), T, P(A), P(B), r, 2.0, P(t), P(dX), R97Q_F32, 0,
                                          P(dA), P(dB), P(ws), ws.numel(), st), "bwd")
        else:
            check(L.r97q_lora_bwd_prep(T, N, K, P(dY), P(A), P(B), P(t), r, 2.0, P(ws), ws.numel(), st), "prep")
            check(L.r97q_lora_bwd_grads(T, N, K, P(X), P(dY), r, P(dA), P(dB), P(ws), ws.numel(), st), "grads")
            check(L.r97q_qlinear_dx_base(C.byref(w.w), P(dY), T, r, P(dX), R97Q_F32, 0, P(ws), ws.numel(), st), "dx")
        torch.cuda.synchronize()
        out[path] = (dX, g)
    assert torch.equal(out["fused"][0], out["stages"][0]) and torch.equal(out["fused"][1], out["stages"][1])
    assert out["fused"][1].abs().max().item() > 0


def test_refusals():
    from r9700training_amd import R97qError
    from r9700training_amd.qlinear import QWeight, fwd_workspace, qlinear_lora_fwd
    from gpu_util import device_desc

    keep = []
    # forms the kernels do not decode themselves take the int8-code form (tests/test_gpu_codes8.py)
    lut = S.trellis(rows=128, cols=256, bits=5, run_rows=64, mad=0, scale_dtype=S.BF16, seed=2)
    assert QWeight(device_desc(lut, keep)).codes8
    rb = S.trellis(rows=128, cols=256, bits=4, run_rows=64, rb=8, mad=1, rowf=True, seed=2)
    assert QWeight(device_desc(rb, keep), scale_col=torch.ones(2, device="cuda")).codes8
    odd = S.trellis(rows=100, cols=256, bits=4, run_rows=100, mad=1, seed=2)
    with pytest.raises(R97qError, match="multiple of 8"):
        QWeight(device_desc(odd, keep))
    p = weight_planes(256, 256, seed=3)
    w = prepared(p, keep)
    X = torch.zeros((64, 256), dtype=torch.bfloat16, device="cuda")
    A = torch.zeros((16, 256), dtype=torch.bfloat16, device="cuda")
    B = torch.zeros((256, 16), dtype=torch.bfloat16, device="cuda")
    small = torch.empty(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(R97qError, match="workspace"):
        qlinear_lora_fwd(w, X, A, B, 2.0, workspace=small)
    A12 = torch.zeros((12, 256), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(R97qError, match="rank"):
        qlinear_lora_fwd(w, X, A12, B[:, :12].contiguous(), 2.0)
