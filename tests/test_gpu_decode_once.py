"""The weight decoded once a call against the fused kernel that decodes it in its main loop.

r97q_set_decode_once picks how the base products meet the weight: R97Q_DECODE_FUSED runs the fused
kernel (qlinear_rt_kernel, each weight tile decoded in the main loop once a 512-token panel),
R97Q_DECODE_ONCE decodes every tile once into the workspace (predecode_kernel, the fused kernel's
LDS tile format) and runs the product over them (qlinear_pd_kernel). Both compute every output with
the same MFMAs over the same operands in the same order, so the whole step -- Y, t, dX, dA, dB --
is the same bits whichever path ran: the tests run it both ways over the trellis code widths, short
and ragged runs, a ragged last token panel, adapter ranks 0-64, a single panel and the int8-code
form. An identity operand reads the decoded tiles back: Y = W^T and dX = W exactly (bf16(code *
scale), the decode the oracle pins).
"""
import numpy as np
import pytest
import torch

import iqr_synth as S
from gpu_util import bf16_tensor, device_desc, host_weight, prepared
from r9700training_amd.qlinear import QWeight

pytestmark = pytest.mark.gpu


@pytest.fixture
def mode():
    from r9700training_amd import R97Q_DECODE_AUTO, lib

    L = lib()
    yield lambda m: L.r97q_set_decode_once(m)
    assert L.r97q_set_decode_once(R97Q_DECODE_AUTO) >= 0


def bf16_round(a):
    return S.bf16_bits_to_f32(S.f32_to_bf16_bits(np.asarray(a, np.float32))).astype(np.float64)


def planes(N, K, bits, run, seed):
    rng = np.random.default_rng(seed + 1)
    sc = (0.75 + 0.5 * rng.random(K // 128)).astype(np.float32)
    return S.trellis(rows=N, cols=K, bits=bits, state_bits=16, run_rows=run, rb=1, mad=1,
                     scale_dtype=S.F32, rowf=True, seed=seed, scale_col=sc)


def weight(p, keep, codes8):
    if not codes8:
        return prepared(p, keep)
    d = device_desc(p, keep)
    sc = torch.from_numpy(p.scale_col).cuda()
    keep.append(sc)
    w = QWeight(d, scale_col=sc, codes8=True)
    assert w.codes8
    return w


def step(w, X, dY, A, B, s):
    from r9700training_amd.qlinear import qlinear_lora_bwd, qlinear_lora_fwd

    Y, t = qlinear_lora_fwd(w, X, A, B, s, y_dtype=torch.float32)
    dX, dA, dB = qlinear_lora_bwd(w, X, dY, A, B, t, s, dx_dtype=torch.float32)
    torch.cuda.synchronize()
    return Y, t, dX, dA, dB


@pytest.mark.parametrize("bits,run,N,K,T,r,codes8", [
    (5, 256, 768, 1024, 1536, 16, False),
    (3, 64, 256, 512, 1100, 8, False),    # a ragged last panel (1100 = 2 x 512 + 76)
    (4, 128, 384, 640, 1024, 0, False),   # no adapter
    (6, 32, 512, 256, 700, 32, False),
    (5, 256, 640, 384, 1030, 64, True),   # the int8-code form, a short last run
    (5, 128, 256, 256, 300, 16, False),   # one panel
])
def test_decoded_once_equals_fused(mode, bits, run, N, K, T, r, codes8):
    from r9700training_amd import R97Q_DECODE_FUSED, R97Q_DECODE_ONCE

    print(f"case bits={bits} run={run} N={N} K={K} T={T} r={r} codes8={codes8}", flush=True)
    rng = np.random.default_rng(bits * 100 + T)
    keep = []
    w = weight(planes(N, K, bits, run, seed=bits + N), keep, codes8)
    X = bf16_tensor(bf16_round(rng.standard_normal((T, K))))
    dY = bf16_tensor(bf16_round(rng.standard_normal((T, N))))
    A = bf16_tensor(bf16_round(0.01 * rng.standard_normal((r, K)))) if r else None
    B = bf16_tensor(bf16_round(0.01 * rng.standard_normal((N, r)))) if r else None
    mode(R97Q_DECODE_FUSED)
    fused = step(w, X, dY, A, B, 2.0)
    mode(R97Q_DECODE_ONCE)
    once = step(w, X, dY, A, B, 2.0)
    for a, b, name in zip(fused, once, ("Y", "t", "dX", "dA", "dB")):
        if a is None:
            continue
        assert not torch.isnan(b).any().item(), f"{name} has NaN"
        assert torch.equal(a, b), f"{name} differs between the two paths"
    print(f"  Y, t, dX, dA, dB equal bit for bit (max |Y| {fused[0].abs().max().item():.3f})", flush=True)


@pytest.mark.parametrize("bits,run,N,K,codes8", [(5, 256, 768, 1024, False), (3, 32, 640, 768, False),
                                                  (6, 128, 1024, 640, True)])
def test_decoded_tiles_read_back(mode, bits, run, N, K, codes8):
    """X = I and dY = I through the decoded-once path read each product's tiles back as
    bf16(code * scale), element for element."""
    from r9700training_amd import R97Q_DECODE_ONCE
    from r9700training_amd.qlinear import qlinear_lora_bwd, qlinear_lora_fwd

    print(f"case read-back bits={bits} run={run} N={N} K={K} codes8={codes8}", flush=True)
    mode(R97Q_DECODE_ONCE)
    keep = []
    p = planes(N, K, bits, run, seed=bits * 3 + K)
    w = weight(p, keep, codes8)
    codes, scale = host_weight(p)
    Wb = S.bf16_bits_to_f32(S.f32_to_bf16_bits(
        (codes.astype(np.float32) * np.repeat(S.bf16_bits_to_f32(scale), 128, axis=1))))
    Y, _ = qlinear_lora_fwd(w, torch.eye(K, dtype=torch.bfloat16, device="cuda"), y_dtype=torch.float32)
    dX, _, _ = qlinear_lora_bwd(w, None, torch.eye(N, dtype=torch.bfloat16, device="cuda"), dx_dtype=torch.float32)
    torch.cuda.synchronize()
    assert np.array_equal(Y.cpu().numpy().T.view(np.uint32), Wb.view(np.uint32))
    assert np.array_equal(dX.cpu().numpy().view(np.uint32), Wb.view(np.uint32))


def test_mode_refusal():
    from r9700training_amd import R97Q_DECODE_AUTO, lib

    L = lib()
    assert L.r97q_set_decode_once(7) == -1
    assert L.r97q_set_decode_once(R97Q_DECODE_AUTO) == R97Q_DECODE_AUTO
