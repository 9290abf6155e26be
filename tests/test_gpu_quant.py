"""The activation quantiser on the card (r97q_quant_act_i8g and its straight-through adjoint)
against the oracle's restatement of the reference's host rows (src/adjoint/host/quant.cpp, pinned in
tests/test_oracle.py by the reference test's known answers).

Bars: codes and scales bit for bit (the kernel runs the host rows' f64 arithmetic); dx within one
f32 rounding of the f64 adjoint."""
import numpy as np
import pytest
import torch

import iqr_synth as S
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _x(rng, rows, n, dtype):
    a = rng.standard_normal((rows, n)).astype(np.float32) * (1 + 3 * rng.random((rows, 1))).astype(np.float32)
    a[0, : min(n, 7)] = 0.0
    if rows > 2:
        a[2, :] = 0.0  # an all-zero row: scale 1, codes 0
    if dtype == torch.bfloat16:
        a = S.bf16_bits_to_f32(S.f32_to_bf16_bits(a))
    return a.astype(np.float64), torch.tensor(a, dtype=torch.float32, device="cuda").to(dtype)


@pytest.mark.parametrize("rows,n,group,rotated", [(33, 384, 128, False), (17, 300, 128, False), (9, 1000, 0, False),
                                                  (40, 512, 128, True), (5, 4096, 4096, True), (64, 256, 32, True)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_quant_matches_oracle(rows, n, group, rotated, dtype):
    from r9700training_amd.quant import quant_act_i8g, quant_act_i8g_bwd

    print(f"case quant rows={rows} n={n} group={group} rotated={rotated} {dtype}", flush=True)
    rng = np.random.default_rng(rows * n + group)
    x, xd = _x(rng, rows, n, dtype)
    codes, scale = quant_act_i8g(xd, group, rotated)
    g = rng.standard_normal((rows, n)).astype(np.float32)
    dx0 = rng.standard_normal((rows, n)).astype(np.float32)
    dx = quant_act_i8g_bwd(xd, scale, torch.tensor(g, device="cuda"), group, rotated,
                           dx=torch.tensor(dx0, device="cuda"))
    torch.cuda.synchronize()
    want_codes, want_scale, _ = O.quant_act_i8g(x, group, rotated)
    assert np.array_equal(codes.cpu().numpy().astype(np.float64), want_codes)
    assert np.array_equal(scale.cpu().numpy(), want_scale.astype(np.float32))
    # the adjoint reads the scale the forward wrote (f32), as the reference's walk hands it back
    want_dx = O.quant_act_i8g_adjoint(x, scale.cpu().numpy().astype(np.float64), g.astype(np.float64), group,
                                      rotated, dx=dx0.astype(np.float64))
    got = dx.cpu().numpy().astype(np.float64)
    assert np.allclose(got, want_dx, rtol=2e-7, atol=1e-30 + 2e-7 * np.abs(want_dx).max())


@pytest.mark.parametrize("rotated", [False, True])
def test_quant_saturated_group_on_the_card(rotated):
    """The reference test's saturated group (tests/host/adjoint_quant.cpp:332-370) through the kernels."""
    from r9700training_amd.quant import quant_act_i8g, quant_act_i8g_bwd

    a = next(1.0 + k / 64.0 for k in range(64)
             if abs((1.0 + k / 64.0) * (1.0 / ((1.0 + k / 64.0) * (1.0 / 127.0)))) > 127.0)
    scale = a * (1.0 / 127.0)
    x = [[0.75 * a, 0.25 * a]] if rotated else [[a, 0.5 * a, -0.25 * a, 0.125 * a]]
    xd = torch.tensor(x, dtype=torch.float32, device="cuda").to(torch.bfloat16)
    n = xd.shape[1]
    codes, sc = quant_act_i8g(xd, n, rotated)
    gz = torch.zeros((1, n), device="cuda")
    g1 = gz.clone()
    g1[0, 1] = 1.0
    g0 = gz.clone()
    g0[0, 0] = 1.0
    d0 = quant_act_i8g_bwd(xd, sc, g0, n, rotated)
    d1 = quant_act_i8g_bwd(xd, sc, g1, n, rotated)
    torch.cuda.synchronize()
    s32 = float(np.float32(scale))
    assert int(codes[0, 0]) == 127 and float(sc[0, 0]) == s32
    assert not d0.any()
    want = [1.0 / s32, -1.0 / s32] if rotated else [0.0, 1.0 / s32, 0.0, 0.0]
    assert np.allclose(d1.cpu().numpy()[0], want, rtol=1e-7, atol=0)


def test_quant_refusals():
    from r9700training_amd import R97qError
    from r9700training_amd.quant import quant_act_i8g

    x = torch.zeros((4, 96), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(R97qError, match="power of two"):
        quant_act_i8g(x, 48, rotated=True)
    with pytest.raises(R97qError, match="power of two"):
        quant_act_i8g(torch.zeros((4, 100), dtype=torch.bfloat16, device="cuda"), 64, rotated=True)


@pytest.mark.parametrize("rows,n,group", [(12, 512, 128), (7, 1024, 1024)])
def test_had_quant_device_row(rows, n, group):
    """The had_quant_act_i8g device row (registered like the reference's, src/adjoint/device/
    quant.hip:958) called through the registry against the oracle's adjoint."""
    import ctypes as C

    from test_rows import check, hook, p

    print(f"case had_quant row rows={rows} n={n} group={group}", flush=True)
    L = hook()
    L.rh_had_quant.argtypes = [C.c_int64] * 3 + [C.c_void_p] * 4
    rng = np.random.default_rng(rows + n)
    x = S.bf16_bits_to_f32(S.f32_to_bf16_bits(rng.standard_normal((rows, n)).astype(np.float32))).astype(np.float64)
    _, scale, _ = O.quant_act_i8g(x, group, True)
    scale = scale.astype(np.float32).astype(np.float64)  # as the forward writes it
    g = rng.standard_normal((rows, n)).astype(np.float32).astype(np.float64)
    dx0 = rng.standard_normal((rows, n))
    dx = dx0.copy()
    check(L, L.rh_had_quant(rows, n, group, p(x), p(scale), p(g), p(dx)))
    want = O.quant_act_i8g_adjoint(x, scale, g, group, True, dx=dx0)
    assert np.allclose(dx, want, rtol=1e-6, atol=1e-6 * np.abs(want - dx0).max())
    # a group wider than the device row serves finds no row (the host row takes it)
    assert L.rh_had_quant(1, 2048, 2048, p(np.zeros(2048)), p(np.ones(1)), p(np.zeros(2048)), p(np.zeros(2048))) == -2
