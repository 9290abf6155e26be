"""The adapter's adjoints as separate calls (r97q_lora_shrink_bwd, r97q_lora_expand_bwd) against the
oracle's restatement of the reference's host rows (src/adjoint/host/lora.cpp:260-328, 451-521).

X and dY are bf16-exact on both sides; the cotangent t_cot handed to the shrink is an arbitrary f64
(rounded to f32 on the way in, then split into [hi | lo] bf16 inside), so every result is held to
1e-4 relative L2, the adapter path's bar."""
import numpy as np
import pytest
import torch

from gpu_util import bf16_tensor, f64, rel_l2
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-4


def bf16_round(a):
    import iqr_synth as S
    return S.bf16_bits_to_f32(S.f32_to_bf16_bits(np.asarray(a, np.float32))).astype(np.float64)


@pytest.mark.parametrize("T,K,r", [(128, 1024, 8), (300, 384, 16), (64, 256, 32), (520, 128, 64)])
def test_shrink_bwd(T, K, r):
    from r9700training_amd.qlinear import lora_shrink_bwd

    print(f"case shrink T={T} K={K} r={r}", flush=True)
    rng = np.random.default_rng(T + K + r)
    x = bf16_round(rng.standard_normal((T, K)))
    A = bf16_round(0.01 * rng.standard_normal((r, K)))
    ct = rng.standard_normal((T, r))
    base = rng.standard_normal((T, K)).astype(np.float32)
    dX = torch.tensor(base, device="cuda")
    dX, dA = lora_shrink_bwd(bf16_tensor(x), bf16_tensor(A), torch.tensor(ct, dtype=torch.float32, device="cuda"),
                             dX=dX, accumulate=True)
    torch.cuda.synchronize()
    slot = np.zeros(T)
    ref_dx, ref_da = O.lora_shrink_adjoint(x, slot, A.reshape(1, r, K), ct.astype(np.float32).astype(np.float64))
    e_dx = rel_l2(f64(dX) - base.astype(np.float64), ref_dx)
    e_da = rel_l2(f64(dA), ref_da)
    print(f"  rel L2 dx {e_dx:.3e} dA {e_da:.3e}", flush=True)
    assert e_dx <= TOL and e_da <= TOL


@pytest.mark.parametrize("T,N,r", [(128, 1024, 8), (300, 384, 16), (64, 256, 32), (520, 128, 64)])
def test_expand_bwd(T, N, r):
    from r9700training_amd.qlinear import lora_expand_bwd

    print(f"case expand T={T} N={N} r={r}", flush=True)
    rng = np.random.default_rng(T + N + r + 1)
    dy = bf16_round(rng.standard_normal((T, N)))
    B = bf16_round(0.01 * rng.standard_normal((N, r)))
    t = rng.standard_normal((T, r)).astype(np.float32).astype(np.float64)
    s = 2.0
    tc0 = rng.standard_normal((T, r)).astype(np.float32)
    t_cot = torch.tensor(tc0, device="cuda")
    t_cot, dB = lora_expand_bwd(bf16_tensor(dy), bf16_tensor(B), s, t=torch.tensor(t, dtype=torch.float32,
                                                                                     device="cuda"), t_cot=t_cot)
    torch.cuda.synchronize()
    slot = np.zeros(T)
    ref_dt, ref_db = O.lora_expand_adjoint(t, slot, B.reshape(1, N, r), np.full((1, N), s), dy)
    e_dt = rel_l2(f64(t_cot) - tc0.astype(np.float64), ref_dt)
    e_db = rel_l2(f64(dB), ref_db)
    print(f"  rel L2 dt {e_dt:.3e} dB {e_db:.3e}", flush=True)
    assert e_dt <= TOL and e_db <= TOL


def test_rows_compose_to_the_fused_backward():
    """expand adjoint -> shrink adjoint (the walk's order) gives the fused backward's dA, dB and
    the adapter part of dX."""
    from r9700training_amd.qlinear import lora_expand_bwd, lora_shrink_bwd

    rng = np.random.default_rng(9)
    T, N, K, r, s = 256, 384, 512, 16, 2.0
    dy = bf16_round(rng.standard_normal((T, N)))
    x = bf16_round(rng.standard_normal((T, K)))
    A = bf16_round(0.01 * rng.standard_normal((r, K)))
    B = bf16_round(0.01 * rng.standard_normal((N, r)))
    t = x @ A.T
    t_cot, dB = lora_expand_bwd(bf16_tensor(dy), bf16_tensor(B), s, t=torch.tensor(t, dtype=torch.float32,
                                                                                     device="cuda"))
    dX, dA = lora_shrink_bwd(bf16_tensor(x), bf16_tensor(A), t_cot)
    torch.cuda.synchronize()
    slot = np.zeros(T)
    ref_dt, ref_db = O.lora_expand_adjoint(t.astype(np.float32).astype(np.float64), slot, B.reshape(1, N, r),
                                           np.full((1, N), s), dy)
    ref_dx, ref_da = O.lora_shrink_adjoint(x, slot, A.reshape(1, r, K), ref_dt)
    assert rel_l2(f64(dB), ref_db) <= TOL
    assert rel_l2(f64(dA), ref_da) <= TOL
    assert rel_l2(f64(dX), ref_dx) <= TOL
