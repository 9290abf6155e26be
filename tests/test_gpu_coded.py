"""The coded (i8a8h) trunk on the card against the oracle's restatement of the reference's host rows
(src/adjoint/host/linear.cpp:245-317, src/adjoint/host/lora.cpp:246-328): the C entries
r97q_gemm_nt_q_fwd, r97q_gemm_nt_q_dx and r97q_lora_shrink_q_bwd, and the device rows gemm_nt_q
and the coded lora_shrink driven through the registry as the reference's walk drives them.

gemm_nt_q's twin sums each 128-column group exactly (int8 products, int32 sums) and folds the groups
in f32: against the oracle's f64 loop only the f32 fold differs, so its bar is 1e-5 (bf16 Y: the
one rounding of the output, 4e-3).

Bars: gemm_nt_q's code cotangent multiplies a stored IQR weight as bf16(code * scale), one rounding
of each weight (~1.65e-3), so it is held to the base products' 2e-3 relative L2 (a weight carried as
codes + scale through the rows library takes the same single rounding). The shrink's cotangents and
dA carry t_cot as an [hi | lo] bf16 pair and x = code * scale as another: 1e-4."""
import ctypes as C

import numpy as np
import pytest
import torch

import iqr_synth as S
from gpu_util import bf16_tensor, dev, device_desc, f64, host_weight, prepared, rel_l2, stored_operand
from oracle import oracle as O
from test_rows import bf16_round, check, hook, p

pytestmark = pytest.mark.gpu

TOL_BASE = 2e-3
TOL_ADAPTER = 1e-4


def weight_planes(N, K, seed):
    rng = np.random.default_rng(seed)
    return S.trellis(rows=N, cols=K, bits=5, state_bits=16, run_rows=128, rb=1, mad=1, scale_dtype=S.F32,
                     rowf=True, seed=seed, scale_col=(0.75 + 0.5 * rng.random(K // 128)).astype(np.float32))


def codes_and_scales(rng, T, K, groups):
    a = np.rint(rng.uniform(-1.0, 1.0, (T, K)) * 60.0)
    s = (0.02 + 0.05 * rng.random((T, groups))).astype(np.float32).astype(np.float64)
    return a, s


TOL_EXACT = 1e-5


def full_range_codes(rng, T, K):
    """int8 activation codes over the whole range, with per-(row, group) f32 scales."""
    a = rng.integers(-127, 128, (T, K)).astype(np.float64)
    s = (0.01 + 0.05 * rng.random((T, K // 128))).astype(np.float32).astype(np.float64)
    return a, s


@pytest.mark.parametrize("T,N,K", [(300, 256, 384), (512, 384, 256), (64, 128, 1024), (1030, 512, 512), (1, 128, 128),
                                   (257, 640, 896)])
def test_gemm_nt_q_fwd(T, N, K):
    from r9700training_amd.qlinear import gemm_nt_q_fwd

    print(f"case gemm_nt_q_fwd T={T} N={N} K={K}", flush=True)
    rng = np.random.default_rng(7 * T + N + K)
    codes, scale = host_weight(weight_planes(N, K, seed=T + 1))
    cd, scd = dev(codes), dev(scale)
    a, a_scale = full_range_codes(rng, T, K)
    ad = torch.tensor(a.astype(np.int8), device="cuda")
    sd = torch.tensor(a_scale.astype(np.float32), device="cuda")
    got = gemm_nt_q_fwd(cd, scd, ad, sd)
    got_bf = gemm_nt_q_fwd(cd, scd, ad, sd, y_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    want = O.gemm_nt_q_twin(a, a_scale, codes, scale)
    e, e_bf = rel_l2(f64(got), want), rel_l2(f64(got_bf), want)
    print(f"  rel L2 Y {e:.3e} bf16 {e_bf:.3e}", flush=True)
    assert e <= TOL_EXACT and e_bf <= 4e-3
    # the activation scale is applied per group: one group's scale doubled moves the result
    a_scale2 = a_scale.copy()
    a_scale2[:, -1] *= 2.0
    assert rel_l2(f64(got), O.gemm_nt_q_twin(a, a_scale2, codes, scale)) > 10 * TOL_EXACT


def test_gemm_nt_q_fwd_c2():
    """C2's square layer (T = N = K = 4096): the whole Y against the oracle on sampled token rows
    (the first, tile-edge, middle and last), and every row at once through the column sums of the
    group products (each group's sum over m of a * a_scale is one row the oracle multiplies)."""
    from r9700training_amd.qlinear import gemm_nt_q_fwd

    print("case gemm_nt_q_fwd C2", flush=True)
    T = N = K = 4096
    rng = np.random.default_rng(4096)
    sc = (0.75 + 0.5 * rng.random(K // 128)).astype(np.float32)
    planes = S.trellis(rows=N, cols=K, bits=5, state_bits=16, run_rows=256, rb=1, mad=1, scale_dtype=S.F32,
                       rowf=True, seed=11, scale_col=sc, packed=True)
    codes, scale = host_weight(planes)
    a, a_scale = full_range_codes(rng, T, K)
    got = f64(gemm_nt_q_fwd(dev(codes), dev(scale), torch.tensor(a.astype(np.int8), device="cuda"),
                            torch.tensor(a_scale.astype(np.float32), device="cuda")))
    rows = np.unique(np.array([0, 1, 31, 32, 255, 256, 2047, 2048, 3839, 3840, 4094, 4095]))
    e = rel_l2(got[rows], O.gemm_nt_q_twin(a[rows], a_scale[rows], codes, scale))
    # sum over m of Y[m, n] = sum_g (sum_m a[m, g-cols] * a_scale[m, g]) . code[n, g-cols] * scale[n, g]:
    # one f64 row per group, through the oracle with unit activation scales
    x = (a.reshape(T, K // 128, 128) * a_scale[:, :, None]).sum(axis=0).reshape(1, K)
    want_sum = O.gemm_nt_q_twin(x, np.ones((1, K // 128)), codes, scale)[0]
    e_sum = rel_l2(got.sum(axis=0), want_sum)
    print(f"  rel L2 sampled rows {e:.3e} column sums {e_sum:.3e}", flush=True)
    assert e <= TOL_EXACT and e_sum <= TOL_EXACT


def test_gemm_nt_q_fwd_refusals():
    from r9700training_amd import R97qError
    from r9700training_amd.qlinear import gemm_nt_q_fwd

    codes = torch.zeros((128, 300), dtype=torch.int8, device="cuda")
    with pytest.raises(R97qError, match="multiples of 128"):
        gemm_nt_q_fwd(codes, torch.zeros((128, 3), dtype=torch.int16, device="cuda"),
                      torch.zeros((8, 300), dtype=torch.int8, device="cuda"), torch.ones((8, 3), device="cuda"))


@pytest.mark.parametrize("T,N,K", [(300, 256, 384), (512, 384, 256), (64, 128, 1024), (1030, 512, 512)])
def test_gemm_nt_q_dx(T, N, K):
    from r9700training_amd.qlinear import gemm_nt_q_dx

    print(f"case gemm_nt_q_dx T={T} N={N} K={K}", flush=True)
    rng = np.random.default_rng(T + N + K)
    planes = weight_planes(N, K, seed=T)
    keep = []
    w = prepared(planes, keep)
    codes, scale = host_weight(planes)
    dy = bf16_round(rng.standard_normal((T, N)))
    a_scale = (0.02 + 0.05 * rng.random((T, K // 128))).astype(np.float32)
    sd = torch.tensor(a_scale, device="cuda")
    got = gemm_nt_q_dx(w, bf16_tensor(dy), sd)
    base = torch.randn((T, K), dtype=torch.float32, device="cuda")
    acc = gemm_nt_q_dx(w, bf16_tensor(dy), sd, dA=base.clone(), accumulate=True)
    got_bf = gemm_nt_q_dx(w, bf16_tensor(dy), sd, da_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    want = O.gemm_nt_q_adjoint(dy, codes, scale, a_scale.astype(np.float64))
    e, e_acc, e_bf = rel_l2(f64(got), want), rel_l2(f64(acc) - f64(base), want), rel_l2(f64(got_bf), want)
    print(f"  rel L2 dA {e:.3e} accumulate {e_acc:.3e} bf16 {e_bf:.3e}", flush=True)
    assert e <= TOL_BASE and e_acc <= TOL_BASE and e_bf <= 2.6e-3
    # the scale is applied: without it the result is far off
    assert rel_l2(f64(got), O.gemm_nt_adjoint(dy, codes, scale)) > 0.5


@pytest.mark.parametrize("T,K,r,groups", [(300, 256, 16, 2), (512, 384, 8, 3), (200, 256, 64, 1), (128, 512, 32, 4)])
def test_lora_shrink_q_bwd(T, K, r, groups):
    from r9700training_amd.qlinear import lora_shrink_q_bwd

    print(f"case lora_shrink_q_bwd T={T} K={K} r={r} groups={groups}", flush=True)
    rng = np.random.default_rng(T + K + r + groups)
    a, a_scale = codes_and_scales(rng, T, K, groups)
    A = bf16_round(0.05 * rng.standard_normal((r, K)))
    ct = rng.standard_normal((T, r)).astype(np.float32).astype(np.float64)
    da0 = rng.standard_normal((T, K)).astype(np.float32)
    ds0 = rng.standard_normal((T, groups)).astype(np.float32)
    da, ds, dA = lora_shrink_q_bwd(torch.tensor(a.astype(np.int8), device="cuda"),
                                   torch.tensor(a_scale.astype(np.float32), device="cuda"), bf16_tensor(A),
                                   torch.tensor(ct.astype(np.float32), device="cuda"),
                                   da=torch.tensor(da0, device="cuda"), ds=torch.tensor(ds0, device="cuda"))
    torch.cuda.synchronize()
    want_da, want_ds, want_dA = O.lora_shrink_q_adjoint(a, a_scale, np.zeros(T), A.reshape(1, r, K), ct)
    e_da = rel_l2(f64(da) - da0.astype(np.float64), want_da)
    e_ds = rel_l2(f64(ds) - ds0.astype(np.float64), want_ds)
    e_dA = rel_l2(f64(dA), want_dA)
    print(f"  rel L2 da {e_da:.3e} ds {e_ds:.3e} dA {e_dA:.3e}", flush=True)
    assert e_da <= TOL_ADAPTER and e_ds <= TOL_ADAPTER and e_dA <= TOL_ADAPTER


@pytest.mark.parametrize("M,N,K,carried", [(96, 256, 384, False), (200, 512, 256, False), (64, 384, 256, True)])
def test_gemm_nt_q_row(M, N, K, carried):
    print(f"case gemm_nt_q row M={M} N={N} K={K} carried={carried}", flush=True)
    L = hook()
    L.rh_gemm_nt_q.argtypes = [C.c_int64] * 3 + [C.c_void_p] * 7
    rng = np.random.default_rng(M + N + K + 7)
    dy = rng.standard_normal((M, N))
    a_scale = (0.02 + 0.05 * rng.random((M, K // 128))).astype(np.float32).astype(np.float64)
    da0 = rng.standard_normal((M, K))
    da = da0.copy()
    planes = weight_planes(N, K, seed=M + 1)
    codes, scale = host_weight(planes)
    if carried:
        bsc = S.bf16_bits_to_f32(scale).astype(np.float64)
        wc = codes.astype(np.float64)  # held: the call reads it through a raw pointer
        check(L, L.rh_gemm_nt_q(M, N, K, p(dy), p(a_scale), None, None, p(wc), p(bsc), p(da)))
    else:
        keep = []
        enc, raw = stored_operand(planes, keep)
        check(L, L.rh_gemm_nt_q(M, N, K, p(dy), p(a_scale), C.addressof(enc), raw.data_ptr(), None, None, p(da)))
    want = O.gemm_nt_q_adjoint(dy, codes, scale, a_scale, da=da0)
    e = rel_l2(da - da0, want - da0)
    print(f"  rel L2 da {e:.3e}", flush=True)
    assert e <= TOL_BASE


@pytest.mark.parametrize("M,K,R,S_,groups,fused", [(40, 256, 16, 2, 2, False), (33, 384, 8, 1, 3, True),
                                                   (64, 256, 32, 2, 1, True)])
def test_lora_shrink_q_row(M, K, R, S_, groups, fused):
    print(f"case coded lora_shrink row M={M} K={K} R={R} S={S_} groups={groups} fused={fused}", flush=True)
    L = hook()
    L.rh_lora_shrink_q.argtypes = [C.c_int64] * 6 + [C.c_char_p] + [C.c_void_p] * 8 + [C.c_int]
    rng = np.random.default_rng(M + K + R)
    a, a_scale = codes_and_scales(rng, M, K, groups)
    slot = np.array([-1 if m == 1 else (S_ if m == 2 else m % S_) for m in range(M)], np.float64)
    la = bf16_round(0.05 * rng.standard_normal((S_, R, K)))
    ct = rng.standard_normal((M, R)).astype(np.float32).astype(np.float64)
    da0 = rng.standard_normal((M, K))
    ds0 = rng.standard_normal((M, groups))
    da, ds = da0.copy(), ds0.copy()
    dA = np.zeros((S_ * R, K), np.float32)
    group = O.group_width(K, groups)
    check(L, L.rh_lora_shrink_q(M, K, R, S_, groups, group, b"i8", p(a), p(a_scale), p(slot), p(la), p(ct), p(da),
                                p(ds), p(dA), int(fused)))
    want_da, want_ds, want_dA = O.lora_shrink_q_adjoint(a, a_scale, slot, la, ct, da=da0, ds=ds0, fused=True)
    e_da, e_ds, e_dA = rel_l2(da - da0, want_da - da0), rel_l2(ds - ds0, want_ds - ds0), rel_l2(dA, want_dA)
    print(f"  rel L2 da {e_da:.3e} ds {e_ds:.3e} dA {e_dA:.3e}", flush=True)
    assert e_da <= TOL_ADAPTER and e_ds <= TOL_ADAPTER and e_dA <= TOL_ADAPTER
    # base rows (1: slot -1, 2: past the pool) get nothing
    assert np.array_equal(da[1:3], da0[1:3]) and np.array_equal(ds[1:3], ds0[1:3])


def test_coded_entry_refusals():
    """The C entry serves K a multiple of 128 (the rows pad other widths) and a group width whose
    groups fit K; it refuses the rest by name."""
    from r9700training_amd import R97qError
    from r9700training_amd.qlinear import lora_shrink_q_bwd

    with pytest.raises(R97qError, match="K a multiple of 128"):
        lora_shrink_q_bwd(torch.zeros((8, 300), dtype=torch.int8, device="cuda"),
                          torch.ones((8, 3), device="cuda"), torch.zeros((16, 300), dtype=torch.bfloat16, device="cuda"),
                          torch.zeros((8, 16), device="cuda"))
    with pytest.raises(R97qError, match="do not fit K"):
        lora_shrink_q_bwd(torch.zeros((8, 256), dtype=torch.int8, device="cuda"),
                          torch.ones((8, 3), device="cuda"), torch.zeros((16, 256), dtype=torch.bfloat16, device="cuda"),
                          torch.zeros((8, 16), device="cuda"), group_width=128)
