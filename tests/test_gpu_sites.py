"""The reference's own adapter sites on the card, through the device rows (libr97rows.so) the way
the reference's walk calls them, with nothing refused.

  * The host test's sites (tests/host/adjoint_lora.cpp:62-69): the three float sites and the three
    coded ones, rank 4 and K = 300 / N = 96 among them, against the golden vectors the reference's
    own host rows wrote (tests/golden/lora_*.npz, tests/golden/make_golden.py), under both the fused
    and the summed naming of the pool's factors.
  * The GPU test's sites (tests/gpu/adjoint_lora.cpp:85-106): the tiny fixture (ranks 16 and 4, K =
    300 with groups 128 / 128 / 44 and N = 96, a rank-2048 pool, the pools of three and two rows) and
    the real model's widths (hidden 5120; q_proj 12288, ffn_down 17408, gate_up 34816 in two
    modules; 1024 and 4096 tokens; ranks 16, 4 and 32), with that test's value rules, for the coded
    shrink and the expand, against the oracle's restatement of the host rows over every element.
  * B = 0, the adapter's first step (tests/host/adjoint_lora.cpp:595-636, docs/adjoints/lora.md:
    158-165): the expand gives t's cotangent exactly nothing and dB its full value; the shrink handed
    that zero gives dA = 0 and the activation's cotangents exactly nothing. And the fused C entry with
    B = 0: Y and dX are the rank-0 products' bits, dA is zero, dB matches the oracle.
  * The stored-weight store under address reuse: a second weight written into the first one's
    buffers under the same encoding object gets its own prepared weight.

The rows carry cotangents as [hi | lo] bf16 pairs and sum in f32: 1e-4 relative L2 everywhere."""
import ctypes as C
import os

import numpy as np
import pytest
import torch

import iqr_synth as S
from gpu_util import bf16_tensor, f64, host_weight, prepared, rel_l2, stored_operand
from oracle import oracle as O
from test_rows import bf16_round, check, hook, p

pytestmark = pytest.mark.gpu

TOL = 1e-4
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bind(L):
    L.rh_lora_shrink_q.argtypes = [C.c_int64] * 6 + [C.c_char_p] + [C.c_void_p] * 8 + [C.c_int]
    return L


def run_shrink_q(L, a, a_scale, slot, la, ct, fused, dtype=b"i8", group=128):
    M, K = a.shape
    S_, R, _ = la.shape
    groups = a_scale.shape[1]
    da, ds = np.zeros((M, K)), np.zeros((M, groups))
    dA = np.zeros((S_ * R, K), np.float32)
    check(L, L.rh_lora_shrink_q(M, K, R, S_, groups, group, dtype, p(a), p(a_scale), p(slot), p(la), p(ct), p(da),
                                p(ds), p(dA), int(fused)))
    return da, ds, dA


def run_shrink(L, x, slot, la, ct, fused):
    M, K = x.shape
    S_, R, _ = la.shape
    dx = np.zeros((M, K))
    dA = np.zeros((S_ * R, K), np.float32)
    check(L, L.rh_lora_shrink(M, K, R, S_, p(x), p(slot), p(la), p(ct), p(dx), p(dA), int(fused)))
    return dx, dA


def run_expand(L, t, slot, lb, sc, cy, fused, t_cot0=None):
    M, R = t.shape
    S_, N, _ = lb.shape
    tc = np.zeros((M, R)) if t_cot0 is None else t_cot0.copy()
    dB = np.zeros(S_ * N * R, np.float32)
    check(L, L.rh_lora_expand(M, N, R, S_, p(t), p(slot), p(lb), p(sc), p(cy), p(tc), p(dB), int(fused), 0, None))
    return tc, dB


def per_slot_sum(leaf, S_, rows, cols):
    """The per-slot leaves ([S, rows, cols], one after another) summed: the golden's one leaf."""
    return leaf.reshape(S_, rows, cols).sum(axis=0)


# ---------------------------------------------------------------- the host test's sites
@pytest.mark.parametrize("name", ["tiny_q_proj", "tiny_gate_proj", "tiny_down_proj"])
def test_float_sites_against_reference_rows(name):
    print(f"case golden float site {name}", flush=True)
    L = hook()
    z = np.load(os.path.join(GOLDEN, f"lora_{name}.npz"))
    x, slot, la, lb, sc, ct, cy, t = (z[k] for k in ("x", "slot", "la", "lb", "sc", "ct", "cy", "t"))
    S_, R, K = la.shape
    N = lb.shape[1]
    for fused in (0, 1):
        dx, dA = run_shrink(L, x, slot, la, ct, fused)
        dt, dB = run_expand(L, t, slot, lb, sc, cy, fused)
        want_da = z[f"da_f{fused}"]
        got_da = dA if fused else per_slot_sum(dA, S_, R, K)
        want_db = z[f"db_f{fused}"]
        got_db = dB.reshape(N, S_ * R) if fused else per_slot_sum(dB, S_, N, R)
        errs = [rel_l2(dx, z[f"dx_f{fused}"]), rel_l2(got_da, want_da), rel_l2(dt, z[f"dt_f{fused}"]),
                rel_l2(got_db, want_db)]
        print(f"  fused={fused} rel L2 dx {errs[0]:.2e} dA {errs[1]:.2e} dt {errs[2]:.2e} dB {errs[3]:.2e}",
              flush=True)
        assert max(errs) <= TOL


@pytest.mark.parametrize("name", ["coded_q_proj", "coded_down_proj", "coded_up_proj"])
def test_coded_sites_against_reference_rows(name):
    print(f"case golden coded site {name}", flush=True)
    L = bind(hook())
    z = np.load(os.path.join(GOLDEN, f"lora_{name}.npz"))
    a, a_scale, slot, la, ct = (z[k] for k in ("a", "a_scale", "slot", "la", "ct"))
    S_, R, K = la.shape
    for fused in (0, 1):
        da, ds, dA = run_shrink_q(L, a, a_scale, slot, la, ct, fused)
        got_dA = dA if fused else per_slot_sum(dA, S_, R, K)
        errs = [rel_l2(da, z[f"da_f{fused}"]), rel_l2(ds, z[f"ds_f{fused}"]), rel_l2(got_dA, z[f"dA_f{fused}"])]
        print(f"  fused={fused} rel L2 da {errs[0]:.2e} ds {errs[1]:.2e} dA {errs[2]:.2e}", flush=True)
        assert max(errs) <= TOL


# ---------------------------------------------------------------- the GPU test's sites
# name, M, K, N, R, S, packed, pooled (tests/gpu/adjoint_lora.cpp:85-111)
GPU_SITES = [
    ("tiny_q_proj_r16", 6, 128, 128, 16, 2, False, False),
    ("tiny_down_proj_r4", 4, 128, 256, 4, 1, False, False),
    ("tiny_up_proj_k300_r4", 5, 300, 96, 4, 2, False, False),
    ("tiny_q_proj_r2048", 5, 128, 128, 2048, 1, False, False),
    ("tiny_q_proj_pool3_r16", 6, 128, 128, 16, 3, False, True),
    ("tiny_q_proj_pool2_r16", 6, 128, 128, 16, 2, False, True),
    ("q_proj_r16_1024", 1024, 5120, 12288, 16, 1, False, False),
    ("q_proj_r16_4096", 4096, 5120, 12288, 16, 1, False, False),
    ("down_proj_r16_1024", 1024, 17408, 5120, 16, 1, False, False),
    ("q_proj_r4_1024", 1024, 5120, 12288, 4, 1, False, False),
    ("gate_up_r32_1024_two_modules", 1024, 5120, 34816, 32, 1, True, False),
]


def slot_of(M, S_, pooled):
    """tests/gpu/adjoint_lora.cpp:121-127."""
    out = []
    for m in range(M):
        if M > 16:
            out.append(0)
        elif pooled:
            out.append(0 if m == 0 else -1 if m == 1 else S_ if m == 2 else 0 if m == 3 else 1)
        else:
            out.append(-1 if m == 1 else S_ if m == 2 else m % S_)
    return np.array(out, np.float64)


def site_values(M, K, N, R, S_, packed, pooled, seed):
    """The value rules of tests/gpu/adjoint_lora.cpp:186-233: integer codes in [-60, 60], positive
    group scales, bf16 factors (a packed B zero outside each row's module), f32 t, alpha / r scales."""
    rng = np.random.default_rng(seed)
    groups = (K + 127) // 128
    a = np.rint(rng.uniform(-1, 1, (M, K)) * 60.0)
    i = np.arange(M * groups).reshape(M, groups)
    a_scale = (0.02 + 0.01 * (i % 7) + 0.004 * np.abs(rng.uniform(-1, 1, (M, groups)))).astype(np.float32)
    la = bf16_round(rng.uniform(-1, 1, (S_, R, K)))
    lb = bf16_round(rng.uniform(-1, 1, (S_, N, R)))
    if packed:
        own = (np.arange(N) >= N // 2).astype(np.int64)
        lb[:, (own[:, None] != (np.arange(R)[None, :] // (R // 2)))] = 0.0
    t = rng.uniform(-1, 1, (M, R)).astype(np.float32).astype(np.float64)
    sc = np.array([[2.0 / (1 + (s % 2))] * N for s in range(S_)], np.float32).astype(np.float64)
    ct = rng.uniform(-1, 1, (M, R)).astype(np.float32).astype(np.float64)
    cy = bf16_round(rng.uniform(-1, 1, (M, N)))
    return a, a_scale.astype(np.float64), slot_of(M, S_, pooled), la, lb, t, sc, ct, cy


@pytest.mark.parametrize("site", GPU_SITES, ids=[s[0] for s in GPU_SITES])
def test_gpu_test_sites(site):
    name, M, K, N, R, S_, packed, pooled = site
    print(f"case gpu site {name} M={M} K={K} N={N} R={R} S={S_}", flush=True)
    L = bind(hook())
    a, a_scale, slot, la, lb, t, sc, ct, cy = site_values(M, K, N, R, S_, packed, pooled, seed=M + K + N + R)
    for fused in ((0, 1) if M <= 16 else (1,)):
        da, ds, dA = run_shrink_q(L, a, a_scale, slot, la, ct, fused)
        want_da, want_ds, want_dA = O.lora_shrink_q_adjoint(a, a_scale, slot, la, ct, fused=True)
        got_dA = dA if fused else dA.reshape(S_ * R, K)  # per-slot leaves stack as the fused factor's blocks
        dt, dB = run_expand(L, t, slot, lb, sc, cy, fused)
        want_dt, want_db = O.lora_expand_adjoint(t, slot, lb, sc, cy, fused=True)
        got_db = dB.reshape(N, S_ * R) if fused else dB.reshape(S_, N, R).transpose(1, 0, 2).reshape(N, S_ * R)
        errs = {"da": rel_l2(da, want_da), "ds": rel_l2(ds, want_ds), "dA": rel_l2(got_dA, want_dA),
                "dt": rel_l2(dt, want_dt), "dB": rel_l2(got_db, want_db)}
        print(f"  fused={fused} " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
        assert max(errs.values()) <= TOL, errs
        if M <= 16:  # base rows get nothing
            base = [m for m in range(M) if slot[m] < 0 or slot[m] >= S_]
            assert not da[base].any() and not ds[base].any() and not dt[base].any()


@pytest.mark.parametrize("dtype", [b"fp8_e4m3", b"fp8_e5m2"])
def test_coded_shrink_fp8_codes(dtype):
    """The fp8 code dtypes (the reference's coded_act): code values an f32 holds exactly."""
    print(f"case coded shrink {dtype.decode()}", flush=True)
    L = bind(hook())
    rng = np.random.default_rng(5)
    M, K, R, S_ = 40, 300, 16, 2
    groups = 3
    mant = 3 if dtype == b"fp8_e4m3" else 2
    a = np.ldexp(np.round(rng.uniform(1, 2, (M, K)) * 2 ** mant) / 2 ** mant, rng.integers(-6, 7, (M, K)))
    a *= np.where(rng.random((M, K)) < 0.5, -1.0, 1.0)
    a_scale = (0.01 + 0.02 * rng.random((M, groups))).astype(np.float32).astype(np.float64)
    slot = np.array([-1 if m == 1 else m % S_ for m in range(M)], np.float64)
    la = bf16_round(0.05 * rng.standard_normal((S_, R, K)))
    ct = rng.standard_normal((M, R)).astype(np.float32).astype(np.float64)
    da, ds, dA = run_shrink_q(L, a, a_scale, slot, la, ct, 1, dtype=dtype)
    want_da, want_ds, want_dA = O.lora_shrink_q_adjoint(a, a_scale, slot, la, ct, fused=True)
    errs = [rel_l2(da, want_da), rel_l2(ds, want_ds), rel_l2(dA, want_dA)]
    print(f"  rel L2 da {errs[0]:.2e} ds {errs[1]:.2e} dA {errs[2]:.2e}", flush=True)
    assert max(errs) <= TOL


# ---------------------------------------------------------------- B = 0
@pytest.mark.parametrize("name", ["coded_q_proj", "coded_up_proj", "tiny_down_proj"])
def test_b_zero_through_the_rows(name):
    print(f"case B = 0 rows {name}", flush=True)
    L = bind(hook())
    z = np.load(os.path.join(GOLDEN, f"lora_{name}.npz"))
    coded = name.startswith("coded")
    rng = np.random.default_rng(3)
    slot, la = z["slot"], z["la"]
    S_, R, K = la.shape
    M = slot.shape[0]
    N = 96 if name == "coded_up_proj" else 128
    t = rng.standard_normal((M, R)).astype(np.float32).astype(np.float64)
    lb = np.zeros((S_, N, R))
    sc = np.full((S_, N), 2.0)
    cy = bf16_round(rng.standard_normal((M, N)))
    t_cot0 = rng.standard_normal((M, R))
    dt, dB = run_expand(L, t, slot, lb, sc, cy, 1, t_cot0=t_cot0)
    assert np.array_equal(dt, t_cot0), "B = 0: the expand adds exactly nothing to t's cotangent"
    _, want_db = O.lora_expand_adjoint(t, slot, lb, sc, cy, fused=True)
    assert dB.any() and rel_l2(dB.reshape(N, S_ * R), want_db) <= TOL
    zero = np.zeros((M, R))
    if coded:
        da, ds, dA = run_shrink_q(L, z["a"], z["a_scale"], slot, la, zero, 1)
        assert not da.any() and not ds.any()
    else:
        dx, dA = run_shrink(L, z["x"], slot, la, zero, 1)
        assert not dx.any()
    assert not dA.any(), "B = 0: dA is exactly zero"


def test_b_zero_through_the_fused_entries():
    from r9700training_amd.qlinear import qlinear_lora_bwd, qlinear_lora_fwd

    print("case B = 0 fused entries", flush=True)
    rng = np.random.default_rng(4)
    T, N, K, r, s = 640, 384, 512, 16, 2.0
    planes = S.trellis(rows=N, cols=K, bits=5, run_rows=128, rowf=True, seed=9,
                       scale_col=(0.75 + 0.5 * rng.random(K // 128)).astype(np.float32))
    keep = []
    w = prepared(planes, keep)
    x, dy = bf16_round(rng.standard_normal((T, K))), bf16_round(rng.standard_normal((T, N)))
    A = bf16_round(0.01 * rng.standard_normal((r, K)))
    Xd, dYd, Ad = bf16_tensor(x), bf16_tensor(dy), bf16_tensor(A)
    Bd = torch.zeros((N, r), dtype=torch.bfloat16, device="cuda")
    Y, t = qlinear_lora_fwd(w, Xd, Ad, Bd, s, y_dtype=torch.float32)
    Y0, _ = qlinear_lora_fwd(w, Xd, None, None, s, y_dtype=torch.float32)
    dX, dA, dB = qlinear_lora_bwd(w, Xd, dYd, Ad, Bd, t, s, dx_dtype=torch.float32)
    dX0, _, _ = qlinear_lora_bwd(w, Xd, dYd, None, None, None, s, dx_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(Y, Y0) and torch.equal(dX, dX0), "B = 0: the base products' bits"
    assert not dA.any().item(), "B = 0: dA is exactly zero"
    codes, scale = host_weight(planes)
    ref = O.qlinear_lora_reference(x, codes, scale, A, np.zeros((N, r)), s, dy)
    e_db, e_t = rel_l2(f64(dB), ref["dB"]), rel_l2(f64(t), ref["t"])
    print(f"  rel L2 dB {e_db:.2e} t {e_t:.2e}", flush=True)
    assert dB.any().item() and e_db <= TOL and e_t <= TOL


# ---------------------------------------------------------------- the store under address reuse
def test_stored_weight_store_under_address_reuse():
    """Weight 1, then weight 2 written into weight 1's freed planes (the caching allocator hands the
    same block back) under the same encoding object, without clearing the store: the second call is
    weight 2's product (the store's print of the planes differs, so it prepares again)."""
    print("case stored weight address reuse", flush=True)
    L = hook()
    M, N, K = 64, 256, 384
    rng = np.random.default_rng(8)
    dy = rng.standard_normal((M, N))
    w1 = S.trellis(rows=N, cols=K, bits=5, run_rows=128, rowf=True, seed=21)
    w2 = S.trellis(rows=N, cols=K, bits=5, run_rows=128, rowf=True, seed=22)
    enc, buf1 = S.joined(w1)
    d1 = torch.from_numpy(buf1).cuda()
    dx1 = np.zeros((M, K))
    check(L, L.rh_gemm_nt(M, N, K, p(dy), C.addressof(enc), d1.data_ptr(), None, p(dx1)))
    addr1 = d1.data_ptr()
    del d1
    torch.cuda.synchronize()
    enc2, buf2 = S.joined(w2)
    C.memmove(C.addressof(enc), C.addressof(enc2), C.sizeof(enc))  # the same encoding object, rewritten
    d2 = torch.from_numpy(buf2).cuda()
    print(f"  planes at {addr1:#x} then {d2.data_ptr():#x}", flush=True)
    dx2 = np.zeros((M, K))
    check(L, L.rh_gemm_nt(M, N, K, p(dy), C.addressof(enc), d2.data_ptr(), None, p(dx2)))
    c1, s1 = host_weight(w1)
    c2, s2 = host_weight(w2)
    e1 = rel_l2(dx1, O.gemm_nt_adjoint(dy, c1, s1))
    e2 = rel_l2(dx2, O.gemm_nt_adjoint(dy, c2, s2))
    print(f"  rel L2 weight 1 {e1:.2e} weight 2 {e2:.2e}", flush=True)
    assert e1 <= 2e-3 and e2 <= 2e-3
