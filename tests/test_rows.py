"""The adjoint rows (libr97rows.so, the r97/adjoint.h contract) driven through the registry the way
the reference's backward walk drives its device rows, against the oracle's restatement of the
reference's host rows (src/adjoint/host/linear.cpp:221-243, src/adjoint/host/lora.cpp:260-328,
451-521).

The CPU test checks the registry's lookup rules and this build's registrations (op, side,
predicate, frozen positions, family). The GPU tests check each row's numbers: activations and
weights are bf16 values on both sides; cotangents are arbitrary f64 (the rows carry them as
[hi | lo] bf16 pairs), so the bar is 1e-4 relative L2 -- except for a stored IQR weight, which the
fused kernels multiply as bf16(code * scale), one rounding of each weight (~1.65e-3): that product
is held to the base products' 2e-3."""
import ctypes as C
import os

import numpy as np
import pytest

import iqr_synth as S

HERE = os.path.dirname(os.path.abspath(__file__))
TOL = 1e-4
TOL_STORED = 2e-3
_P = C.c_void_p


def hook():
    path = os.path.join(HERE, "rows", "librowshook.so")
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built (run __graft_entry__.build())")
    L = C.CDLL(path)
    L.rh_last_error.restype = C.c_char_p
    L.rh_registry_selftest.restype = C.c_int
    L.rh_gemm_nt.argtypes = [C.c_int64, C.c_int64, C.c_int64, _P, _P, _P, _P, _P]
    L.rh_lora_shrink.argtypes = [C.c_int64] * 4 + [_P] * 6 + [C.c_int]
    L.rh_lora_expand.argtypes = [C.c_int64] * 4 + [_P] * 7 + [C.c_int, C.c_int, _P]
    L.rh_lora_expand_op.argtypes = [C.c_char_p] + [C.c_int64] * 4 + [_P] * 7 + [C.c_int, C.c_int, _P]
    L.rh_weights_prepared.restype = C.c_int64
    L.rh_scratch_stats.argtypes = [C.POINTER(C.c_int64)] * 3
    L.rh_scratch_alloc.restype = _P
    L.rh_scratch_alloc.argtypes = [C.c_int64]
    L.rh_scratch_free.argtypes = [_P]
    return L


def scratch(L):
    v = [C.c_int64() for _ in range(3)]
    L.rh_scratch_stats(*[C.byref(x) for x in v])
    return tuple(x.value for x in v)  # live, peak, allocations


def p(a):
    return None if a is None else a.ctypes.data


def check(L, rc):
    if rc != 0:
        raise RuntimeError(L.rh_last_error().decode())


def bf16_round(a):
    return S.bf16_bits_to_f32(S.f32_to_bf16_bits(np.asarray(a, np.float32))).astype(np.float64)


def rel_l2(got, want):
    num = np.linalg.norm((np.asarray(got, np.float64) - np.asarray(want, np.float64)).ravel())
    den = np.linalg.norm(np.asarray(want, np.float64).ravel())
    return float(num / den) if den > 0 else float(num)


def test_registry_rules_and_registrations():
    line = hook().rh_registry_selftest()
    assert line == 0, f"registry self-test failed at rows_hook.cpp:{line}"


def test_scratch_ledger_without_a_card():
    """The ledger's bookkeeping that needs no device memory (src/adjoint/device/scratch.h:15-48): a
    request of no bytes, and a null or unknown block returned, change nothing."""
    L = hook()
    assert L.rh_scratch_reset() == 0
    assert scratch(L) == (0, 0, 0)
    assert L.rh_scratch_alloc(0) is None and L.rh_scratch_alloc(-8) is None
    L.rh_scratch_free(None)
    L.rh_scratch_free(C.c_void_p(0x1000))
    assert scratch(L) == (0, 0, 0)


@pytest.mark.gpu
def test_scratch_ledger_rows_return_their_scratch():
    """A row's device buffers are scratch of its call: the ledger reports the call's peak and holds
    nothing once the row returns, as the reference's device tests read it
    (tests/support/device_check.h:252-262); a block still held makes the reset throw, naming the bytes."""
    from gpu_util import stored_operand

    print("case scratch ledger over a gemm_nt row", flush=True)
    L = hook()
    M, N, K = 96, 256, 384
    rng = np.random.default_rng(5)
    planes = S.trellis(rows=N, cols=K, bits=5, state_bits=16, run_rows=128, rb=1, mad=1, scale_dtype=S.F32,
                       rowf=True, seed=3)
    keep = []
    enc, raw = stored_operand(planes, keep)
    dy, dx = rng.standard_normal((M, N)), np.zeros((M, K))
    assert L.rh_scratch_reset() == 0
    check(L, L.rh_gemm_nt(M, N, K, p(dy), C.addressof(enc), raw.data_ptr(), None, p(dx)))
    live, peak, allocs = scratch(L)
    print(f"  live {live} peak {peak} allocations {allocs}", flush=True)
    # the row's uploads (dy as a bf16 [hi | lo] pair) and its f32 result at least
    assert live == 0 and allocs >= 2 and peak >= M * N * 4 + M * K * 4
    blk = L.rh_scratch_alloc(4096)
    assert blk and scratch(L)[0] == 4096
    assert L.rh_scratch_reset() == -1 and "4096 bytes" in L.rh_last_error().decode()
    L.rh_scratch_free(blk)
    assert L.rh_scratch_reset() == 0 and scratch(L) == (0, 0, 0)


@pytest.mark.gpu
@pytest.mark.parametrize("form", ["lut-bf16", "mad-rb", "e4m3-scale1"])
def test_gemm_nt_row_other_forms(form):
    """A stored weight in a form the kernels do not decode themselves (a stored LUT with bf16 block
    scales, rb > 1 row blocks, e4m3 block scales with scale.1) reaches the row through the same
    stored-weight store, prepared once into the int8-code form."""
    from gpu_util import host_weight, stored_operand
    from oracle import oracle as O

    print(f"case gemm_nt stored form {form}", flush=True)
    L = hook()
    M, N, K = 72, 256, 384
    rng = np.random.default_rng(len(form))
    kw = {"lut-bf16": dict(bits=4, state_bits=16, run_rows=128, rb=1, mad=0, scale_dtype=S.BF16),
          "mad-rb": dict(bits=4, state_bits=16, run_rows=128, rb=8, mad=1, scale_dtype=S.F32, rowf=True),
          "e4m3-scale1": dict(bits=5, state_bits=12, run_rows=128, rb=1, mad=0, scale_dtype=S.E4M3, second=True)}[form]
    planes = S.trellis(rows=N, cols=K, seed=7, **kw)
    keep = []
    enc, raw = stored_operand(planes, keep)
    dy = rng.standard_normal((M, N))
    dx0 = rng.standard_normal((M, K))
    dx = dx0.copy()
    check(L, L.rh_gemm_nt(M, N, K, p(dy), C.addressof(enc), raw.data_ptr(), None, p(dx)))
    codes, scale = host_weight(planes)
    want = O.gemm_nt_adjoint(dy, codes, scale, dx=dx0)
    e = rel_l2(dx - dx0, want - dx0)
    print(f"  rel L2 dx {e:.3e}", flush=True)
    assert e <= TOL_STORED


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,dense", [(96, 256, 384, False), (200, 512, 256, False), (64, 384, 256, True)])
def test_gemm_nt_row(M, N, K, dense):
    from gpu_util import host_weight, stored_operand
    from oracle import oracle as O

    print(f"case gemm_nt M={M} N={N} K={K} dense={dense}", flush=True)
    L = hook()
    rng = np.random.default_rng(M + N + K)
    dy = rng.standard_normal((M, N))
    dx0 = rng.standard_normal((M, K))
    dx = dx0.copy()
    if dense:
        W = bf16_round(0.02 * rng.standard_normal((N, K)))
        check(L, L.rh_gemm_nt(M, N, K, p(dy), None, None, p(W), p(dx)))
        want = dx0 + dy @ W
    else:
        planes = S.trellis(rows=N, cols=K, bits=5, state_bits=16, run_rows=128, rb=1, mad=1, scale_dtype=S.F32,
                           rowf=True, seed=M, scale_col=(0.75 + 0.5 * rng.random(K // 128)).astype(np.float32))
        keep = []
        enc, raw = stored_operand(planes, keep)
        check(L, L.rh_gemm_nt(M, N, K, p(dy), C.addressof(enc), raw.data_ptr(), None, p(dx)))
        codes, scale = host_weight(planes)
        want = O.gemm_nt_adjoint(dy, codes, scale, dx=dx0)
        # a second call reuses the prepared weight
        before = L.rh_weights_prepared()
        dx2 = dx0.copy()
        check(L, L.rh_gemm_nt(M, N, K, p(dy), C.addressof(enc), raw.data_ptr(), None, p(dx2)))
        assert L.rh_weights_prepared() == before and np.array_equal(dx2, dx)
    e = rel_l2(dx - dx0, want - dx0)
    print(f"  rel L2 dx {e:.3e}", flush=True)
    assert e <= (TOL if dense else TOL_STORED)


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,R,S,fused", [(128, 256, 16, 1, False), (200, 384, 8, 2, False), (160, 256, 32, 3, True)])
def test_lora_shrink_row(M, K, R, S, fused):
    from oracle import oracle as O

    print(f"case lora_shrink M={M} K={K} R={R} S={S} fused={fused}", flush=True)
    L = hook()
    rng = np.random.default_rng(M + K + R + S)
    x = bf16_round(rng.standard_normal((M, K)))
    la = bf16_round(0.02 * rng.standard_normal((S, R, K)))
    slot = rng.integers(-1, S + 1, M).astype(np.float64)  # -1 and S are base rows
    ct = rng.standard_normal((M, R))
    dx0 = rng.standard_normal((M, K))
    dx = dx0.copy()
    dA = np.zeros(S * R * K, np.float32)
    check(L, L.rh_lora_shrink(M, K, R, S, p(x), p(slot), p(la), p(ct), p(dx), p(dA), int(fused)))
    ref_dx, ref_da = O.lora_shrink_adjoint(x, slot, la, ct.astype(np.float32).astype(np.float64), dx=dx0, fused=True)
    e_dx = rel_l2(dx - dx0, ref_dx - dx0)
    e_da = rel_l2(dA, ref_da.ravel())
    print(f"  rel L2 dx {e_dx:.3e} dA {e_da:.3e}", flush=True)
    assert e_dx <= TOL and e_da <= TOL


@pytest.mark.gpu
@pytest.mark.parametrize("op,M,N,R,S,scaled,fused,in_place",
                         [("lora_expand", 128, 256, 16, 1, True, False, True),
                          ("lora_expand", 200, 384, 8, 2, True, False, False),
                          ("lora_expand", 96, 256, 64, 2, False, True, False),
                          ("lora_expand_mm", 200, 384, 8, 2, True, False, True),
                          ("lora_expand_mm", 96, 256, 64, 2, False, True, False)])
def test_lora_expand_row(op, M, N, R, S, scaled, fused, in_place):
    """The expand's device row, and lora_expand_mm's (the same adjoint: the mm form rounds t to bf16
    in its twin only, src/adjoint/host/lora.cpp:33-35), against the oracle's host adjoint."""
    from oracle import oracle as O

    print(f"case {op} M={M} N={N} R={R} S={S} scaled={scaled} fused={fused} in_place={in_place}", flush=True)
    L = hook()
    rng = np.random.default_rng(M + N + R + S + 7)
    t = rng.standard_normal((M, R)).astype(np.float32).astype(np.float64)
    lb = bf16_round(0.02 * rng.standard_normal((S, N, R)))
    slot = rng.integers(-1, S + 1, M).astype(np.float64)
    scale = (1.0 + rng.random((S, N))) if scaled else None
    cy = rng.standard_normal((M, N))
    tc0 = rng.standard_normal((M, R))
    tc = tc0.copy()
    dB = np.zeros(S * N * R, np.float32)
    base = np.zeros((M, N))
    check(L, L.rh_lora_expand_op(op.encode(), M, N, R, S, p(t), p(slot), p(lb), p(scale), p(cy), p(tc), p(dB),
                                 int(fused), int(in_place), p(base)))
    ref_dt, ref_db = O.lora_expand_adjoint(t, slot, lb, scale if scaled else np.ones((S, N)), cy, dt=tc0,
                                           fused=True)
    e_dt = rel_l2(tc - tc0, ref_dt - tc0)
    # the fused leaf is [N, S*R]; one leaf a slot is that leaf's slot columns
    want_db = ref_db if fused else ref_db.reshape(N, S, R).transpose(1, 0, 2)
    got_db = dB.reshape(N, S * R) if fused else dB.reshape(S, N, R)
    e_db = rel_l2(got_db, want_db)
    print(f"  rel L2 dt {e_dt:.3e} dB {e_db:.3e}", flush=True)
    assert e_dt <= TOL and e_db <= TOL
    if in_place:
        assert np.array_equal(base, cy)


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,R,S,fused", [(32, 200, 12, 1, False), (20, 128, 100, 2, True)])
def test_lora_shrink_row_any_rank_and_width(M, K, R, S, fused):
    """A rank the kernels do not run at (12: padded to 16; 100: a chunk of 64 and one of 36, padded
    to 64) and a K off a multiple of 128 (200: padded to 256) are served exactly."""
    from oracle import oracle as O

    print(f"case lora_shrink padded M={M} K={K} R={R} S={S} fused={fused}", flush=True)
    L = hook()
    rng = np.random.default_rng(M + K + R)
    x = bf16_round(rng.standard_normal((M, K)))
    la = bf16_round(0.02 * rng.standard_normal((S, R, K)))
    slot = np.array([-1 if m == 1 else (S if m == 2 else m % S) for m in range(M)], np.float64)
    ct = rng.standard_normal((M, R)).astype(np.float32).astype(np.float64)
    dx0 = rng.standard_normal((M, K))
    dx = dx0.copy()
    dA = np.zeros(S * R * K, np.float32)
    check(L, L.rh_lora_shrink(M, K, R, S, p(x), p(slot), p(la), p(ct), p(dx), p(dA), int(fused)))
    ref_dx, ref_da = O.lora_shrink_adjoint(x, slot, la, ct, dx=dx0, fused=True)
    e_dx, e_da = rel_l2(dx - dx0, ref_dx - dx0), rel_l2(dA, ref_da.ravel())
    print(f"  rel L2 dx {e_dx:.3e} dA {e_da:.3e}", flush=True)
    assert e_dx <= TOL and e_da <= TOL


@pytest.mark.gpu
def test_grad_stage_flush_rounds_once():
    """The step's staging (r97/grad_stage.h, the reference's src/adjoint/device/grad_stage.cpp): a
    block is zeroed on the first ask and the same buffer after; a second shape under the name is
    refused; the flush adds bf16(total) (RNE) into an existing leaf and makes a missing one."""
    L = hook()
    L.rh_stage_flush.argtypes = [_P, _P, _P, C.c_int64, _P, _P]
    rng = np.random.default_rng(9)
    n = 5000
    a = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    a[:3] = [1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8)]  # ties: to the even bf16 significand
    b = rng.standard_normal(n).astype(np.float32)
    base = rng.standard_normal(n).astype(np.float32)
    out, out_y = np.zeros(n, np.float32), np.zeros(n, np.float32)
    line = L.rh_stage_flush(p(a), p(b), p(base), n, p(out), p(out_y))
    assert line == 0, f"stage check failed at rows_hook.cpp:{line}"
    rb = lambda x: S.bf16_bits_to_f32(S.f32_to_bf16_bits(x))
    assert np.array_equal(out, base + rb(a)) and np.array_equal(out_y, rb(b))
    assert out[0] - base[0] == np.float32(1.0) and out[1] - base[1] != np.float32(1.0 + 3 * 2 ** -8)
