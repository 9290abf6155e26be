"""The CPU oracle pinned before it is trusted.

Each check is chosen so a plausible mistake fails it: the golden vectors written by the
reference's own host rows (tests/golden/make_golden.py), the reference rows themselves when
oracle/_ref was built, and independent closed forms / invariants (exhaustive format tables from
numpy and torch, a numpy restatement of the state walk, f64 matmul, finite differences, the
adjoint identity, chunk == whole).
"""
import glob
import hashlib
import os

import numpy as np
import pytest
import torch

import iqr_synth as S
from oracle import oracle as O

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def have_ref():
    return O.ref() is not None


# ------------------------------------------------------------------ scalar formats
def test_bf16_to_f32_exhaustive():
    L = O.lib()
    bits = np.arange(1 << 16, dtype=np.uint16)
    got = np.array([L.orc_bf16_to_f32(int(b)) for b in bits], np.float32)
    want = S.bf16_bits_to_f32(bits)
    # ctypes hands the value back through a double, which quiets a signalling NaN: NaNs are
    # compared as NaN, every other value bit for bit
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_bf16_matches_torch_rne():
    L = O.lib()
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.4e38, -3.4e38, 1e-40, np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    got = np.array([L.orc_f32_to_bf16(float(v)) for v in vals], np.uint16)
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    # NaN: quiet bit set, payload kept (src/iqr_decode.h:121)
    nan = np.array([0x7F800001], np.uint32).view(np.float32)[0]
    assert L.orc_f32_to_bf16(float(nan)) & 0x7FC0 == 0x7FC0


def test_f16_to_f32_exhaustive():
    L = O.lib()
    bits = np.arange(1 << 16, dtype=np.uint16)
    got = np.array([L.orc_f16_to_f32(int(b)) for b in bits], np.float32)
    want = bits.view(np.float16).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))
    assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)])


def test_e4m3_to_f32_exhaustive():
    L = O.lib()
    bits = np.arange(256, dtype=np.uint8)
    got = np.array([L.orc_e4m3_to_f32(int(b)) for b in bits], np.float32)
    want = torch.from_numpy(bits).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])


# ------------------------------------------------------------------ state value
@pytest.mark.parametrize("A,B", [(0x1, 0x0), (0xABCDEF, 0x12345678), (0xFFFFFF, 0xFFFFFFFF)])
def test_state_value_all_states(A, B):
    d = O.Desc()
    d.mad, d.mad_a, d.mad_b = 1, A, B
    L = O.lib()
    got = np.array([L.orc_state_value(d, st) for st in range(1 << 16)], np.int64)
    assert np.array_equal(got, S.mad_lut(A, B, 16).astype(np.int64))
    assert got.min() >= -126 and got.max() <= 126


# ------------------------------------------------------------------ decode
def planes_from(z):
    p = S.Planes(rows=int(z["rows"]), cols=int(z["cols"]), bits=int(z["bits"]),
                 state_bits=int(z["state_bits"]), run_rows=int(z["run_rows"]), rb=int(z["rb"]),
                 mad=int(z["mad"]), round_mad=int(z["round_mad"]), mad_a=int(z["mad_a"]),
                 mad_b=int(z["mad_b"]), scale_dtype=int(z["scale_dtype"]),
                 scale_block_cols=int(z["scale_block_cols"]), affine=int(z["affine"]),
                 zero_bits=int(z["zero_bits"]))
    p.codes = z["codes"].copy()
    p.scale = z["scale"].copy()
    if "lut" in z:
        p.lut = z["lut"].copy()
    if "scale2" in z:
        p.scale2 = z["scale2"].copy()
        p.scale2_dtype = int(z["scale2_dtype"])
        p.scale2_row_bytes = int(z["scale2_row_bytes"])
    if "zero" in z:
        p.zero = z["zero"].copy()
    return p


DECODE_FILES = sorted(glob.glob(os.path.join(G, "decode_*.npz")))
DECODE_FILES = [f for f in DECODE_FILES if "digest" not in f]


@pytest.mark.parametrize("path", DECODE_FILES, ids=lambda p: os.path.basename(p)[7:-4])
def test_decode_golden(path):
    z = np.load(path)
    p = planes_from(z)
    assert O.validate(p.desc()) == 0
    codes, scale = O.decode(p.desc())
    assert np.array_equal(codes, z["out_codes"])
    assert np.array_equal(scale, z["out_scale"])
    # a chunk at a run boundary equals the whole's rows
    if p.affine:
        c = O.decode(p.desc(row0=128, rows=100))
        assert np.array_equal(c[0], z["chunk_codes"]) and np.array_equal(c[1], z["chunk_scale"])
        assert np.array_equal(c[0], codes[128:228])
    else:
        run = p.run_rows
        c = O.decode(p.desc(row0=run, rows=run))
        assert np.array_equal(c[0], z["chunk_codes"]) and np.array_equal(c[1], z["chunk_scale"])
        assert np.array_equal(c[0], codes[run:2 * run]) and np.array_equal(c[1], scale[run:2 * run])
    if "short_chunk_refused" in z:
        assert O.validate(p.desc(rows=p.rows - (p.run_rows // 2 + 4))) == int(z["short_chunk_refused"]) == 1


def test_decode_trunk256_digest():
    z = np.load(os.path.join(G, "decode_trunk256_digest.npz"))
    p = S.trellis(rows=768, cols=512, bits=5, state_bits=16, run_rows=256, rb=1, mad=1,
                  scale_dtype=S.F32, rowf=True, seed=int(z["seed"]))
    codes, scale = O.decode(p.desc())
    assert hashlib.sha256(codes.tobytes()).hexdigest() == str(z["codes_sha"])
    assert hashlib.sha256(scale.tobytes()).hexdigest() == str(z["scale_sha"])


def window_decode(p: S.Planes):
    """Independent numpy statement of the trellis decode for rb = 1: the state of row n is the
    last ceil(L/b) codes of its column, the rows before the run's first wrapping to the run's end,
    masked to L bits; the value is the state's codebook entry; the scale is the block's."""
    raw = S.unpack_rows(p.codes, p.bits, p.cols).astype(np.int64)
    c = -(-p.state_bits // p.bits)
    st = np.zeros_like(raw)
    for r0 in range(0, p.rows, p.run_rows):
        r1 = min(r0 + p.run_rows, p.rows)
        n = np.arange(r0, r1)
        acc = np.zeros((r1 - r0, p.cols), np.int64)
        for q in range(c):
            src = r0 + (n - r0 - q) % (r1 - r0)
            acc |= raw[src] << (q * p.bits)
        st[r0:r1] = acc & ((1 << p.state_bits) - 1)
    return p.lut[st]


@pytest.mark.parametrize("bits,L,run", [(5, 16, 256), (3, 16, 64), (4, 12, 32), (6, 16, 128)])
def test_decode_matches_window_statement(bits, L, run):
    p = S.trellis(rows=2 * run + run // 2, cols=256, bits=bits, state_bits=L, run_rows=run, mad=1,
                  scale_dtype=S.BF16, seed=bits * 100 + L)
    codes, _ = O.decode(p.desc())
    assert np.array_equal(codes, window_decode(p))


@pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built")
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_decode_matches_reference_fresh(seed):
    for name, kw in S.decode_cases(run_rows=32):
        kw = dict(kw, seed=kw["seed"] + 17 * seed)
        p = S.trellis(**kw)
        a = O.decode(p.desc())
        b = O.decode(p.desc(), use_ref=True)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]), name


def test_validate_refusals():
    p = S.trellis(rows=128, cols=256, bits=5, run_rows=64, seed=5)
    ok = p.desc()
    assert O.validate(ok) == 0
    cases = {
        "cols not /128": dict(cols=200),
        "row0 off a run": dict(row0=32),
        "rb not dividing run": dict(rb=3),
        "bits 0": dict(bits=0),
        "state bits 25": dict(state_bits=25),
        "no codebook": dict(mad=0, lut=None),
        "rows past end": dict(rows=256),
        "run shorter than seam": dict(run_rows=2, rows=128),
    }
    for name, ch in cases.items():
        d = O.Desc.from_buffer_copy(ok)
        for k, v in ch.items():
            setattr(d, k, v)
        assert O.validate(d) == 1, name
        if have_ref():
            assert O.validate(d, use_ref=True) == 1, name


def test_fold_scale_col_one_rounding():
    rng = np.random.default_rng(3)
    row = (rng.random(64) * 1e-3).astype(np.float32)
    fac = (0.5 + rng.random(8)).astype(np.float32)
    got = O.fold_scale_col(row, fac)
    want = S.f32_to_bf16_bits((row[:, None] * fac[None, :]).astype(np.float32))
    assert np.array_equal(got, want)
    # two roundings (bf16(row) then the product) differ somewhere: the test has teeth
    two = S.f32_to_bf16_bits(S.bf16_bits_to_f32(S.f32_to_bf16_bits(row))[:, None] * fac[None, :])
    assert not np.array_equal(got, two)


# ------------------------------------------------------------------ gemm_nt
def w_of(codes, scale):
    K = codes.shape[1]
    return codes.astype(np.float64) * np.repeat(S.bf16_bits_to_f32(scale).astype(np.float64), 128, axis=1)[:, :K]


@pytest.mark.parametrize("name", ["small", "wide", "tall"])
def test_gemm_nt_golden(name):
    z = np.load(os.path.join(G, f"linear_{name}.npz"))
    y = O.gemm_nt_twin(z["x"], z["codes"], z["scale"])
    dx = O.gemm_nt_adjoint(z["dy"], z["codes"], z["scale"], dx=z["dx0"])
    assert np.array_equal(y, z["y"])
    assert np.array_equal(dx, z["dx"])
    W = w_of(z["codes"], z["scale"])
    np.testing.assert_allclose(y, z["x"] @ W.T, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dx, z["dx0"] + z["dy"] @ W, rtol=1e-12, atol=1e-12)
    # the adjoint identity <dy, twin(x)> == <adj(dy), x>
    adj = O.gemm_nt_adjoint(z["dy"], z["codes"], z["scale"])
    assert abs(np.sum(z["dy"] * y) - np.sum(adj * z["x"])) < 1e-9 * np.abs(np.sum(z["dy"] * y)) + 1e-12


def test_gemm_nt_rows_subset_and_threads():
    z = np.load(os.path.join(G, "linear_small.npz"))
    full = O.gemm_nt_twin(z["x"], z["codes"], z["scale"])
    rows = np.array([0, 3, 5])
    part = O.gemm_nt_twin(z["x"], z["codes"], z["scale"], rows=rows)
    assert np.array_equal(part[rows], full[rows])
    O.set_threads(1)
    try:
        one = O.gemm_nt_twin(z["x"], z["codes"], z["scale"])
    finally:
        O.set_threads(0)
    assert np.array_equal(one, full)


# ------------------------------------------------------------------ LoRA
LORA = ["tiny_q_proj", "tiny_gate_proj", "tiny_down_proj"]


@pytest.mark.parametrize("name", LORA)
def test_lora_golden(name):
    z = np.load(os.path.join(G, f"lora_{name}.npz"))
    t = O.lora_shrink_twin(z["x"], z["slot"], z["la"])
    assert np.array_equal(t, z["t"])
    assert np.array_equal(O.lora_expand_twin(z["t"], z["slot"], z["lb"], z["sc"]), z["y"])
    assert np.array_equal(O.lora_expand_twin(z["t"], z["slot"], z["lb"], z["sc"], mm=True), z["y_mm"])
    for fused in (0, 1):
        dx, da = O.lora_shrink_adjoint(z["x"], z["slot"], z["la"], z["ct"], fused=bool(fused))
        dt, db = O.lora_expand_adjoint(z["t"], z["slot"], z["lb"], z["sc"], z["cy"], fused=bool(fused))
        assert np.array_equal(dx, z[f"dx_f{fused}"])
        assert np.array_equal(da, z[f"da_f{fused}"])
        assert np.array_equal(dt, z[f"dt_f{fused}"])
        assert np.array_equal(db, z[f"db_f{fused}"])


def slot_matrix(slot, S_):
    s = np.where((slot >= 0) & (slot < S_), slot, -1).astype(np.int64)
    return s


@pytest.mark.parametrize("name", LORA)
def test_lora_closed_forms_and_base_rows(name):
    z = np.load(os.path.join(G, f"lora_{name}.npz"))
    x, slot, la, lb, sc, ct, cy = (z[k] for k in ("x", "slot", "la", "lb", "sc", "ct", "cy"))
    S_, R, K = la.shape
    N = lb.shape[1]
    s = slot_matrix(slot, S_)
    t = O.lora_shrink_twin(x, slot, la)
    dx, da = O.lora_shrink_adjoint(x, slot, la, ct, fused=True)
    dt, db = O.lora_expand_adjoint(t, slot, lb, sc, cy, fused=True)
    for m in range(x.shape[0]):
        if s[m] < 0:  # a base row is neither read nor written
            assert not t[m].any() and not dx[m].any() and not dt[m].any()
            continue
        np.testing.assert_allclose(t[m], la[s[m]] @ x[m], rtol=1e-12)
        np.testing.assert_allclose(dx[m], ct[m] @ la[s[m]], rtol=1e-12, atol=1e-15)
        np.testing.assert_allclose(dt[m], (cy[m] * sc[s[m]]) @ lb[s[m]], rtol=1e-12, atol=1e-15)
    for q in range(S_):
        rows = s == q
        np.testing.assert_allclose(da[q * R:(q + 1) * R], ct[rows].T @ x[rows], rtol=2e-6, atol=1e-6)
        np.testing.assert_allclose(db[:, q * R:(q + 1) * R], (cy[rows] * sc[q]).T @ t[rows], rtol=2e-6, atol=1e-6)


def test_lora_finite_differences():
    """Central differences of the twins at eps 1e-6 (tests/support/adjoint_check.h:342-510)."""
    z = np.load(os.path.join(G, "lora_tiny_q_proj.npz"))
    x, slot, la, lb, sc = (z[k] for k in ("x", "slot", "la", "lb", "sc"))
    rng = np.random.default_rng(0)
    ct = rng.standard_normal((x.shape[0], la.shape[1]))
    dx, _ = O.lora_shrink_adjoint(x, slot, la, ct)
    eps = 1e-6
    for (m, k) in [(0, 3), (3, 100), (5, 127)]:
        xp, xm = x.copy(), x.copy()
        xp[m, k] += eps
        xm[m, k] -= eps
        fd = np.sum(ct * (O.lora_shrink_twin(xp, slot, la) - O.lora_shrink_twin(xm, slot, la))) / (2 * eps)
        assert abs(fd - dx[m, k]) <= 1e-6 * max(1.0, abs(fd))
    t = O.lora_shrink_twin(x, slot, la)
    cy = rng.standard_normal((x.shape[0], lb.shape[1]))
    dt, _ = O.lora_expand_adjoint(t, slot, lb, sc, cy)
    for (m, j) in [(0, 0), (4, 15), (3, 7)]:
        tp, tm = t.copy(), t.copy()
        tp[m, j] += eps
        tm[m, j] -= eps
        fd = np.sum(cy * (O.lora_expand_twin(tp, slot, lb, sc) - O.lora_expand_twin(tm, slot, lb, sc))) / (2 * eps)
        assert abs(fd - dt[m, j]) <= 1e-6 * max(1.0, abs(fd))


def test_lora_b_zero_start():
    """B = 0 (the adapter's start): dt = 0 and dA = 0 while dB != 0 (docs/adjoints/lora.md)."""
    z = np.load(os.path.join(G, "lora_tiny_gate_proj.npz"))
    x, slot, la, sc, cy = (z[k] for k in ("x", "slot", "la", "sc", "cy"))
    lb = np.zeros_like(z["lb"])
    t = O.lora_shrink_twin(x, slot, la)
    dt, db = O.lora_expand_adjoint(t, slot, lb, sc, cy)
    _, da = O.lora_shrink_adjoint(x, slot, la, dt)
    assert not dt.any() and not da.any() and np.abs(db).max() > 0


@pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built")
def test_rows_match_reference_fresh():
    rng = np.random.default_rng(99)
    M, N, K, R = 7, 256, 384, 8
    p = S.trellis(rows=N, cols=K, bits=5, run_rows=128, rowf=True, seed=9,
                  scale_col=(0.5 + rng.random(K // 128)).astype(np.float32))
    codes, _ = O.decode(p.desc())
    scale = O.fold_scale_col(p.scale.view(np.float32).reshape(-1), p.scale_col)
    x = rng.standard_normal((M, K))
    dy = rng.standard_normal((M, N))
    assert np.array_equal(O.gemm_nt_twin(x, codes, scale), O.gemm_nt_twin(x, codes, scale, use_ref=True))
    assert np.array_equal(O.gemm_nt_adjoint(dy, codes, scale), O.gemm_nt_adjoint(dy, codes, scale, use_ref=True))
    slot = np.array([0, 1, -1, 0, 2, 1, 0], np.float64)
    la = rng.standard_normal((2, R, K))
    lb = rng.standard_normal((2, N, R))
    sc = rng.random((2, N))
    ct = rng.standard_normal((M, R))
    t = O.lora_shrink_twin(x, slot, la)
    assert np.array_equal(t, O.lora_shrink_twin(x, slot, la, use_ref=True))
    for fused in (False, True):
        a = O.lora_shrink_adjoint(x, slot, la, ct, fused=fused)
        b = O.lora_shrink_adjoint(x, slot, la, ct, fused=fused, use_ref=True)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
        a = O.lora_expand_adjoint(t, slot, lb, sc, dy, fused=fused)
        b = O.lora_expand_adjoint(t, slot, lb, sc, dy, fused=fused, use_ref=True)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_c1_reference_composition():
    """Config 1 composed from the oracle equals the reference rows' composition (digests)."""
    z = np.load(os.path.join(G, "c1_reference.npz"))
    rng = np.random.default_rng(int(z["seed"]))
    T, N, K, R = (int(z[k]) for k in ("T", "N", "K", "R"))
    bf = lambda a: S.bf16_bits_to_f32(S.f32_to_bf16_bits(np.asarray(a, np.float32))).astype(np.float64)
    factor = (0.75 + 0.5 * rng.random(K // 128)).astype(np.float32)
    assert np.array_equal(factor, z["factor"])
    p = S.trellis(rows=N, cols=K, bits=5, state_bits=16, run_rows=256, rb=1, mad=1,
                  scale_dtype=S.F32, rowf=True, seed=1001, scale_col=factor)
    codes, _ = O.decode(p.desc())
    scale = O.fold_scale_col(p.scale.view(np.float32).reshape(-1), factor)
    assert hashlib.sha256(codes.tobytes()).hexdigest() == str(z["codes_sha"])
    assert hashlib.sha256(scale.tobytes()).hexdigest() == str(z["scale_sha"])
    x = bf(rng.standard_normal((T, K)))
    dy = bf(rng.standard_normal((T, N)))
    A = bf(0.01 * rng.standard_normal((R, K)))
    B = bf(0.01 * rng.standard_normal((N, R)))
    out = O.qlinear_lora_reference(x, codes, scale, A, B, float(z["s"]), dy)
    assert np.array_equal(out["t"], z["t"])
    assert np.array_equal(out["dA"], z["dA"]) and np.array_equal(out["dB"], z["dB"])
    assert np.array_equal(out["y"][[0, 1, 63, 127]], z["y_rows"])
    assert np.array_equal(out["dx"][[0, 1, 63, 127]], z["dx_rows"])
    assert hashlib.sha256(out["y"].tobytes()).hexdigest() == str(z["y_sha"])
    assert hashlib.sha256(out["dx"].tobytes()).hexdigest() == str(z["dx_sha"])


# ------------------------------------------------------------------ the coded (i8a8h) trunk
def test_group_width_reference_cases_and_property():
    # lora.cpp:64-69: 300 over three columns is groups of 128, 128, 44; one column spans the row
    assert O.group_width(300, 3) == 128 and O.group_width(300, 1) == 300 and O.group_width(256, 2) == 128
    assert O.group_width(0, 3) == 1
    for k in range(1, 700, 7):
        for groups in range(1, 9):
            w = O.group_width(k, groups)
            # every column's group index k // w stays inside the stream's `groups` columns
            assert -(-k // w) <= groups and w >= -(-k // groups), (k, groups, w)
    # a power-of-two width that splits k into exactly `groups` groups is the one read back
    for p2 in (16, 64, 128, 256):
        for groups in (2, 3, 5, 8):
            for tail in (0, 1, p2 // 2, p2 - 1):
                k = (groups - 1) * p2 + (tail if tail else p2)
                assert O.group_width(k, groups) == p2, (k, groups)


@pytest.mark.parametrize("name", ["q_small", "q_one", "q_odd"])
def test_gemm_nt_q_golden_and_closed_form(name):
    z = np.load(os.path.join(G, f"linear_{name}.npz"))
    a, a_scale, dy, da0, codes, scale = (z[k] for k in ("a", "a_scale", "dy", "da0", "codes", "scale"))
    y = O.gemm_nt_q_twin(a, a_scale, codes, scale)
    da = O.gemm_nt_q_adjoint(dy, codes, scale, a_scale, da=da0)
    assert np.array_equal(y, z["y"])
    assert np.array_equal(da, z["da"])
    # closed forms: x = a * a_scale (per row, group), W = code * scale
    K = a.shape[1]
    x = a * np.repeat(a_scale, 128, axis=1)[:, :K]
    W = w_of(codes, scale)
    np.testing.assert_allclose(y, x @ W.T, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(da, da0 + (dy @ W) * np.repeat(a_scale, 128, axis=1)[:, :K], rtol=1e-12, atol=1e-12)
    # the code basis: <dy, twin(a + e)> - <dy, twin(a)> == <adj(dy), e> with the scale held
    e = np.random.default_rng(3).standard_normal(a.shape)
    lhs = np.sum(dy * O.gemm_nt_q_twin(a + e, a_scale, codes, scale)) - np.sum(dy * y)
    rhs = np.sum(O.gemm_nt_q_adjoint(dy, codes, scale, a_scale) * e)
    assert abs(lhs - rhs) <= 1e-9 * (abs(lhs) + 1.0)
    # a wrong basis (the value-space cotangent, no a_scale) fails the identity
    bad = np.sum((dy @ W) * e)
    assert abs(lhs - bad) > 1e-3 * abs(lhs)


@pytest.mark.parametrize("name", ["coded_q_proj", "coded_down_proj", "coded_up_proj"])
def test_lora_shrink_q_golden_and_closed_forms(name):
    z = np.load(os.path.join(G, f"lora_{name}.npz"))
    a, a_scale, slot, la, ct = (z[k] for k in ("a", "a_scale", "slot", "la", "ct"))
    t = O.lora_shrink_q_twin(a, a_scale, slot, la)
    assert np.array_equal(t, z["t"])
    for fused in (0, 1):
        da, ds, dA = O.lora_shrink_q_adjoint(a, a_scale, slot, la, ct, fused=bool(fused))
        assert np.array_equal(da, z[f"da_f{fused}"])
        assert np.array_equal(ds, z[f"ds_f{fused}"])
        assert np.array_equal(dA, z[f"dA_f{fused}"])
    S_, R, K = la.shape
    groups = a_scale.shape[1]
    gw = O.group_width(K, groups)
    gidx = np.arange(K) // gw
    x = a * a_scale[:, gidx]
    s = slot_matrix(slot, S_)
    da, ds, dA = O.lora_shrink_q_adjoint(a, a_scale, slot, la, ct, fused=True)
    for m in range(a.shape[0]):
        if s[m] < 0:
            assert not t[m].any() and not da[m].any() and not ds[m].any()
            continue
        g = ct[m] @ la[s[m]]
        np.testing.assert_allclose(t[m], la[s[m]] @ x[m], rtol=1e-12)
        np.testing.assert_allclose(da[m], g * a_scale[m, gidx], rtol=1e-12, atol=1e-15)
        np.testing.assert_allclose(ds[m], np.bincount(gidx, weights=g * a[m], minlength=groups), rtol=1e-10,
                                   atol=1e-12)
        # the scale cotangent is the twin's derivative in the scale: d<ct, t>/d a_scale[m, q]
        for q in range(groups):
            hsc = a_scale.copy()
            h = 1e-6 * a_scale[m, q]
            hsc[m, q] += h
            tp = O.lora_shrink_q_twin(a, hsc, slot, la)
            hsc[m, q] -= 2 * h
            tm = O.lora_shrink_q_twin(a, hsc, slot, la)
            fd = (np.sum(ct * tp) - np.sum(ct * tm)) / (2 * h)
            assert abs(fd - ds[m, q]) <= 1e-6 * (abs(ds[m, q]) + 1e-3)
    for q in range(S_):
        rows = s == q
        np.testing.assert_allclose(dA[q * R:(q + 1) * R], ct[rows].T @ x[rows], rtol=2e-6, atol=1e-6)


@pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built")
def test_coded_rows_match_reference_fresh():
    rng = np.random.default_rng(77)
    M, N, K = 5, 128, 256
    codes = rng.integers(-126, 127, size=(N, K)).astype(np.int8)
    scale = S.f32_to_bf16_bits((1e-3 * (0.5 + rng.random((N, K // 128)))).astype(np.float32))
    a = np.rint(rng.uniform(-60, 60, (M, K)))
    a_scale = (0.01 + 0.05 * rng.random((M, K // 128))).astype(np.float32).astype(np.float64)
    dy = rng.standard_normal((M, N))
    assert np.array_equal(O.gemm_nt_q_twin(a, a_scale, codes, scale),
                          O.gemm_nt_q_twin(a, a_scale, codes, scale, use_ref=True))
    assert np.array_equal(O.gemm_nt_q_adjoint(dy, codes, scale, a_scale),
                          O.gemm_nt_q_adjoint(dy, codes, scale, a_scale, use_ref=True))
    slot = np.array([0, -1, 2, 1, 0], np.float64)
    la = S.bf16_bits_to_f32(S.f32_to_bf16_bits(rng.standard_normal((2, 8, K)).astype(np.float32))).astype(np.float64)
    ct = rng.standard_normal((M, 8))
    got = O.lora_shrink_q_adjoint(a, a_scale, slot, la, ct)
    want = O.lora_shrink_q_adjoint(a, a_scale, slot, la, ct, use_ref=True)
    for g_, w_ in zip(got, want):
        assert np.array_equal(g_, w_)


# ------------------------------------------------------------------ AdamW
def test_adamw_schedule_and_clip_known_answers():
    """tests/host/optim.cpp:134-164: the schedule's values and the 3-4-5 clip."""
    cfg = O.AdamWConfig.make(lr=2e-3, warmup_steps=10, total_steps=100, lr_floor_frac=0.1)
    floor = 2e-3 * 0.1
    assert O.scheduled_lr(cfg, 0) == 0.0
    assert abs(O.scheduled_lr(cfg, 1) - 2e-3 * 0.1) < 1e-6 and abs(O.scheduled_lr(cfg, 5) - 2e-3 * 0.5) < 1e-6
    assert abs(O.scheduled_lr(cfg, 10) - 2e-3) < 1e-6
    assert abs(O.scheduled_lr(cfg, 55) - 0.5 * (floor + 2e-3)) < 1e-6
    assert abs(O.scheduled_lr(cfg, 100) - floor) < 1e-6 and abs(O.scheduled_lr(cfg, 500) - floor) < 1e-6
    nocos = O.AdamWConfig.make(lr=3e-3)
    assert O.scheduled_lr(nocos, 1) == np.float32(3e-3) and O.scheduled_lr(nocos, 77) == np.float32(3e-3)
    g = [np.array([3.0, 4.0], np.float32)]
    assert abs(O.clip_global_norm(g, 2.5) - 5.0) < 1e-5
    assert abs(g[0][0] - 1.5) < 1e-5 and abs(g[0][1] - 2.0) < 1e-5
    O.clip_global_norm(g, 100.0)
    assert abs(g[0][0] - 1.5) < 1e-5


def test_adamw_golden_and_f64_restatement():
    z = np.load(os.path.join(G, "adamw_runs.npz"))
    params0 = [z[f"w{i}"] for i in range(3)]
    grads = [[z[f"g{s}_{i}"] for i in range(3)] for s in range(6)]
    for name in ("plain", "schedule_clip_decay", "accumulate"):
        kw = {"plain": {}, "schedule_clip_decay": dict(lr=1e-2, warmup_steps=2, total_steps=5, lr_floor_frac=0.1,
                                                       weight_decay=0.05, clip_norm=1.0),
              "accumulate": dict(lr=3e-3, accum_steps=2, clip_norm=1e3)}[name]
        cfg = O.AdamWConfig.make(**kw)
        opt = O.AdamW(cfg, [p.copy() for p in params0], decay=list(z["decay"]))
        for g in grads:
            opt.step(g)
        for i in range(3):
            for k, arr in (("w", opt.w), ("m", opt.m), ("v", opt.v), ("acc", opt.acc)):
                assert np.array_equal(arr[i], z[f"{name}_{k}{i}"]), (name, k, i)
        assert opt.step_count.value == z[f"{name}_updates"] and opt.pending.value == z[f"{name}_pending"]
    # an f64 restatement of the plain run (tests/host/optim.cpp:35-46), to 1e-6
    cfg = O.AdamWConfig.make()
    w = [p.astype(np.float64) for p in params0]
    m = [np.zeros_like(x) for x in w]
    v = [np.zeros_like(x) for x in w]
    for t, g in enumerate(grads, start=1):
        for i in range(3):
            m[i] = 0.9 * m[i] + 0.1 * g[i]
            v[i] = 0.999 * v[i] + 0.001 * g[i].astype(np.float64) ** 2
            mh, vh = m[i] / (1 - 0.9 ** t), v[i] / (1 - 0.999 ** t)
            w[i] = w[i] - 1e-3 * (mh / (np.sqrt(vh) + 1e-8))
    for i in range(3):
        assert np.max(np.abs(w[i] - z[f"plain_w{i}"])) < 1e-6


# ---------------------------------------------------------------- the vocabulary head
def _vocab_classes(rng, K, sizes, vocab, offset, stray=0):
    """Classes of random int8 rows with bf16 row scales, ids a shuffle of this rank's vocabulary
    (plus `stray` ids outside it), and a scale.col each."""
    ids_all = rng.permutation(vocab) + offset
    out, at = [], 0
    for n in sizes:
        ids = ids_all[at:at + n].astype(np.int32)
        at += n
        if stray:
            ids[:stray] = offset + vocab + rng.integers(0, 50, stray)  # past the vocabulary
            ids[stray:2 * stray] = offset - 1 - rng.integers(0, max(offset, 1), stray)  # before it
        codes = rng.integers(-127, 128, (n, K)).astype(np.int8)
        gscale = S.f32_to_bf16_bits((0.001 + 0.01 * rng.random((n, 1))).astype(np.float32)).repeat(K // 128, 1)
        cf = (0.5 + rng.random(K // 128)).astype(np.float32)
        out.append((codes, gscale.astype(np.uint16), ids, cf))
    return out


def test_fwht128_is_the_sylvester_hadamard():
    import scipy.linalg

    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 384))
    H = scipy.linalg.hadamard(128).astype(np.float64)
    want = np.concatenate([x[:, b:b + 128] @ H.T for b in range(0, 384, 128)], axis=1)
    assert np.allclose(O.fwht128(x), want, rtol=0, atol=1e-12)
    assert np.allclose(O.fwht128(O.fwht128(x)), 128 * x, rtol=0, atol=1e-10)


def test_vocab_head_one_hot_known_answer():
    """The reference test's check (tests/gpu/vocab_head.cpp): a one-hot cotangent row per class
    selects that class's weight row, scaled by its row scale and the class's scale.col; the transform
    follows."""
    rng = np.random.default_rng(5)
    K, vocab, rows = 256, 900, 4
    cls = _vocab_classes(rng, K, [300, 400, 200], vocab, 0)
    dy = np.zeros((rows, vocab), np.uint16)
    picks = []
    for m in range(rows):
        for c, (codes, gscale, ids, cf) in enumerate(cls):
            r = 17 * m + 5 * c + 3
            dy[m, ids[r]] = 0x3F80  # 1.0
            picks.append((m, c, r))
    want = np.zeros((rows, K))
    for m, c, r in picks:
        codes, gscale, ids, cf = cls[c]
        want[m] += (codes[r].astype(np.float64) * S.bf16_bits_to_f32(gscale[r]).astype(np.float64).repeat(128)
                    * np.repeat(cf.astype(np.float64), 128))
    for transform in (0, 128):
        got = O.vocab_head_transpose(dy, cls, transform=transform)
        ref = want if transform == 0 else O.fwht128(want)
        assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    # teeth: the scale.col dropped, the transform doubled
    no_cf = [(c, g, i, np.ones_like(f)) for c, g, i, f in cls]
    assert not np.allclose(O.vocab_head_transpose(dy, no_cf, transform=128), O.fwht128(want))
    assert not np.allclose(O.vocab_head_transpose(dy, cls, transform=128), 2 * O.fwht128(want))


def test_vocab_head_matches_matmul_and_ignores_stray_ids():
    rng = np.random.default_rng(9)
    K, vocab, offset, rows = 384, 1500, 700, 9
    cls = _vocab_classes(rng, K, [500, 600, 300], vocab, offset, stray=6)
    dy = S.f32_to_bf16_bits(rng.standard_normal((rows, vocab)).astype(np.float32))
    d0 = rng.standard_normal((rows, K))
    want = d0.copy()
    dyf = S.bf16_bits_to_f32(dy).astype(np.float64)
    for codes, gscale, ids, cf in cls:
        inside = (ids >= offset) & (ids < offset + vocab)
        g = np.zeros((rows, len(ids)))
        g[:, inside] = dyf[:, ids[inside] - offset]
        W = codes.astype(np.float64) * np.repeat(S.bf16_bits_to_f32(gscale).astype(np.float64), 128, axis=1)
        want += (g @ W) * np.repeat(cf.astype(np.float64), 128)
    got = O.vocab_head_transpose(dy, cls, vocab_offset=offset, d_x=d0)
    assert np.allclose(got, want, rtol=1e-10, atol=1e-9)
    # the transform runs over the whole of d_x once the classes are in
    got_t = O.vocab_head_transpose(dy, cls, vocab_offset=offset, transform=128, d_x=d0)
    assert np.allclose(got_t, O.fwht128(want), rtol=1e-10, atol=1e-8)


# ---------------------------------------------------------------- the activation quantiser
def _scanned_amax():
    """tests/host/adjoint_quant.cpp:236-243: the first a = 1 + k/64 whose own scale clamps it."""
    for k in range(64):
        a = 1.0 + k / 64.0
        s = a * (1.0 / 127.0)
        if abs(a * (1.0 / s)) > 127.0:
            return a
    raise AssertionError("no clamping amax")


@pytest.mark.parametrize("rotated", [False, True])
def test_quant_saturated_group_known_answers(rotated):
    """tests/host/adjoint_quant.cpp:332-370: the clamped code and its scale, the masked cotangent,
    an inside code's cotangent divided by the scale and rotated back."""
    a = _scanned_amax()
    scale = a * (1.0 / 127.0)
    x = np.array([[0.75 * a, 0.25 * a]]) if rotated else np.array([[a, 0.5 * a, -0.25 * a, 0.125 * a]])
    n = x.shape[1]
    codes, sc, live = O.quant_act_i8g(x, n, rotated)
    assert codes[0, 0] == 127.0 and sc[0, 0] == scale
    g = np.zeros((1, n))
    g[0, 0] = 1.0
    assert not O.quant_act_i8g_adjoint(x, sc, g, n, rotated).any()
    g = np.zeros((1, n))
    g[0, 1] = 1.0
    dx = O.quant_act_i8g_adjoint(x, sc, g, n, rotated)
    want = [1.0 / scale, -1.0 / scale] if rotated else [0.0, 1.0 / scale, 0.0, 0.0]
    assert np.array_equal(dx[0], want)


@pytest.mark.parametrize("rotated", [False, True])
def test_quant_zero_group_passes_through(rotated):
    """tests/host/adjoint_quant.cpp:378-430: the zero group's codes and scale, e0 back through the
    adjoint, and W (1, .., 1) = (t, 0, .., 0) for the rotation's transpose."""
    rows, n, group = (2, 8, 8) if rotated else (2, 6, 3)
    x = np.zeros((rows, n))
    codes, sc, _ = O.quant_act_i8g(x, group, rotated)
    assert not codes.any() and (sc == 1.0).all()
    first = np.zeros((rows, n))
    first[:, ::group] = 1.0
    dx = O.quant_act_i8g_adjoint(x, sc, first, group, rotated)
    assert np.array_equal(dx, np.ones((rows, n)) if rotated else first)
    dy = O.quant_act_i8g_adjoint(x, sc, np.ones((rows, n)), group, rotated)
    want = np.zeros((rows, n))
    want[:, ::group] = group
    assert np.array_equal(dy, want if rotated else np.ones((rows, n)))


@pytest.mark.parametrize("n,group,rotated", [(384, 128, False), (300, 128, False), (200, 0, False), (256, 64, True),
                                             (512, 512, True)])
def test_quant_against_numpy_and_the_transpose(n, group, rotated):
    """The codes against numpy's rint/clip over scipy's Hadamard (ties to even on exact halves);
    the adjoint is the transpose of the straight-through linearisation: <g, J e> == <J^T g, e>."""
    import scipy.linalg

    rng = np.random.default_rng(n + group)
    rows = 5
    x = S.bf16_bits_to_f32(S.f32_to_bf16_bits(rng.standard_normal((rows, n)).astype(np.float32))).astype(np.float64)
    x[1, :] = 0.0  # a zero row
    t = group if rotated else (n if group <= 0 or group > n else group)
    v = x.copy()
    if rotated:
        H = scipy.linalg.hadamard(t).astype(np.float64)
        v = np.concatenate([v[:, b:b + t] @ H.T for b in range(0, n, t)], axis=1)
    # exact halves: place u = k + 0.5 at a known scale in row 2's first group
    codes, sc, live = O.quant_act_i8g(x, group, rotated)
    ngrp = sc.shape[1]
    for r in range(rows):
        for gi in range(ngrp):
            seg = v[r, gi * t:(gi + 1) * t]
            amax = np.abs(seg).max()
            s = amax * (1.0 / 127.0) if amax > 0 else 1.0
            assert sc[r, gi] == s
            u = seg * (1.0 / s)
            assert np.array_equal(codes[r, gi * t:gi * t + len(seg)], np.clip(np.rint(u), -127, 127))
    # ties to even: a group whose values sit on halves of its own scale
    hx = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5]])
    hc, hs, _ = O.quant_act_i8g(hx, 0, False)
    assert hs[0, 0] == 1.0 and np.array_equal(hc[0], [127, 0, 2, 2, 0, -2])
    # transpose of the linearisation: J e = live * (W e) / s per group
    g = rng.standard_normal((rows, n))
    e = rng.standard_normal((rows, n))
    We = e.copy()
    if rotated:
        We = np.concatenate([We[:, b:b + t] @ H.T for b in range(0, n, t)], axis=1)
    Je = live * We / np.repeat(sc, t, axis=1)[:, :n]
    JTg = O.quant_act_i8g_adjoint(x, sc, g, group, rotated)
    assert abs((g * Je).sum() - (JTg * e).sum()) <= 1e-9 * (abs((g * Je).sum()) + 1)
