"""The fused quantiser producers on the card (r97q_fused_had_quant_i8g and its adjoint:
rmsnorm_had_quant_i8g, gated_had_quant_i8g, gate_had_quant_i8g) against the oracle's restatement of
the reference's host rows (src/adjoint/host/quant.cpp:896-1405 over src/adjoint/host/elementwise.cpp's
parts; pinned in tests/test_oracle_fused.py).

Bars: codes and scales bit for bit, and the part's output rounded to bf16 bit for bit (the kernel
forms the part in f64 as the host twins do; its exp and its row sum may differ from the host's by
an f64 ulp, which moves a code only for a value within an ulp of a rounding edge -- none in these
seeded cases). The adjoint within 2e-6 relative of the f64 composition (one f32 rounding of the
result, plus the f32 accumulate), with the f32 scale the forward wrote."""
import numpy as np
import pytest
import torch

import iqr_synth as S
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TORCH = {"bf16": torch.bfloat16, "f32": torch.float32, "f64": torch.float64}


def _inputs(part, rows, n, dtype, seed, spread=1.5):
    rng = np.random.default_rng(seed)
    x0 = rng.standard_normal((rows, 2 * n if part == "silu_mul" else n)) * spread
    x0 *= 1 + 3 * rng.random((rows, 1))
    x1 = {"rmsnorm": rng.standard_normal(n) * 0.3, "silu_mul": None,
          "sigmoid_mul": rng.standard_normal((rows, n))}[part]
    if part == "rmsnorm" and rows > 2:
        x0[2] = 0.0  # a zero row: rs = 1/sqrt(eps), y = 0, scale 1, codes 0
    if dtype != "f64":
        x0 = S.bf16_bits_to_f32(S.f32_to_bf16_bits(x0.astype(np.float32))) if dtype == "bf16" else x0.astype(np.float32)
        x0 = x0.astype(np.float64)
        if x1 is not None:
            x1 = (S.bf16_bits_to_f32(S.f32_to_bf16_bits(x1.astype(np.float32))) if dtype == "bf16"
                  else x1.astype(np.float32)).astype(np.float64)
    dev = lambda a: None if a is None else torch.tensor(a, dtype=torch.float64, device="cuda").to(TORCH[dtype])  # noqa
    return rng, x0, x1, dev(x0), dev(x1)


def _bf16_of(y):
    return S.f32_to_bf16_bits(y.astype(np.float32))


KW = {"rmsnorm": dict(eps=1e-6, wadd=1.0, mult=1.0), "silu_mul": {}, "sigmoid_mul": {}}
CASES = [(33, 256, 128), (5, 96, 32), (7, 1024, 1024), (3, 64, 1), (2, 48, 16), (16, 5120, 128), (4, 384, 64)]


@pytest.mark.parametrize("rows,n,group", CASES)
@pytest.mark.parametrize("part", ["rmsnorm", "silu_mul", "sigmoid_mul"])
@pytest.mark.parametrize("dtype", ["bf16", "f64"])
def test_fused_matches_oracle(part, rows, n, group, dtype):
    from r9700training_amd.quant import fused_had_quant_i8g, fused_had_quant_i8g_bwd

    print(f"case fused {part} rows={rows} n={n} group={group} {dtype}", flush=True)
    kw = KW[part]
    rng, x0, x1, d0, d1 = _inputs(part, rows, n, dtype, rows * 1000 + n + group)
    codes, scale, y = fused_had_quant_i8g(part, d0, d1, group, want_y=True, **kw)
    torch.cuda.synchronize()
    wy, wc, ws = O.fused_quant(part, x0, x1, group, **kw)
    assert np.array_equal(codes.cpu().numpy().astype(np.float64), wc)
    assert np.array_equal(scale.cpu().numpy(), ws.astype(np.float32))
    assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), _bf16_of(wy))

    g = torch.tensor(rng.standard_normal((rows, n)), dtype=torch.float32, device="cuda")
    go = torch.tensor(rng.standard_normal((rows, n)), dtype=torch.float32, device="cuda")
    base0 = torch.tensor(rng.standard_normal(tuple(d0.shape)), dtype=torch.float32, device="cuda")
    dx0, dx1 = fused_had_quant_i8g_bwd(part, d0, d1, group, scale, g, go, dx0=base0.clone(), **kw)
    torch.cuda.synchronize()
    s64 = scale.cpu().numpy().astype(np.float64)
    w0, w1 = O.fused_quant_adjoint(part, x0, x1, group, s64, g.cpu().numpy().astype(np.float64),
                                   go.cpu().numpy().astype(np.float64), **kw)
    got0 = dx0.cpu().numpy().astype(np.float64) - base0.cpu().numpy().astype(np.float64)
    assert np.allclose(got0, w0, rtol=2e-6, atol=2e-6 * np.abs(w0).max() + 4e-7 * np.abs(base0.cpu().numpy()).max())
    if part == "sigmoid_mul":
        assert np.allclose(dx1.cpu().numpy(), w1, rtol=2e-6, atol=2e-6 * np.abs(w1).max())


@pytest.mark.parametrize("part", ["rmsnorm", "silu_mul", "sigmoid_mul"])
def test_fused_mask_engaged(part):
    """A scale below the forward's (as a tape's cotangent may arrive against) clamps part of every
    group: the dropped elements must match the host rule |v / scale| > 127 exactly."""
    from r9700training_amd.quant import fused_had_quant_i8g, fused_had_quant_i8g_bwd

    rows, n, group = 9, 512, 128
    print(f"case fused mask {part}", flush=True)
    kw = KW[part]
    rng, x0, x1, d0, d1 = _inputs(part, rows, n, "bf16", 4242)
    _, scale, _ = fused_had_quant_i8g(part, d0, d1, group, **kw)
    small = (scale * 0.55).contiguous()
    g = torch.tensor(rng.standard_normal((rows, n)), dtype=torch.float32, device="cuda")
    dx0, dx1 = fused_had_quant_i8g_bwd(part, d0, d1, group, small, g, None, **kw)
    torch.cuda.synchronize()
    w0, w1 = O.fused_quant_adjoint(part, x0, x1, group, small.cpu().numpy().astype(np.float64),
                                   g.cpu().numpy().astype(np.float64), None, **kw)
    assert np.allclose(dx0.cpu().numpy(), w0, rtol=2e-6, atol=2e-6 * np.abs(w0).max())
    if dx1 is not None:
        assert np.allclose(dx1.cpu().numpy(), w1, rtol=2e-6, atol=2e-6 * np.abs(w1).max())


def test_fused_full_width_rows():
    """The reference test's largest shape (tests/gpu/adjoint_quant.cpp:61-67: 4096 x 5120, group
    128) for the norm, and the gate at its live width 6144 (48 groups)."""
    from r9700training_amd.quant import fused_had_quant_i8g, fused_had_quant_i8g_bwd

    for part, rows, n in [("rmsnorm", 4096, 5120), ("sigmoid_mul", 1024, 6144)]:
        print(f"case fused full {part} rows={rows} n={n}", flush=True)
        kw = KW[part]
        rng, x0, x1, d0, d1 = _inputs(part, rows, n, "bf16", rows + n)
        codes, scale, _ = fused_had_quant_i8g(part, d0, d1, 128, **kw)
        g = torch.tensor(rng.standard_normal((rows, n)), dtype=torch.float32, device="cuda")
        dx0, dx1 = fused_had_quant_i8g_bwd(part, d0, d1, 128, scale, g, None, **kw)
        torch.cuda.synchronize()
        wy, wc, ws = O.fused_quant(part, x0, x1, 128, **kw)
        assert np.array_equal(codes.cpu().numpy().astype(np.float64), wc)
        assert np.array_equal(scale.cpu().numpy(), ws.astype(np.float32))
        w0, _ = O.fused_quant_adjoint(part, x0, x1, 128, scale.cpu().numpy().astype(np.float64),
                                      g.cpu().numpy().astype(np.float64), None, **kw)
        assert np.allclose(dx0.cpu().numpy(), w0, rtol=2e-6, atol=2e-6 * np.abs(w0).max())


def test_fused_refusals():
    from r9700training_amd import R97qError
    from r9700training_amd.quant import fused_had_quant_i8g

    x = torch.zeros((4, 96), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(96, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(R97qError, match="power of two"):
        fused_had_quant_i8g("rmsnorm", x, w, 48)
    x2 = torch.zeros((1, 4096), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(R97qError, match="wider"):
        fused_had_quant_i8g("silu_mul", x2, None, 2048)
    with pytest.raises(ValueError):
        fused_had_quant_i8g("sigmoid_mul", x, None, 32)
    with pytest.raises(ValueError):
        fused_had_quant_i8g("tanh_mul", x, None, 32)


@pytest.mark.parametrize("part", ["rmsnorm", "silu_mul", "sigmoid_mul"])
@pytest.mark.parametrize("layout", [0, 1, 2])
def test_fused_device_row(part, layout):
    """The device rows, registered like the reference's (src/adjoint/device/quant.hip:959-961),
    called through the registry on the schema's record (layout 0), the live tape's (1: the part's
    output written beside the codes, the norm's phantom write ahead of them) and with a direct-path
    write over the input's buffer (2), against the oracle's composition; the norm with a read set
    that leaves two rows out."""
    import ctypes as C

    from test_rows import check, hook, p

    rows, n, group = 12, 256, 64
    print(f"case fused row {part} layout={layout}", flush=True)
    L = hook()
    L.rh_fused_quant.argtypes = ([C.c_int32, C.c_int64, C.c_int64, C.c_int64, C.c_int32] + [C.c_void_p] * 6 +
                                 [C.c_double] * 3 + [C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p])
    kw = dict(eps=1e-5, wadd=1.0, mult=1.25) if part == "rmsnorm" else {}
    full = dict(eps=1e-6, wadd=0.0, mult=1.0) | kw
    rng, x0, x1, _, _ = _inputs(part, rows, n, "bf16", 99 + layout)
    _, _, scale = O.fused_quant(part, x0, x1, group, **kw)
    scale = scale.astype(np.float32).astype(np.float64)
    g = rng.standard_normal((rows, n)).astype(np.float32).astype(np.float64)
    gout = rng.standard_normal((rows, n)).astype(np.float32).astype(np.float64) if layout >= 1 else None
    gdir = rng.standard_normal(x0.shape).astype(np.float32).astype(np.float64) if layout >= 2 else None
    read = np.array([r for r in range(rows) if r not in (3, 7)], np.int64) if part == "rmsnorm" else None
    dx0 = rng.standard_normal(x0.shape)
    dx1 = rng.standard_normal((rows, n)) if part == "sigmoid_mul" else np.zeros(1)
    base0, base1 = dx0.copy(), dx1.copy()
    zeros = np.zeros((rows, n))
    check(L, L.rh_fused_quant(("rmsnorm", "silu_mul", "sigmoid_mul").index(part), rows, n, group, layout, p(x0),
                              p(x1) if x1 is not None else None, p(scale), p(g),
                              p(gout if gout is not None else zeros), p(gdir) if gdir is not None else None,
                              full["eps"], full["wadd"], full["mult"], p(read) if read is not None else None,
                              len(read) if read is not None else -1, p(dx0), p(dx1)))
    # a write over the input's buffer of the part's own width (the norm's, the gate's) is the part's
    # output written in place, so its cotangent goes through the part (src/adjoint/host/quant.cpp:
    # 1345-1352); only the gated producer's, gate_up's 2n wide, is the direct path
    direct = gdir is not None and part == "silu_mul"
    g_part = gout if gdir is None or direct else gout + gdir
    w0, w1 = O.fused_quant_adjoint(part, x0, x1, group, scale, g, g_part, **kw)
    if read is not None:
        w0[[3, 7]] = 0.0
    want0 = base0 + w0 + (gdir if direct else 0.0)
    assert np.allclose(dx0, want0, rtol=2e-6, atol=2e-6 * np.abs(w0).max())
    if part == "sigmoid_mul":
        assert np.allclose(dx1, base1 + w1, rtol=2e-6, atol=2e-6 * np.abs(w1).max())


def test_fused_device_row_refuses_unserved_layout():
    """Five writes (the phantom, the codes, the scale, the output and a direct path) is not a layout
    the reference's row serves (src/adjoint/device/quant.hip:631-643): refused by name, nothing added."""
    import ctypes as C

    from test_rows import hook, p

    rows, n, group = 4, 128, 128
    L = hook()
    L.rh_fused_quant.argtypes = ([C.c_int32, C.c_int64, C.c_int64, C.c_int64, C.c_int32] + [C.c_void_p] * 6 +
                                 [C.c_double] * 3 + [C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p])
    x = np.ones((rows, n))
    dx0 = np.zeros((rows, n))
    rc = L.rh_fused_quant(0, rows, n, group, 3, p(x), p(np.ones(n)), p(np.ones((rows, 1))), p(x), p(x), p(x),
                          1e-6, 0.0, 1.0, None, -1, p(dx0), p(np.zeros(1)))
    assert rc == -1 and "not a layout this row serves" in L.rh_last_error().decode()
    assert not dx0.any()
