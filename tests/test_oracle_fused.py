"""The oracle's fused quantiser producers (rmsnorm_had_quant_i8g, gated_had_quant_i8g and
gate_had_quant_i8g; src/adjoint/host/quant.cpp:896-1405) and their elementwise parts
(src/adjoint/host/elementwise.cpp: rmsnorm, silu_mul, act_mul with act = sigmoid), pinned on the CPU.

The parts: bit for bit against the reference's own rows (golden vectors written from oracle/_ref,
and fresh inputs where oracle/_ref was built), closed forms, and central finite differences of the
twin for the adjoint. The fused rows themselves need radiance's rad_plugin.h, which the reference
tree does not hold, so they are not built: the forward is pinned as the reference's part followed
by the pinned quantiser plus the quantiser's half-step property, and the adjoint by central finite
differences of the straight-through surrogate
    L(x) = sum(g . live . H part(x) / s) + sum(g_out . part(x))     (live, s frozen at the base point)
whose gradient is the composition's; a composition with the rotation, the mask or the output term
dropped is shown to miss it."""
import glob
import os

import numpy as np
import pytest
from scipy.linalg import hadamard

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def have_ref():
    try:
        return O.ref() is not None
    except OSError:
        return False


def bf16r(a):
    a = np.asarray(a, np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


def inputs(part, rows, n, rng, scale=1.5):
    x0 = bf16r(rng.standard_normal((rows, 2 * n if part == "silu_mul" else n)) * scale)
    x1 = {"rmsnorm": bf16r(rng.standard_normal(n) * 0.3), "silu_mul": None,
          "sigmoid_mul": bf16r(rng.standard_normal((rows, n)))}[part]
    return x0, x1


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "part_*.npz"))),
                         ids=lambda p: os.path.basename(p)[5:-4])
def test_part_golden(path):
    z = np.load(path)
    part = str(z["part"])
    kw = dict(eps=float(z["eps"]), wadd=float(z["wadd"]), mult=float(z["mult"]))
    x1 = z["x1"] if "x1" in z else None
    assert np.array_equal(O.part_twin(part, z["x0"], x1, **kw), z["y"])
    dx0, dx1 = O.part_adjoint(part, z["x0"], x1, z["dy"], **kw)
    assert np.array_equal(dx0, z["dx0"])
    if "dx1" in z:
        assert np.array_equal(dx1, z["dx1"])


@pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built")
@pytest.mark.parametrize("part", ["rmsnorm", "silu_mul", "sigmoid_mul"])
def test_part_matches_reference_fresh(part):
    rng = np.random.default_rng(77)
    for rows, n, kw in [(1, 64, dict(eps=1e-6, wadd=1.0)), (9, 320, dict(eps=1e-5, wadd=0.0, mult=0.5)),
                        (4, 1000, dict(eps=3e-4, wadd=-0.25, mult=2.0))]:
        x0, x1 = inputs(part, rows, n, rng, scale=4.0)
        dy = rng.standard_normal((rows, n))
        assert np.array_equal(O.part_twin(part, x0, x1, **kw), O.part_twin(part, x0, x1, use_ref=True, **kw))
        a = O.part_adjoint(part, x0, x1, dy, **kw)
        b = O.part_adjoint(part, x0, x1, dy, use_ref=True, **kw)
        assert np.array_equal(a[0], b[0])
        if part == "sigmoid_mul":
            assert np.array_equal(a[1], b[1])


def test_part_closed_forms():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 256)) * 3.0
    # the norm without gain: each row's mean square is ms / (ms + eps); scale invariance at eps = 0
    y = O.part_twin("rmsnorm", x, None, eps=1e-6)
    ms = (x * x).mean(axis=1)
    assert np.allclose((y * y).mean(axis=1), ms / (ms + 1e-6), rtol=1e-12)
    assert np.allclose(O.part_twin("rmsnorm", 7.0 * x, None, eps=0.0), O.part_twin("rmsnorm", x, None, eps=0.0),
                       rtol=1e-12, atol=1e-14)
    # the gain enters as (w + wadd) * mult per column
    w = rng.standard_normal(256)
    g = O.part_twin("rmsnorm", x, w, eps=1e-6, wadd=0.5, mult=3.0)
    assert np.allclose(g, y * (w + 0.5) * 3.0, rtol=1e-13)
    # silu(0) = 0 and silu(g) * u at u = 1 is g * sigmoid(g); sigmoid(0) * b = b / 2
    gu = np.concatenate([np.zeros((2, 8)), np.ones((2, 8))], axis=1)
    assert not O.part_twin("silu_mul", gu).any()
    gv = np.linspace(-6, 6, 16).reshape(2, 8)
    s = O.part_twin("silu_mul", np.concatenate([gv, np.ones((2, 8))], axis=1))
    assert np.allclose(s, gv / (1.0 + np.exp(-gv)), rtol=1e-15)
    b = rng.standard_normal((2, 8))
    assert np.array_equal(O.part_twin("sigmoid_mul", np.zeros((2, 8)), b), b / 2)


def _fd_grad(f, x, h):
    g = np.zeros_like(x)
    flat, gf = x.reshape(-1), g.reshape(-1)
    for i in range(flat.size):
        keep = flat[i]
        flat[i] = keep + h
        up = f(x)
        flat[i] = keep - h
        dn = f(x)
        flat[i] = keep
        gf[i] = (up - dn) / (2 * h)
    return g


@pytest.mark.parametrize("part", ["rmsnorm", "silu_mul", "sigmoid_mul"])
def test_part_adjoint_finite_differences(part):
    rng = np.random.default_rng(11)
    rows, n = 2, 24
    x0, x1 = inputs(part, rows, n, rng)
    dy = rng.standard_normal((rows, n))
    kw = dict(eps=1e-5, wadd=0.5, mult=1.25) if part == "rmsnorm" else {}
    d0, d1 = O.part_adjoint(part, x0, x1, dy, **kw)
    fd0 = _fd_grad(lambda z: float((O.part_twin(part, z, x1, **kw) * dy).sum()), x0.copy(), 1e-6)
    assert np.allclose(d0, fd0, rtol=1e-6, atol=1e-7)
    if part == "sigmoid_mul":
        fd1 = _fd_grad(lambda z: float((O.part_twin(part, x0, z, **kw) * dy).sum()), x1.copy(), 1e-6)
        assert np.allclose(d1, fd1, rtol=1e-6, atol=1e-7)


def _rot(y, group):
    """The unnormalised Walsh-Hadamard transform of each group, by the butterfly stages in the
    reference's order, so the f64 values (and a clamp decision an ulp from the grid's edge) are the
    quantiser's own; equal to the Sylvester matrix product up to rounding."""
    rows, n = y.shape
    v = np.array(y, np.float64).reshape(rows, n // group, group)
    h = 1
    while h < group:
        w = v.reshape(rows, n // group, group // (2 * h), 2, h)
        a, b = w[:, :, :, 0, :].copy(), w[:, :, :, 1, :].copy()
        w[:, :, :, 0, :], w[:, :, :, 1, :] = a + b, a - b
        h *= 2
    return v.reshape(rows, n)


def test_rotation_is_sylvester():
    y = np.random.default_rng(2).standard_normal((3, 256))
    want = (y.reshape(3, 2, 128) @ hadamard(128).astype(np.float64)).reshape(3, 256)
    assert np.allclose(_rot(y, 128), want, rtol=1e-13, atol=1e-12)


PARTS = [("rmsnorm", dict(eps=1e-6, wadd=1.0)), ("silu_mul", {}), ("sigmoid_mul", {})]


@pytest.mark.parametrize("part,kw", PARTS, ids=[p for p, _ in PARTS])
@pytest.mark.parametrize("group", [32, 128])
def test_fused_forward(part, kw, group):
    rng = np.random.default_rng(group)
    rows, n = 5, 256
    x0, x1 = inputs(part, rows, n, rng)
    y, codes, scale = O.fused_quant(part, x0, x1, group, **kw)
    yr = O.part_twin(part, x0, x1, use_ref=True, **kw) if have_ref() else O.part_twin(part, x0, x1, **kw)
    assert np.array_equal(y, yr)
    c2, s2, _ = O.quant_act_i8g(yr, group, True)
    assert np.array_equal(codes, c2) and np.array_equal(scale, s2)
    # the half-step property: every code is the rotated value over its group's scale, rounded
    u = _rot(y, group) / np.repeat(scale, group, axis=1)
    assert np.abs(u - codes).max() <= 0.5 + 1e-9
    assert np.abs(codes).max() == 127 and (np.abs(codes) <= 127).all()


def _surrogate(part, x1_or_x0, which, other, group, g, live, s, g_out, kw):
    x0, x1 = (x1_or_x0, other) if which == 0 else (other, x1_or_x0)
    y = O.part_twin(part, x0, x1, **kw)
    v = _rot(y, group) / s
    out = float((g * live * v).sum())
    if g_out is not None:
        out += float((g_out * y).sum())
    return out


@pytest.mark.parametrize("part,kw", PARTS, ids=[p for p, _ in PARTS])
@pytest.mark.parametrize("shrink", [1.0, 0.6])
@pytest.mark.parametrize("with_out", [False, True])
def test_fused_adjoint_finite_differences(part, kw, shrink, with_out):
    """The composition's gradient against the straight-through surrogate's finite differences;
    shrink < 1 hands the adjoint a scale below the forward's, so the clamp mask engages."""
    rng = np.random.default_rng(int(shrink * 10) + with_out)
    rows, n, group = 2, 64, 32
    x0, x1 = inputs(part, rows, n, rng)
    y, _, scale = O.fused_quant(part, x0, x1, group, **kw)
    scale = scale * shrink
    s = np.repeat(scale, group, axis=1)
    u = _rot(y, group) * (1.0 / s)
    live = (np.abs(u) <= 127.0).astype(np.float64)
    if shrink < 1.0:
        assert 0 < live.sum() < live.size
    g = rng.standard_normal((rows, n))
    g_out = rng.standard_normal((rows, n)) if with_out else None
    d0, d1 = O.fused_quant_adjoint(part, x0, x1, group, scale, g, g_out, **kw)
    h = 1e-6
    fd0 = _fd_grad(lambda z: _surrogate(part, z, 0, x1, group, g, live, s, g_out, kw), x0.copy(), h)
    tol = dict(rtol=1e-5, atol=1e-5 * np.abs(fd0).max())
    assert np.allclose(d0, fd0, **tol)
    if part == "sigmoid_mul":
        fd1 = _fd_grad(lambda z: _surrogate(part, z, 1, x0, group, g, live, s, g_out, kw), x1.copy(), h)
        assert np.allclose(d1, fd1, rtol=1e-5, atol=1e-5 * np.abs(fd1).max())
    # the same check catches a composition missing a piece
    e = _rot(live * g / s, group) + (0.0 if g_out is None else g_out)
    assert np.allclose(O.part_adjoint(part, x0, x1, e, **kw)[0], fd0, **tol)
    wrong = [live * g / s + (0.0 if g_out is None else g_out),      # no rotation back
             _rot(g / s, group) + (0.0 if g_out is None else g_out)]  # no mask
    if with_out:
        wrong.append(_rot(live * g / s, group))                          # the output term dropped
    for w in wrong:
        if shrink == 1.0 and w is wrong[1]:
            continue  # the forward's own scale clamps nothing, so no mask is the right answer there
        assert not np.allclose(O.part_adjoint(part, x0, x1, w, **kw)[0], fd0, **tol)


def test_fused_refusals():
    x = np.zeros((2, 96))
    with pytest.raises(ValueError):
        O.fused_quant("rmsnorm", x, np.ones(96), 48)  # not a power of two
    with pytest.raises(ValueError):
        O.fused_quant_adjoint("sigmoid_mul", x, x, 32, np.zeros((2, 3)), x)  # a zero scale
