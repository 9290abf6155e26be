"""The int8-code form on the card: every weight form the decode reads (the reference's decode case
list, tests/host/iqr_decode.cpp:465-492, and its affine grids, :344-391) prepared once into the
fused kernels' tiled int8 codes + transposed bf16 scale, then run through the same fused forward and
dX kernels as the trellis forms.

Bars: the prepared codes and scale are the oracle's decode (the reference's r97_iqr_decode values and
its scale.col fold), bit for bit; the kernels' decoded tile read back through an identity operand is
bf16(code * scale), bit for bit; Y and dX are within the base products' relative L2 2e-3 of the f64
host rows. On a trellis form the int8-code kernels and the trellis kernels compute the same bits."""
import numpy as np
import pytest
import torch

import iqr_synth as S
from gpu_util import bf16_tensor, dev, device_desc, f64, host_weight, rel_l2
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL_BASE = 2e-3


def forms():
    out = [(name, c) for name, c in S.decode_cases(run_rows=256)]
    out.append(("affine-bf16", dict(affine=True, rows=256, cols=384, bits=4, zero_bits=4, scale_dtype=S.BF16, seed=7)))
    out.append(("affine-f16", dict(affine=True, rows=384, cols=256, bits=3, zero_bits=8, scale_dtype=S.F16, seed=8)))
    return out


FORMS = forms()


def planes_of(c):
    c = dict(c)
    if c.pop("affine", False):
        return S.affine(c["rows"], c["cols"], c["bits"], c["zero_bits"], c["scale_dtype"], seed=c["seed"])
    return S.trellis(**c)


def prepare(p, keep, codes8=False):
    from r9700training_amd.qlinear import QWeight

    d = device_desc(p, keep)
    sc = None
    if p.scale_col is not None:
        sc = dev(p.scale_col)
        keep.append(sc)
    return QWeight(d, scale_col=sc, codes8=codes8)


def untile(w):
    """The prepared int8-code form back in the reference's grids: codes [N, K], scale bits [N, K/128]."""
    N, K = w.rows, w.cols
    # unit byte 16*(c>>1) + 2*i + (c&1): [n8][k4][c>>1][i][c&1]
    units = w.stream_plane.cpu().numpy().view(np.int8)[: N * K].reshape(N // 8, K // 4, 2, 8, 2)
    codes = units.transpose(0, 3, 1, 2, 4).reshape(N, K)
    scale = w.scale_t.cpu().numpy().view(np.uint16).reshape(K // 128, N).T
    return codes, scale


def decoded_tile(codes, scale):
    return S.bf16_bits_to_f32(S.f32_to_bf16_bits(
        codes.astype(np.float32) * np.repeat(S.bf16_bits_to_f32(scale), 128, axis=1)))


@pytest.mark.parametrize("name,c", FORMS, ids=[f[0] for f in FORMS])
def test_prepared_form_is_the_decode(name, c):
    """Every form: the prepared int8 codes and scale are the oracle's decode, bit for bit (forms the
    kernels decode themselves are asked for the int8-code form explicitly)."""
    print(f"case codes8 prepare {name}", flush=True)
    p = planes_of(c)
    keep = []
    w = prepare(p, keep, codes8=True)
    auto = prepare(p, keep)
    torch.cuda.synchronize()
    codes, scale = host_weight(p)
    got_codes, got_scale = untile(w)
    assert np.array_equal(got_codes, codes)
    assert np.array_equal(got_scale, scale.astype(np.uint16))
    # the automatic choice: the trellis kernels where they serve the form, else the int8-code form
    trellis_served = (not p.affine and p.mad and p.rb == 1 and p.state_bits == 16 and 3 <= p.bits <= 6
                      and p.rows % 32 == 0 and p.run_rows % 32 == 0)
    assert auto.codes8 == (not trellis_served)
    if auto.codes8:
        a_codes, a_scale = untile(auto)
        assert np.array_equal(a_codes, codes) and np.array_equal(a_scale, got_scale)


KERNEL_FORMS = [f for f in FORMS if f[1]["rows"] % 128 == 0]


@pytest.mark.parametrize("name,c", KERNEL_FORMS, ids=[f[0] for f in KERNEL_FORMS])
def test_kernels_read_the_decode(name, c):
    """An identity operand reads the fused kernels' decoded tile back: bf16(code * scale) exactly,
    in the forward (X = I) and in dX (dY = I)."""
    from r9700training_amd.qlinear import qlinear_lora_bwd, qlinear_lora_fwd

    print(f"case codes8 identity {name}", flush=True)
    p = planes_of(c)
    keep = []
    w = prepare(p, keep, codes8=True)
    N, K = p.rows, p.cols
    Wb = decoded_tile(*host_weight(p))
    Y, _ = qlinear_lora_fwd(w, torch.eye(K, dtype=torch.bfloat16, device="cuda"), y_dtype=torch.float32)
    dX, _, _ = qlinear_lora_bwd(w, None, torch.eye(N, dtype=torch.bfloat16, device="cuda"), dx_dtype=torch.float32)
    torch.cuda.synchronize()
    assert np.array_equal(Y.cpu().numpy().T.view(np.uint32), Wb.view(np.uint32))
    assert np.array_equal(dX.cpu().numpy().view(np.uint32), Wb.view(np.uint32))


@pytest.mark.parametrize("name", ["stored-u4", "embedding", "mad-rb", "lut-rb", "e4m3-128", "affine-bf16"])
@pytest.mark.parametrize("T,r", [(300, 16), (640, 0)])
def test_forward_backward_against_oracle(name, T, r):
    from r9700training_amd.qlinear import qlinear_lora_bwd, qlinear_lora_fwd

    print(f"case codes8 fwd/bwd {name} T={T} r={r}", flush=True)
    p = planes_of(dict(FORMS)[name])
    keep = []
    w = prepare(p, keep)
    assert w.codes8
    codes, scale = host_weight(p)
    rng = np.random.default_rng(T + r)
    N, K = p.rows, p.cols
    bf = lambda a: S.bf16_bits_to_f32(S.f32_to_bf16_bits(np.asarray(a, np.float32))).astype(np.float64)
    x, dy = bf(rng.standard_normal((T, K))), bf(rng.standard_normal((T, N)))
    if r:
        A, B = bf(0.01 * rng.standard_normal((r, K))), bf(0.01 * rng.standard_normal((N, r)))
        s = 2.0
        Y, t = qlinear_lora_fwd(w, bf16_tensor(x), bf16_tensor(A), bf16_tensor(B), s, y_dtype=torch.float32)
        dX, dA, dB = qlinear_lora_bwd(w, bf16_tensor(x), bf16_tensor(dy), bf16_tensor(A), bf16_tensor(B), t, s,
                                      dx_dtype=torch.float32)
        torch.cuda.synchronize()
        ref = O.qlinear_lora_reference(x, codes, scale, A, B, s, dy)
        assert rel_l2(f64(dA), ref["dA"]) <= 1e-4 and rel_l2(f64(dB), ref["dB"]) <= 1e-4
    else:
        Y, _ = qlinear_lora_fwd(w, bf16_tensor(x), y_dtype=torch.float32)
        dX, _, _ = qlinear_lora_bwd(w, None, bf16_tensor(dy), dx_dtype=torch.float32)
        torch.cuda.synchronize()
        ref = dict(y=O.gemm_nt_twin(x, codes, scale), dx=O.gemm_nt_adjoint(dy, codes, scale))
    ey, edx = rel_l2(f64(Y), ref["y"]), rel_l2(f64(dX), ref["dx"])
    print(f"  rel L2 Y {ey:.3e} dX {edx:.3e}", flush=True)
    assert ey <= TOL_BASE and edx <= TOL_BASE


@pytest.mark.parametrize("T,N,K,bits", [(1000, 384, 512, 5), (512, 256, 256, 3)])
def test_int8_form_matches_trellis_kernels_bits(T, N, K, bits):
    """A trunk trellis weight through both kernel forms: the same decoded tile and the same MFMA
    order, so the same bits (Y, dX and the adapter's grads), and QWeight.from_decoded of the
    standalone decode's grids gives them too."""
    from r9700training_amd.qlinear import QWeight, iqr_decode, qlinear_lora_bwd, qlinear_lora_fwd

    print(f"case codes8 vs trellis T={T} N={N} K={K} bits={bits}", flush=True)
    rng = np.random.default_rng(T)
    p = S.trellis(rows=N, cols=K, bits=bits, state_bits=16, run_rows=128, rb=1, mad=1, scale_dtype=S.F32,
                  rowf=True, seed=T, scale_col=(0.75 + 0.5 * rng.random(K // 128)).astype(np.float32))
    keep = []
    trellis = prepare(p, keep)
    coded = prepare(p, keep, codes8=True)
    assert not trellis.codes8 and coded.codes8
    # the standalone decode's canonical grids, then the scale.col fold as the reference's join does
    codes_d = torch.empty((N, K), dtype=torch.int8, device="cuda")
    scale_d = torch.empty((N, K // 128), dtype=torch.int16, device="cuda")
    iqr_decode(device_desc(p, keep), codes_d, scale_d)
    torch.cuda.synchronize()
    _, folded = host_weight(p)
    scale_d = torch.from_numpy(folded.astype(np.uint16).view(np.int16)).cuda()
    decoded = QWeight.from_decoded(codes_d, scale_d)
    r, s = 16, 2.0
    X = bf16_tensor(rng.standard_normal((T, K)))
    dY = bf16_tensor(rng.standard_normal((T, N)))
    A = bf16_tensor(0.01 * rng.standard_normal((r, K)))
    B = bf16_tensor(0.01 * rng.standard_normal((N, r)))
    outs = []
    for w in (trellis, coded, decoded):
        Y, t = qlinear_lora_fwd(w, X, A, B, s, y_dtype=torch.float32)
        dX, dA, dB = qlinear_lora_bwd(w, X, dY, A, B, t, s, dx_dtype=torch.float32)
        outs.append((Y, dX, dA, dB))
    torch.cuda.synchronize()
    for other in outs[1:]:
        for a, b in zip(outs[0], other):
            assert torch.equal(a, b)


def test_from_decoded_refusals():
    from r9700training_amd import R97qError
    from r9700training_amd.qlinear import QWeight

    with pytest.raises(R97qError, match="multiple"):
        QWeight.from_decoded(torch.zeros((12, 256), dtype=torch.int8, device="cuda"),
                             torch.zeros((12, 2), dtype=torch.int16, device="cuda"))
    with pytest.raises(ValueError):
        QWeight.from_decoded(torch.zeros((16, 256), dtype=torch.int8, device="cuda"),
                             torch.zeros((16, 3), dtype=torch.int16, device="cuda"))
