"""The fused path at the benchmark configurations' full layer shapes.

Every distinct projection shape of configs C2-C5 (T tokens, N outputs, K inputs, rank r), with
W as uniform trellis.mad b5 codes in 256-row runs, an f32 row scale and a scale.col plane, X and dY
N(0,1) bf16, A and B N(0, 0.01) bf16, s = 2 (inputs drawn on the card from a seeded generator).
What is checked:

* sampled token rows of Y and dX (the first, tile-edge, middle and last tokens, as
  tests/gpu/adjoint_linear.cpp samples them) against the oracle's restatement of the reference
  host rows (src/adjoint/host/linear.cpp, lora.cpp) on those rows, within relative L2 2e-3;
* every row at once through the column sums: sum_m Y[m] = (sum_m X[m]).W^T + s.(sum_m t[m]).B^T
  and sum_m dX[m] = (sum_m dY[m]).W + (sum_m dt[m]).A (the path is linear in the token rows),
  the right-hand products by the oracle on the one summed row, within 2e-3;
* t (all T x r), dA and dB (whole) against f64 products of the same bf16 inputs (float64 GEMMs
  in torch, an implementation independent of this library's kernels), within 1e-4. The oracle's
  own adapter loops walk dY with stride N and take minutes at these sizes; at small sizes
  test_gpu_qlinear.py holds t, dA and dB to the oracle itself;
* every element of Y and dX against the host rows' arithmetic done in float64 GEMMs on the card:
  the weight is the oracle's decode (code * scale in f64, the reference's weight value,
  src/adjoint/host/linear.cpp:118-190), Y = X.W^T + s.t.B^T and dX = dY.W + dt.A with t and dt the
  f64 products above; the whole tensor within relative L2 2e-3 and its worst row within 3e-3.
"""
import numpy as np
import pytest
import torch

import iqr_synth as S
from gpu_util import f64, host_weight, prepared, rel_l2
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL_BASE = 2e-3
TOL_ADAPTER = 1e-4

# (name, T, N, K, r): C2; C3 gate/up and down; C4 qkv+gate and out; C5 attn-in, attn-out, gate/up, down
SHAPES = [
    ("c2", 4096, 4096, 4096, 16),
    ("c3-gate-up", 8192, 12288, 4096, 32),
    ("c3-down", 8192, 4096, 12288, 32),
    ("c4-qkv-gate", 16384, 8192, 2048, 64),
    ("c4-out", 16384, 2048, 4096, 64),
    ("c5-attn-in", 32768, 8192, 2048, 16),
    ("c5-attn-out", 32768, 2048, 4096, 16),
    ("c5-gate-up", 32768, 6144, 2048, 16),
    ("c5-down", 32768, 2048, 6144, 16),
    # two of the reference's published shapes (docs/kernels/linear.md:261-268) whose tile counts
    # leave the CUs mostly idle, so the fused kernel splits their reductions (split-K): attn_k/v's
    # twin (64 tiles) and attn_qg's adjoint at 1024 tokens (80 tiles)
    ("ref-attn-kv", 4096, 1024, 5120, 16),
    ("ref-attn-qg-1024", 1024, 12288, 5120, 16),
    # and two whose 320 tiles fill one round and a quarter of another: the tiles of the partial
    # round split four ways (attn_qg's adjoint at 4096 tokens, ffn_down's twin), the rest whole
    ("ref-attn-qg-4096", 4096, 12288, 5120, 16),
    ("ref-ffn-down", 4096, 5120, 17408, 16),
]


def sample_rows(T, rng):
    edges = [0, 1, 63, 64, 511, 512, T // 2 - 1, T // 2, T - 513, T - 512, T - 65, T - 2, T - 1]
    return np.unique(np.concatenate([np.array(edges), rng.integers(0, T, 6)]))


@pytest.mark.parametrize("name,T,N,K,r", SHAPES, ids=[s[0] for s in SHAPES])
def test_full_shape(name, T, N, K, r):
    print(f"case {name} T={T} N={N} K={K} r={r}", flush=True)
    from r9700training_amd.qlinear import qlinear_lora_bwd, qlinear_lora_fwd

    seed = sum(map(ord, name))
    rng = np.random.default_rng(seed)
    sc = (0.75 + 0.5 * rng.random(K // 128)).astype(np.float32)
    p = S.trellis(rows=N, cols=K, bits=5, state_bits=16, run_rows=256, rb=1, mad=1, scale_dtype=S.F32,
                  rowf=True, seed=seed + 1, scale_col=sc, packed=True)
    keep = []
    w = prepared(p, keep)
    codes, scale = host_weight(p)
    g = torch.Generator(device="cuda").manual_seed(seed)
    randn = lambda shape, std=1.0: (std * torch.randn(shape, generator=g, device="cuda")).to(torch.bfloat16)
    Xd, dYd = randn((T, K)), randn((T, N))
    Ad, Bd = randn((r, K), 0.01), randn((N, r), 0.01)
    s = 2.0

    Y, t = qlinear_lora_fwd(w, Xd, Ad, Bd, s, y_dtype=torch.float32)
    dX, dA, dB = qlinear_lora_bwd(w, Xd, dYd, Ad, Bd, t, s, dx_dtype=torch.float32)
    torch.cuda.synchronize()

    # every element, against float64 GEMMs on the card over the oracle's decoded weight
    W64 = torch.from_numpy(codes).cuda().double() * torch.from_numpy(
        S.bf16_bits_to_f32(scale).astype(np.float64)).cuda().repeat_interleave(128, dim=1)
    X64, dY64, A64, B64 = Xd.double(), dYd.double(), Ad.double(), Bd.double()
    t64 = X64 @ A64.T.contiguous()
    dt64 = s * (dY64 @ B64)

    def whole(got, ref, what):
        err = got.double() - ref
        e = float(torch.linalg.vector_norm(err) / torch.linalg.vector_norm(ref))
        er = float((torch.linalg.vector_norm(err, dim=1) / torch.linalg.vector_norm(ref, dim=1)).max())
        print(f"  every element of {what}: rel L2 {e:.3e}, worst row {er:.3e}", flush=True)
        assert e <= TOL_BASE and er <= 1.5 * TOL_BASE, what

    whole(Y, X64 @ W64.T.contiguous() + s * (t64 @ B64.T.contiguous()), "Y")
    whole(dX, dY64 @ W64 + dt64 @ A64, "dX")
    del W64, X64, dY64, A64, B64, t64, dt64
    torch.cuda.empty_cache()
    rows = sample_rows(T, rng)
    ridx = torch.from_numpy(rows).cuda()
    got_y, got_dx = f64(Y.index_select(0, ridx)), f64(dX.index_select(0, ridx))
    ysum, dxsum = Y.sum(0, dtype=torch.float64).cpu().numpy(), dX.sum(0, dtype=torch.float64).cpu().numpy()
    got_t, got_dA, got_dB = t.double(), dA.double(), dB.double()
    del Y, dX
    torch.cuda.synchronize()

    # sampled rows, by the oracle
    host = lambda a: a.float().cpu().numpy()
    A, B = host(Ad), host(Bd)
    ref = O.qlinear_lora_reference(host(Xd.index_select(0, ridx)), codes, scale, A, B, s,
                                   host(dYd.index_select(0, ridx)))
    ey, edx = rel_l2(got_y, ref["y"]), rel_l2(got_dx, ref["dx"])
    print(f"  rows {rows.size}: rel L2  Y {ey:.3e}  dX {edx:.3e}", flush=True)
    assert ey <= TOL_BASE and edx <= TOL_BASE

    # the adapter's whole outputs, against float64 products
    X64, dY64, A64, B64 = Xd.double(), dYd.double(), Ad.double(), Bd.double()
    t_ref = X64 @ A64.T.contiguous()
    dt_ref = s * (dY64 @ B64)
    dB_ref = s * (dY64.T.contiguous() @ t_ref)
    dA_ref = dt_ref.T.contiguous() @ X64
    rel = lambda a, b: float(torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(b))
    et, eA, eB = rel(got_t, t_ref), rel(got_dA, dA_ref), rel(got_dB, dB_ref)
    print(f"  rel L2  t {et:.3e}  dA {eA:.3e}  dB {eB:.3e}", flush=True)
    assert et <= TOL_ADAPTER and eA <= TOL_ADAPTER and eB <= TOL_ADAPTER

    # every row through the column sums, the products by the oracle
    xsum, dysum = X64.sum(0).cpu().numpy(), dY64.sum(0).cpu().numpy()
    tsum, dtsum = t_ref.sum(0).cpu().numpy(), dt_ref.sum(0).cpu().numpy()
    del X64, dY64
    one = np.zeros(1)
    ysum_ref = O.lora_expand_twin(tsum[None], one, B.reshape(1, N, r), np.full((1, N), s),
                                  y=O.gemm_nt_twin(xsum[None], codes, scale))[0]
    dxsum_ref = O.gemm_nt_adjoint(dysum[None], codes, scale, dx=dtsum[None] @ A.astype(np.float64))[0]
    es, edxs = rel_l2(ysum, ysum_ref), rel_l2(dxsum, dxsum_ref)
    print(f"  column sums rel L2  Y {es:.3e}  dX {edxs:.3e}", flush=True)
    assert es <= TOL_BASE and edxs <= TOL_BASE


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_split_tail_accumulate(dtype):
    """dX added into an existing dX where the product splits only its partial last round: a 4096 x
    5120 weight at 4096 tokens has 8 x 40 = 320 dX tiles, so the first 256 run whole and the last 64
    split four ways over the 64-step reduction; the reduce launch adds the ranges in order and then
    into dX (f32, or bf16 with its one more rounding)."""
    T, N, K, r, s = 4096, 4096, 5120, 16, 2.0
    print(f"case split-tail dX T={T} N={N} K={K} {dtype}", flush=True)
    from r9700training_amd.qlinear import qlinear_lora_bwd, qlinear_lora_fwd

    seed = 4099
    rng = np.random.default_rng(seed)
    sc = (0.75 + 0.5 * rng.random(K // 128)).astype(np.float32)
    p = S.trellis(rows=N, cols=K, bits=5, state_bits=16, run_rows=256, rb=1, mad=1, scale_dtype=S.F32,
                  rowf=True, seed=seed + 1, scale_col=sc, packed=True)
    keep = []
    w = prepared(p, keep)
    codes, scale = host_weight(p)
    g = torch.Generator(device="cuda").manual_seed(seed)
    randn = lambda shape, std=1.0: (std * torch.randn(shape, generator=g, device="cuda")).to(torch.bfloat16)
    Xd, dYd = randn((T, K)), randn((T, N))
    Ad, Bd = randn((r, K), 0.01), randn((N, r), 0.01)
    dX0 = (0.5 * torch.randn((T, K), generator=g, device="cuda")).to(dtype)
    _, t = qlinear_lora_fwd(w, Xd, Ad, Bd, s, y_dtype=torch.float32)
    dX, _, _ = qlinear_lora_bwd(w, Xd, dYd, Ad, Bd, t, s, dX=dX0.clone(), accumulate=True)
    torch.cuda.synchronize()
    W64 = torch.from_numpy(codes).cuda().double() * torch.from_numpy(
        S.bf16_bits_to_f32(scale).astype(np.float64)).cuda().repeat_interleave(128, dim=1)
    dY64 = dYd.double()
    ref = dX0.double() + dY64 @ W64 + (s * (dY64 @ Bd.double())) @ Ad.double()
    e = float(torch.linalg.vector_norm(dX.double() - ref) / torch.linalg.vector_norm(ref))
    print(f"  dX (+)= rel L2 {e:.3e}", flush=True)
    assert e <= (TOL_BASE if dtype == torch.float32 else 1.3 * TOL_BASE)
