"""Write the golden vectors under tests/golden/ from the REFERENCE's own host rows.

Run in the build container, where oracle/_ref/libr97ref.so was compiled from the reference's host
sources (oracle/Makefile): every expected output below is what the reference's r97_iqr_decode_host
(src/iqr_decode.h:353-376), gemm_nt / gemm_nt_q twins and adjoints (src/adjoint/host/linear.cpp:
193-317), float / coded lora_shrink and lora_expand twins and adjoints
(src/adjoint/host/lora.cpp:204-521) and the AdamW Optimiser (src/optim.cpp) return for the
seeded inputs stored beside them. The fixtures are data only (inputs and expected outputs); the
reference's source never enters the repository.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

from oracle import oracle as O  # noqa: E402
import iqr_synth as S  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def bf16r(a):
    """round to the bf16 grid (RNE), as f64"""
    return S.bf16_bits_to_f32(S.f32_to_bf16_bits(np.asarray(a, np.float32))).astype(np.float64)


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def planes_dict(p: S.Planes):
    d = dict(rows=p.rows, cols=p.cols, bits=p.bits, state_bits=p.state_bits, run_rows=p.run_rows,
             rb=p.rb, mad=p.mad, round_mad=p.round_mad, mad_a=p.mad_a, mad_b=p.mad_b,
             scale_dtype=p.scale_dtype, scale_block_cols=p.scale_block_cols, affine=p.affine,
             codes=p.codes, scale=p.scale, zero_bits=p.zero_bits)
    if not p.mad and p.lut is not None:
        d["lut"] = p.lut
    if p.scale2 is not None:
        d["scale2"] = p.scale2
        d["scale2_dtype"] = p.scale2_dtype
        d["scale2_row_bytes"] = p.scale2_row_bytes
    if p.zero is not None:
        d["zero"] = p.zero
    return d


def decode_fixtures():
    for name, kw in S.decode_cases(run_rows=64):
        p = S.trellis(**kw)
        d = p.desc()
        assert O.validate(d, use_ref=True) == 0, name
        codes, scale = O.decode(d, use_ref=True)
        run = p.run_rows
        chunk = O.decode(p.desc(row0=run, rows=run), use_ref=True)
        extra = {}
        # a chunk ending inside the short last run must be refused (iqr_decode.cpp:334-338)
        if p.rows % run:
            bad = p.desc(rows=p.rows - (run // 2 + 4))
            extra["short_chunk_refused"] = O.validate(bad, use_ref=True)
        np.savez_compressed(os.path.join(OUT, f"decode_{name}.npz"), **planes_dict(p),
                            out_codes=codes, out_scale=scale, chunk_codes=chunk[0],
                            chunk_scale=chunk[1], **extra)
        print("decode", name, codes.shape)
    for name, kw in S.AFFINE_CASES:
        p = S.affine(**kw)
        codes, scale = O.decode(p.desc(), use_ref=True)
        chunk = O.decode(p.desc(row0=128, rows=100), use_ref=True)
        np.savez_compressed(os.path.join(OUT, f"decode_affine_{name}.npz"), **planes_dict(p),
                            out_codes=codes, out_scale=scale, chunk_codes=chunk[0],
                            chunk_scale=chunk[1])
        print("decode affine", name, codes.shape)
    # The trunk form at its real run length (256 rows, b5 L16 mad, f32 row scale): too large to
    # store whole, so the planes are regenerated from the seed and the outputs pinned by digest.
    p = S.trellis(rows=768, cols=512, bits=5, state_bits=16, run_rows=256, rb=1, mad=1,
                  scale_dtype=S.F32, rowf=True, seed=4242)
    codes, scale = O.decode(p.desc(), use_ref=True)
    np.savez_compressed(os.path.join(OUT, "decode_trunk256_digest.npz"), seed=4242, rows=768,
                        cols=512, codes_sha=digest(codes), scale_sha=digest(scale),
                        first_rows_codes=codes[:8], first_rows_scale=scale[:8])
    print("decode trunk256 digest")


def stored_weight(N, K, seed, scale_col=None):
    """A decoded trunk-form weight (int8 codes + folded bf16 scale) from the reference decode."""
    p = S.trellis(rows=N, cols=K, bits=5, state_bits=16, run_rows=min(256, N), rb=1, mad=1,
                  scale_dtype=S.F32, rowf=True, seed=seed, scale_col=scale_col)
    codes, scale = O.decode(p.desc(), use_ref=True)
    row = p.scale.view(np.float32).reshape(-1)
    folded = O.fold_scale_col(row, p.scale_col)
    return codes, folded


def linear_fixtures():
    rng = np.random.default_rng(7)
    sites = {"small": (6, 256, 256, 501), "wide": (5, 384, 128, 502), "tall": (3, 128, 512, 503)}
    for name, (M, N, K, seed) in sites.items():
        factor = (0.75 + 0.5 * rng.random(K // 128)).astype(np.float32)
        codes, scale = stored_weight(N, K, seed=seed, scale_col=factor)
        x = bf16r(rng.standard_normal((M, K)))
        dy = bf16r(rng.standard_normal((M, N)))
        dx0 = rng.standard_normal((M, K))  # the adjoint adds into what is there
        y = O.gemm_nt_twin(x, codes, scale, use_ref=True)
        dx = O.gemm_nt_adjoint(dy, codes, scale, dx=dx0, use_ref=True)
        np.savez_compressed(os.path.join(OUT, f"linear_{name}.npz"), x=x, dy=dy, dx0=dx0,
                            codes=codes, scale=scale, y=y, dx=dx)
        print("linear", name)


# The reference's float LoRA sites (tests/host/adjoint_lora.cpp:60-67): name, M, K, N, R, S.
LORA_SITES = [("tiny_q_proj", 6, 128, 128, 16, 2), ("tiny_gate_proj", 5, 128, 256, 16, 1),
              ("tiny_down_proj", 4, 256, 128, 4, 1)]


def slots_of(M, S_):
    # row 1 a base row spelled -1, row 2 one spelled past the pool (adjoint_lora.cpp:70-74)
    return np.array([-1 if m == 1 else (S_ if m == 2 else m % S_) for m in range(M)], np.float64)


def lora_fixtures():
    rng = np.random.default_rng(11)
    for name, M, K, N, R, S_ in LORA_SITES:
        slot = slots_of(M, S_)
        x = bf16r(rng.standard_normal((M, K)))
        la = bf16r(0.05 * rng.standard_normal((S_, R, K)))
        lb = bf16r(0.05 * rng.standard_normal((S_, N, R)))
        sc = np.full((S_, N), 2.0) * (1.0 + 0.1 * rng.random((S_, N)))
        ct = rng.standard_normal((M, R))
        cy = bf16r(rng.standard_normal((M, N)))
        t = O.lora_shrink_twin(x, slot, la, use_ref=True)
        y = O.lora_expand_twin(t, slot, lb, sc, use_ref=True)
        y_mm = O.lora_expand_twin(t, slot, lb, sc, mm=True, use_ref=True)
        out = {}
        for fused in (0, 1):
            dx, da = O.lora_shrink_adjoint(x, slot, la, ct, fused=bool(fused), use_ref=True)
            dt, db = O.lora_expand_adjoint(t, slot, lb, sc, cy, fused=bool(fused), use_ref=True)
            out.update({f"dx_f{fused}": dx, f"da_f{fused}": da, f"dt_f{fused}": dt, f"db_f{fused}": db})
        np.savez_compressed(os.path.join(OUT, f"lora_{name}.npz"), x=x, slot=slot, la=la, lb=lb,
                            sc=sc, ct=ct, cy=cy, t=t, y=y, y_mm=y_mm, **out)
        print("lora", name)


# The coded trunk (i8a8h). gemm_nt_q over a stored weight at the reference test's shapes
# (tests/host/adjoint_linear.cpp:180-182: M, N, K) and the coded LoRA sites
# (tests/host/adjoint_lora.cpp:66-68: name, M, K, N, R, S, group), with the test's value rules:
# integer codes in [-60, 60], one positive f32 scale a (row, group).
LINEAR_Q_SITES = [("q_small", 4, 256, 128, 601), ("q_one", 1, 128, 256, 602), ("q_odd", 7, 320, 384, 603)]
LORA_Q_SITES = [("coded_q_proj", 3, 128, 4, 2, 128), ("coded_down_proj", 4, 256, 4, 1, 128),
                ("coded_up_proj", 5, 300, 4, 2, 128)]


def codes_and_scales(rng, M, K, groups):
    a = np.rint(rng.uniform(-1.0, 1.0, (M, K)) * 60.0)
    i = np.arange(M * groups).reshape(M, groups)
    a_scale = (0.02 + 0.01 * (i % 7) + 0.004 * np.abs(rng.uniform(-1.0, 1.0, (M, groups)))).astype(np.float32)
    return a, a_scale.astype(np.float64)


def linear_q_fixtures():
    rng = np.random.default_rng(17)
    for name, M, N, K, seed in LINEAR_Q_SITES:
        factor = (0.75 + 0.5 * rng.random(K // 128)).astype(np.float32)
        codes, scale = stored_weight(N, K, seed=seed, scale_col=factor)
        a, a_scale = codes_and_scales(rng, M, K, K // 128)
        dy = rng.standard_normal((M, N))
        da0 = rng.standard_normal((M, K))
        y = O.gemm_nt_q_twin(a, a_scale, codes, scale, use_ref=True)
        da = O.gemm_nt_q_adjoint(dy, codes, scale, a_scale, da=da0, use_ref=True)
        np.savez_compressed(os.path.join(OUT, f"linear_{name}.npz"), a=a, a_scale=a_scale, dy=dy, da0=da0,
                            codes=codes, scale=scale, y=y, da=da)
        print("linear", name)


def lora_q_fixtures():
    rng = np.random.default_rng(19)
    for name, M, K, R, S_, group in LORA_Q_SITES:
        groups = (K + group - 1) // group
        slot = slots_of(M, S_)
        a, a_scale = codes_and_scales(rng, M, K, groups)
        la = bf16r(rng.uniform(-1.0, 1.0, (S_, R, K)))
        ct = rng.standard_normal((M, R))
        t = O.lora_shrink_q_twin(a, a_scale, slot, la, use_ref=True)
        out = {}
        for fused in (0, 1):
            da, ds, dA = O.lora_shrink_q_adjoint(a, a_scale, slot, la, ct, fused=bool(fused), use_ref=True)
            out.update({f"da_f{fused}": da, f"ds_f{fused}": ds, f"dA_f{fused}": dA})
        np.savez_compressed(os.path.join(OUT, f"lora_{name}.npz"), a=a, a_scale=a_scale, slot=slot, la=la,
                            ct=ct, t=t, **out)
        print("lora", name)


# AdamW (src/optim.cpp): the reference's Optimiser over LoRA-shaped parameters (an A [16, 256], a
# B [384, 16] and a short vector excluded from weight decay; 10501 elements, so the clip's 4096-element
# chunks span parameters), six gradient sets, under three configurations: the defaults; warm-up +
# cosine with weight decay and a clip that bites; and accumulation over two calls with a clip that
# does not.
ADAMW_CONFIGS = {
    "plain": dict(),
    "schedule_clip_decay": dict(lr=1e-2, warmup_steps=2, total_steps=5, lr_floor_frac=0.1, weight_decay=0.05,
                                clip_norm=1.0),
    "accumulate": dict(lr=3e-3, accum_steps=2, clip_norm=1e3),
}


def adamw_fixture():
    rng = np.random.default_rng(23)
    params = [(0.05 * rng.standard_normal((16, 256))).astype(np.float32),
              (0.05 * rng.standard_normal((384, 16))).astype(np.float32),
              rng.standard_normal(5).astype(np.float32)]
    decay = [1, 1, 0]
    grads = [[(0.1 * rng.standard_normal(p.shape)).astype(np.float32) for p in params] for _ in range(6)]
    out = {f"w{i}": p for i, p in enumerate(params)}
    for s_ in range(6):
        for i in range(3):
            out[f"g{s_}_{i}"] = grads[s_][i]
    for name, kw in ADAMW_CONFIGS.items():
        cfg = O.AdamWConfig.make(**kw)
        w, m, v, acc, (upd, pend) = O.adamw_run_ref(cfg, params, grads, decay=decay)
        for i in range(3):
            out[f"{name}_w{i}"], out[f"{name}_m{i}"], out[f"{name}_v{i}"], out[f"{name}_acc{i}"] = w[i], m[i], v[i], acc[i]
        out[f"{name}_updates"], out[f"{name}_pending"] = upd, pend
    np.savez_compressed(os.path.join(OUT, "adamw_runs.npz"), decay=np.array(decay), **out)
    print("adamw")


def c1_fixture():
    """Config 1 composed from the reference rows: W 1024x1024 from
    N(0, 0.02) through this repo's quantizer is not available to the reference, so the stored
    weight here is a trunk-form plane decoded by the reference; X, dY fp32 N(0,1) rounded to bf16
    on both sides; r 8, alpha 16; A, B ~ N(0, 0.01). Full outputs are pinned by digest, with the
    first rows and dA / dB stored."""
    rng = np.random.default_rng(1001)
    T, N, K, R = 128, 1024, 1024, 8
    s = 16.0 / R
    factor = (0.75 + 0.5 * rng.random(K // 128)).astype(np.float32)
    codes, scale = stored_weight(N, K, seed=1001, scale_col=factor)
    x = bf16r(rng.standard_normal((T, K)))
    dy = bf16r(rng.standard_normal((T, N)))
    A = bf16r(0.01 * rng.standard_normal((R, K)))
    B = bf16r(0.01 * rng.standard_normal((N, R)))
    slot = np.zeros(T)
    sc = np.full((1, N), s)
    y = O.gemm_nt_twin(x, codes, scale, use_ref=True)
    t = O.lora_shrink_twin(x, slot, A.reshape(1, R, K), use_ref=True)
    y = y + O.lora_expand_twin(t, slot, B.reshape(1, N, R), sc, use_ref=True)
    dt, dB = O.lora_expand_adjoint(t, slot, B.reshape(1, N, R), sc, dy, use_ref=True)
    dx, dA = O.lora_shrink_adjoint(x, slot, A.reshape(1, R, K), dt, use_ref=True)
    dx = O.gemm_nt_adjoint(dy, codes, scale, dx=dx, use_ref=True)
    np.savez_compressed(os.path.join(OUT, "c1_reference.npz"), seed=1001, T=T, N=N, K=K, R=R, s=s,
                        factor=factor, y_sha=digest(y), dx_sha=digest(dx), t=t, dA=dA, dB=dB,
                        y_rows=y[[0, 1, 63, 127]], dx_rows=dx[[0, 1, 63, 127]],
                        codes_sha=digest(codes), scale_sha=digest(scale))
    print("c1 reference")


PART_CASES = [
    # name, part, rows, n, eps, wadd, mult (the fused producers' parts; wadd 1 is Qwen3.5's w + 1 norm)
    ("rmsnorm_wadd1", "rmsnorm", 6, 256, 1e-6, 1.0, 1.0),
    ("rmsnorm_scaled", "rmsnorm", 3, 160, 1e-5, 0.5, 1.25),
    ("silu_mul", "silu_mul", 5, 192, 0.0, 0.0, 1.0),
    ("sigmoid_mul", "sigmoid_mul", 7, 128, 0.0, 0.0, 1.0),
]


def part_fixtures():
    """The elementwise parts of the fused quantiser producers: the reference's rmsnorm, silu_mul and
    act_mul (act = sigmoid) twins and host adjoints (src/adjoint/host/elementwise.cpp:278-347,
    459-641) on seeded bf16 inputs and an f32 cotangent."""
    for name, part, rows, n, eps, wadd, mult in PART_CASES:
        rng = np.random.default_rng(len(name) * 7919 + rows)
        w0 = 2 * n if part == "silu_mul" else n
        x0 = bf16r(rng.standard_normal((rows, w0)) * 1.5)
        x1 = {"rmsnorm": bf16r(rng.standard_normal(n) * 0.3), "silu_mul": None,
              "sigmoid_mul": bf16r(rng.standard_normal((rows, n)))}[part]
        dy = rng.standard_normal((rows, n)).astype(np.float32).astype(np.float64)
        y = O.part_twin(part, x0, x1, eps, wadd, mult, use_ref=True)
        dx0, dx1 = O.part_adjoint(part, x0, x1, dy, eps, wadd, mult, use_ref=True)
        d = dict(part=part, eps=eps, wadd=wadd, mult=mult, x0=x0, dy=dy, y=y, dx0=dx0)
        if x1 is not None:
            d["x1"] = x1
        if dx1 is not None:
            d["dx1"] = dx1
        np.savez_compressed(os.path.join(OUT, f"part_{name}.npz"), **d)


if __name__ == "__main__":
    if O.ref() is None:
        sys.exit("oracle/_ref/libr97ref.so is not built (make -C oracle, needs /root/reference)")
    decode_fixtures()
    linear_fixtures()
    lora_fixtures()
    linear_q_fixtures()
    lora_q_fixtures()
    adamw_fixture()
    part_fixtures()
    c1_fixture()
