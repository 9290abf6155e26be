#!/usr/bin/env python3
"""bench.py -- the fused IQR-linear + LoRA forward+backward on one MI355X.

One step = one forward and one backward of the adapted linear on one batch of synthetic input:
  forward   t = X.A^T, Y = X.W^T + s.t.B^T                 (r97q_lora_fwd_prep, r97q_qlinear_fwd_base)
  backward  dt = s.dY.B, dA += dt^T.X, dB += s.dY^T.t,
            dX = dY.W + dt.A                               (r97q_qlinear_lora_bwd: the down product, the
                                                            factor gradients' chunk sums, the dX product
                                                            that then adds those sums in)
W is an IQR trunk-form weight (b5 trellis.mad, L 16, 256-row runs, f32 row scale + scale.col)
quantized from W ~ N(0, 0.02) by this repo's quantizer; X, dY bf16 N(0,1); A, B bf16 N(0, 0.01).
Default workload: C2, 4096 x 4096, T 4096, rank 16, alpha 32.

Prints ONE JSON line (rank 0): the step's whole-job TFLOP/s over the timed steps (nothing else on
the stream between them), the dominant kernel's roofline (HIP events around the base products'
launches -- the forward's in a second run of as many steps, the dX product's in as many backwards
through the stand-alone stages, where its launch holds the product alone: a timing event between
two kernels costs several microseconds of GPU time, so the events stay out of the steps `value` is
timed on), its HBM
traffic per launch from the
committed FETCH_SIZE / WRITE_SIZE profile of the same sources (null when the sources changed since)
and a CPU baseline (the reference's own host rows, oracle/_ref, on the box's host cores, over a
bounded row sample).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
PEAK_INT8_TOPS = 5000.0     # MI355X dense int8 MFMA

CONFIGS = {
    # name: (T, N, K, rank, alpha)
    "c1": (128, 1024, 1024, 8, 16.0),
    "c2": (4096, 4096, 4096, 16, 32.0),
}


DECODE_MODES = {"auto": 0, "once": 1, "fused": 2}  # R97Q_DECODE_AUTO / _ONCE / _FUSED (include/r97q.h)
# the library's automatic choice (csrc/qlinear.hip, decode_once): the weight decoded once from
# 16384 tokens on, and from 8192 for weights of 2^23 values or more
DECODE_ONCE_MIN_T, DECODE_ONCE_MIN_T_LARGE, DECODE_ONCE_LARGE = 16384, 8192, 1 << 23


def mfma_ceiling(L, torch, iters=24000, reps=3):
    """The card's sustained bf16 MFMA rate with nothing else to do (r97q_mfma_probe): median of
    `reps` launches of about 40 ms each, random operands and zero operands, in TFLOP/s."""
    from r9700training_amd import _ptr, _stream, check

    out = torch.empty(256 * 512, dtype=torch.float32, device="cuda")
    st = _stream(torch.cuda.current_stream())
    res = {}
    for zero in (0, 1):
        rates = []
        for _ in range(reps + 1):  # the first launch ramps the clock
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            check(L.r97q_mfma_probe(iters, zero, _ptr(out), out.numel(), st), "r97q_mfma_probe")
            b.record()
            b.synchronize()
            rates.append(L.r97q_mfma_probe_flops(iters) / (a.elapsed_time(b) * 1e-3) / 1e12)
        res["zero_operands" if zero else "random_operands"] = round(sorted(rates[1:])[len(rates[1:]) // 2], 1)
    return res


def decode_label(once):
    """once / fused / mixed over the projections of a workload"""
    return "once" if all(once) else "fused" if not any(once) else "mixed"


def decodes_once(mode, T, N, K):
    return mode == "once" or (mode == "auto" and (T >= DECODE_ONCE_MIN_T or
                                                  (T >= DECODE_ONCE_MIN_T_LARGE and N * K >= DECODE_ONCE_LARGE)))


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--out-dtype", default="f32", choices=["f32", "bf16"],
                    help="Y and dX dtype (f32: the parity contract's single rounding)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="target CPU work for the cpu_baseline sample (0 = skip)")
    ap.add_argument("--seed", type=int, default=2001)
    ap.add_argument("--weight-form", default="trellis", choices=["trellis", "codes8"],
                    help="the prepared weight the kernels read: the trellis stream (decoded inside the "
                         "kernels), or the same weight in the int8-code form")
    ap.add_argument("--workload", default="qlinear",
                    choices=["qlinear", "vocab_head", "c3_block", "c4_attn", "c5_stack", "coded_fwd", "ref_shapes",
                             "fused_quant"],
                    help="qlinear: the C2 fwd+bwd step (the headline); vocab_head: the vocabulary head's "
                         "transposed product at a 248320-row head, n_embd 2048, --vocab-rows token rows; "
                         "c3_block / c4_attn / c5_stack: one whole LoRA step of BASELINE's MLP block (T=8192, "
                         "rank 32), attention projections (T=16384, rank 64) or 24-layer stack (T=32768, rank 16 "
                         "on every projection); "
                         "coded_fwd: gemm_nt_q's twin (int8 codes x the int8-code weight) at C2's square layer; "
                         "ref_shapes: the stored-weight gemm_nt twin and adjoint alone at the shapes the reference "
                         "publishes its device adjoint at (docs/kernels/linear.md:261-268); "
                         "fused_quant: the fused quantiser producers' forward and adjoint at the live widths")
    ap.add_argument("--decode", default="auto", choices=sorted(DECODE_MODES),
                    help="how the base products meet the weight (r97q_set_decode_once): fused (each tile "
                         "decoded in the product's main loop, once a 512-token panel), once (the whole weight "
                         "decoded once a call into the workspace, then the product over the decoded tiles), "
                         "auto (the library's choice: once from 16384 tokens on, from 8192 for weights of "
                         "2^23 values or more)")
    ap.add_argument("--vocab-rows", type=int, default=4096)
    ap.add_argument("--settle-s", type=float, default=1.5,
                    help="untimed steps for this long before the warmup steps, so the GPU's clocks leave their "
                         "idle state before anything is timed (declared in the line as clock_settle)")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="run only a plain device copy of this many MiB (3 launches), the known-size "
                         "kernel that scales rocprofv3's FETCH_SIZE / WRITE_SIZE to bytes")
    return ap.parse_args()


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "qlinear_c2_traffic.json")


def profiled_traffic(kernel, config):
    """HBM bytes per launch of `kernel` from the committed counter profile, if it was taken on this
    config and on the kernel sources as they are now; else None."""
    import hashlib

    try:
        with open(TRAFFIC_PROFILE) as f:
            prof = json.load(f)
    except (OSError, ValueError):
        return None
    h = hashlib.sha256()
    for src in prof.get("sources", []):
        try:
            with open(os.path.join(ROOT, src), "rb") as f:
                h.update(f.read())
        except OSError:
            return None
    if config != "c2" or h.hexdigest()[:16] != prof.get("sources_sha256_16"):
        return None
    kernels = prof.get("kernels", {})
    # a kernel is looked up by the name the line gives it (qlinear_rt_kernel<dx>), or by its name
    # without template arguments
    k = kernels.get(kernel) or next((v for n, v in kernels.items() if n.split("<")[0] == kernel), None)
    return None if k is None else k["traffic_bytes"]


def flops(T, N, K, r):
    """Algorithmic FLOPs of one fwd+bwd (the base weight is frozen: no dW)."""
    return 4 * T * N * K + 6 * T * r * (K + N)


def make_inputs(T, N, K, r, seed, device, weight_form="trellis"):
    import numpy as np
    import torch

    from r9700training_amd.qlinear import QWeight, device_desc
    from r9700training_amd.quantize import quantize_trellis

    rng = np.random.default_rng(seed)
    W = (0.02 * rng.standard_normal((N, K))).astype(np.float32)
    q = quantize_trellis(W, bits=5, state_bits=16, run_rows=256)
    codes = torch.from_numpy(q["codes"]).to(device)
    scale = torch.from_numpy(q["row_scale"].view(np.uint8).reshape(N, 4).copy()).to(device)
    col = torch.from_numpy(q["col_factor"]).to(device)
    d = device_desc(dict(codes=codes, scale=scale), N, K, dict(
        bits=5, state_bits=16, run_rows=256, rb=1, mad=1, round_mad=1, mad_a=q["mad_a"], mad_b=q["mad_b"],
        codes_row_bytes=q["codes"].shape[1], scale_dtype=0, scale_block_cols=0, scale_row_bytes=4))
    w = QWeight(d, scale_col=col, codes8=weight_form == "codes8")
    g = torch.Generator(device="cpu").manual_seed(seed + 1)
    X = torch.randn((T, K), generator=g).to(torch.bfloat16).to(device)
    dY = torch.randn((T, N), generator=g).to(torch.bfloat16).to(device)
    A = (0.01 * torch.randn((r, K), generator=g)).to(torch.bfloat16).to(device)
    B = (0.01 * torch.randn((N, r), generator=g)).to(torch.bfloat16).to(device)
    return dict(w=w, q=q, X=X, dY=dY, A=A, B=B, keep=(codes, scale, col))


def host_cores():
    """The host cores this process may use: its CPU affinity, at most 16 (one GPU's share of a GPU
    box's cores)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def ref_decode(codes_p, rs, col_factor, N, K, mad_a, mad_b):
    """The stored weight the host rows read: the reference's r97_iqr_decode_host (oracle/_ref, else the
    oracle's restatement) over a b5 trellis.mad weight with an f32 row scale, then scale.col folded
    in. Returns (codes, scale, seconds)."""
    import numpy as np

    from oracle import oracle as O
    from oracle.oracle import Desc

    codes_p = np.ascontiguousarray(codes_p)
    rs = np.ascontiguousarray(rs, dtype=np.float32)
    d = Desc()
    d.rows_all, d.cols, d.row0, d.rows = N, K, 0, N
    d.bits, d.state_bits, d.run_rows, d.rb, d.mad, d.round_mad = 5, 16, 256, 1, 1, 1
    d.mad_a, d.mad_b = mad_a, mad_b
    d.codes, d.codes_row_bytes = codes_p.ctypes.data, codes_p.shape[1]
    d.scale, d.scale_dtype, d.scale_block_cols, d.scale_row_bytes = rs.ctypes.data, 0, 0, 4
    t0 = time.perf_counter()
    codes, _ = O.decode(d, use_ref=O.ref() is not None)
    scale = O.fold_scale_col(rs, np.asarray(col_factor, np.float32))
    return codes, scale, time.perf_counter() - t0


def settle(step, seconds, torch, chunk=20):
    """Run `step` (untimed) for about `seconds`, synchronising every `chunk` steps: the GPU's clocks
    ramp from idle over the first few hundred milliseconds of work. Returns the line's clock_settle."""
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(chunk):
            step()
        n += chunk
        torch.cuda.synchronize()
    return {"s": round(time.perf_counter() - t0, 3), "steps": n,
            "what": "untimed steps run before the warmup steps, so the clocks leave their idle state first"}


def cpu_baseline(projs, T, r, s, target_s, nthreads, layers=1, reps=3, what="", unit="TFLOP/s"):
    """The reference's own host path (oracle/_ref: its r97_iqr_decode_host, gemm_nt twin and adjoint,
    float lora_shrink / lora_expand twins and adjoints, f64 with its parallel_for) on `nthreads`
    threads, over an evenly spaced sample of token rows of every projection in `projs`, timed `reps`
    times (the median taken) and extrapolated linearly in tokens (and in layers) to the whole step.
    Each projection is a dict: N, K, codes / scale (the decoded stored weight), decode_s, A [r, K],
    B [N, r] (f64), rows(idx) -> (x [m, K], dy [m, N]) f64."""
    import numpy as np

    from oracle import oracle as O

    use_ref = O.ref() is not None
    os.environ["R97_THREADS"] = str(nthreads)
    O.set_threads(nthreads)

    def path(rows):
        for pj in projs:
            N, K = pj["N"], pj["K"]
            x, dy = pj["rows"](rows)
            M = len(rows)
            slot = np.zeros(M)
            sc = np.full((1, N), s)
            codes, scale, A, B = pj["codes"], pj["scale"], pj["A"], pj["B"]
            O.gemm_nt_twin(x, codes, scale, use_ref=use_ref)
            t = O.lora_shrink_twin(x, slot, A.reshape(1, r, K), use_ref=use_ref)
            O.lora_expand_twin(t, slot, B.reshape(1, N, r), sc, use_ref=use_ref)
            dt, _ = O.lora_expand_adjoint(t, slot, B.reshape(1, N, r), sc, dy, use_ref=use_ref)
            O.lora_shrink_adjoint(x, slot, A.reshape(1, r, K), dt, use_ref=use_ref)
            O.gemm_nt_adjoint(dy, codes, scale, use_ref=use_ref)

    probe = np.arange(min(T, 2 * nthreads))
    t0 = time.perf_counter()
    path(probe)
    per_row = (time.perf_counter() - t0) / len(probe)
    n = int(max(len(probe), min(T, target_s / reps / max(per_row, 1e-9))))
    n = max(2 * nthreads, (n // (2 * nthreads)) * (2 * nthreads))
    rows = np.linspace(0, T - 1, n).astype(np.int64)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        path(rows)
        times.append(time.perf_counter() - t0)
    t_rows = sorted(times)[len(times) // 2]
    decode_s = sum(pj["decode_s"] for pj in projs)
    step_s = (decode_s + t_rows * (T / n)) * layers
    total = layers * sum(flops(T, pj["N"], pj["K"], r) for pj in projs)
    return {
        "value": round(total / step_s / 1e12, 6) if unit == "TFLOP/s" else round(T / step_s, 3),
        "unit": unit,
        "tflops": round(total / step_s / 1e12, 6),
        "s_per_step": round(step_s, 2),
        "cores": nthreads,
        "kind": "reference" if use_ref else "port",
        "sample": f"{n} of {T} token rows (evenly spaced) of {len(projs)} projection(s){what} through decode + "
                  f"gemm_nt twin/adjoint + lora shrink/expand twins/adjoints, f64, {nthreads} threads; the "
                  f"median of {reps} passes ({', '.join(f'{x:.1f}' for x in times)} s) extrapolated linearly "
                  f"in tokens" + (f" and in layers (x{layers})" if layers > 1 else "") +
                  f" ({decode_s:.2f} s decode; {step_s:.1f} s per full step; nproc {os.cpu_count()}, "
                  f"affinity {host_cores()})",
    }


def c2_projection(inp, T, N, K, r):
    """The C2 layer as cpu_baseline's projection: the decoded stored weight and the step's inputs."""
    import numpy as np

    q = inp["q"]
    codes, scale, dec_s = ref_decode(q["codes"], q["row_scale"], q["col_factor"], N, K, q["mad_a"], q["mad_b"])
    X = inp["X"].float().cpu().numpy().astype(np.float64)
    dY = inp["dY"].float().cpu().numpy().astype(np.float64)
    return dict(N=N, K=K, codes=codes, scale=scale, decode_s=dec_s,
                A=inp["A"].float().cpu().numpy().astype(np.float64),
                B=inp["B"].float().cpu().numpy().astype(np.float64),
                rows=lambda idx: (X[idx], dY[idx]))


VOCAB_CLASSES = [32768, 65536, 98304, 51712]  # rows a class (one trellis width each): 248320 in all
VOCAB_EMBD = 2048


def rows_cpu_baseline(fn, rows, target_s, nthreads, ops, unit, fixed_s=0.0, what="", reps=3, div=1e12,
                      kind=None):
    """A host path timed over token rows: `fn(idx)` runs it over the rows idx (numpy int64), first on a
    probe to price a row, then on an evenly spaced sample sized for about target_s over `reps` passes
    (the median taken), extrapolated linearly to all `rows`; `fixed_s` (a once-a-call cost, the
    weight's decode) added. ops: the whole call's operations (or bytes), for `value` = ops / seconds /
    div in `unit`. The host path is the reference's own code from oracle/_ref when built
    ("reference"), else the oracle's restatement ("port"); `kind` overrides."""
    import numpy as np

    from oracle import oracle as O

    os.environ["R97_THREADS"] = str(nthreads)
    O.set_threads(nthreads)
    probe = np.arange(min(rows, 2 * nthreads))
    t0 = time.perf_counter()
    fn(probe)
    per_row = (time.perf_counter() - t0) / len(probe)
    n = int(max(len(probe), min(rows, target_s / reps / max(per_row, 1e-9))))
    n = max(len(probe), n // len(probe) * len(probe))
    idx = np.linspace(0, rows - 1, n).astype(np.int64)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn(idx)
        times.append(time.perf_counter() - t0)
    t_rows = sorted(times)[len(times) // 2]
    call_s = fixed_s + t_rows * rows / n
    return {
        "value": round(ops / call_s / div, 6), "unit": unit, "s_per_call": round(call_s, 4), "cores": nthreads,
        "kind": kind or ("reference" if O.ref() is not None else "port"),
        "sample": f"{n} of {rows} token rows (evenly spaced){what}, f64, {nthreads} threads; the median of "
                  f"{reps} passes ({', '.join(f'{x:.2f}' for x in times)} s) extrapolated linearly in rows"
                  + (f", plus the weight's decode once ({fixed_s:.2f} s)" if fixed_s else ""),
    }


def vocab_cpu_baseline(src, dy, K, target_s, nthreads, reps=3):
    """The host restatement of the reference's vocabulary-head kernels (oracle: orc_vocab_class_product
    and orc_fwht128, f64, following src/adjoint/device/vocab_head.hip:88-163) over an evenly spaced
    sample of token rows, split over `nthreads` threads, plus every class's decode (the reference's
    r97_iqr_decode_host from oracle/_ref when built, else the oracle's), as the reference decodes
    each call; the rows timed `reps` times (the median) and extrapolated linearly to all rows.
    src: (packed codes, f32 row scale, scale.col, ids, rows) a class, on the card; dy: bf16 on the
    card."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    import torch

    from oracle import oracle as O

    O.set_threads(nthreads)
    decode_s, classes = 0.0, []
    for codes_d, scale_d, cf_d, ids_d, n in src:
        codes, scale, s = ref_decode(codes_d.cpu().numpy(), scale_d.cpu().numpy().view(np.float32),
                                     np.ones(K // 128, np.float32), n, K, 0x2F1E3D | 1, 0x9E3779B9)
        decode_s += s
        classes.append((codes, scale, ids_d.cpu().numpy(), cf_d.cpu().numpy()))
    rows = dy.shape[0]

    def bits(idx):
        it = torch.from_numpy(np.asarray(idx, np.int64)).to(dy.device)
        return dy.index_select(0, it).view(torch.int16).cpu().numpy().view(np.uint16)

    def run(b):  # the sample's rows, a block a thread (the C calls release the GIL)
        parts = np.array_split(np.arange(b.shape[0]), nthreads)
        with ThreadPoolExecutor(nthreads) as ex:
            list(ex.map(lambda p: O.vocab_head_transpose(b[p], classes, transform=128), [p for p in parts if len(p)]))

    probe = bits(np.arange(min(rows, nthreads)))
    t0 = time.perf_counter()
    run(probe)
    per_pass_row = (time.perf_counter() - t0) / probe.shape[0]  # per row, all threads busy
    n = int(max(nthreads, min(rows, target_s / reps / max(per_pass_row, 1e-9))))
    n = max(nthreads, n // nthreads * nthreads)
    sample = bits(np.linspace(0, rows - 1, n).astype(np.int64))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run(sample)
        times.append(time.perf_counter() - t0)
    t_rows = sorted(times)[len(times) // 2]
    call_s = decode_s + t_rows * rows / n
    vocab = sum(c[0].shape[0] for c in classes)
    return {
        "value": round(2.0 * rows * vocab * K / call_s / 1e12, 6), "unit": "TFLOP/s",
        "s_per_call": round(call_s, 1), "cores": nthreads, "kind": "port",
        "sample": f"{n} of {rows} token rows (evenly spaced) through the classes' products and the transform "
                  f"(f64, {nthreads} threads, a block of rows each), the median of {reps} passes "
                  f"({', '.join(f'{x:.1f}' for x in times)} s) extrapolated linearly in rows, plus the "
                  f"classes' decode once ({decode_s:.2f} s, {'the reference' if O.ref() is not None else 'the oracle'}"
                  f"'s host decode)",
    }


def vocab_head_bench(args):
    """The vocabulary head's transposed product (r97q_vocab_head_transpose) on a synthetic head the
    size of the reference container's (four b5 trellis.mad classes, f32 row scale + scale.col, the
    fwht128 transform), d_x += H . sum_c (dy[:, ids_c] . W_c) * scale.col_c over --vocab-rows rows.
    Each call decodes the classes into its workspace, as the reference's does."""
    import numpy as np
    import torch

    from r9700training_amd.qlinear import device_desc
    from r9700training_amd.vocab_head import VocabHead

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    rows, K = args.vocab_rows, VOCAB_EMBD
    vocab = sum(VOCAB_CLASSES)
    g = torch.Generator(device="cuda").manual_seed(args.seed)
    perm = torch.randperm(vocab, device="cuda", generator=g).to(torch.int32)
    rng = np.random.default_rng(args.seed)
    classes, keep, src, at = [], [], [], 0
    for n in VOCAB_CLASSES:
        codes = torch.randint(0, 256, (n, K * 5 // 8), dtype=torch.uint8, device="cuda", generator=g)
        scale = torch.from_numpy((0.0005 + 0.01 * rng.random(n)).astype(np.float32).view(np.uint8)).to(dev)
        cf = torch.from_numpy((0.5 + rng.random(K // 128)).astype(np.float32)).to(dev)
        d = device_desc(dict(codes=codes, scale=scale), n, K, dict(
            bits=5, state_bits=16, run_rows=256, rb=1, mad=1, round_mad=1, mad_a=0x2F1E3D | 1, mad_b=0x9E3779B9,
            codes_row_bytes=K * 5 // 8, scale_dtype=0, scale_block_cols=0, scale_row_bytes=4))
        ids = perm[at:at + n].sort().values.contiguous()  # a class's ids ascend, as a partition of the vocabulary
        at += n
        classes.append((d, ids, cf))
        keep += [codes, scale, cf, ids]
        src.append((codes, scale, cf, ids, n))
    head = VocabHead(K, vocab, classes, transform=128)
    dy = torch.randn((rows, vocab), dtype=torch.bfloat16, device=dev, generator=g)
    d_x = torch.zeros((rows, K), device=dev)
    ws = torch.empty(head.workspace_bytes(rows), dtype=torch.uint8, device=dev)
    steps, warmup = max(1, min(args.steps, 20)), max(1, min(args.warmup, 5))
    for _ in range(warmup):
        head.transpose(dy, d_x, ws)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        head.transpose(dy, d_x, ws)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    flops = 2.0 * rows * vocab * K
    tf = flops / (ms * 1e-3) / 1e12
    cpu = vocab_cpu_baseline(src, dy, K, args.cpu_seconds, min(8, host_cores())) if args.cpu_seconds > 0 else None
    print(json.dumps({
        "metric": "vocab head transposed product TFLOP/s (decode + gather + MFMA + transform per call)",
        "value": round(tf, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_call": round(ms, 4), "higher_is_better": True, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"vocab head: {len(VOCAB_CLASSES)} b5 trellis.mad classes, {vocab} rows in all, "
                               f"n_embd {K}, fwht128, {rows} token rows", "classes": VOCAB_CLASSES,
                   "n_embd": K, "rows": rows},
        "roofline": {"bound": "mfma", "achieved": round(tf, 3), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf / PEAK_BF16_TFLOPS, 4), "traffic": None},
        **({"cpu_baseline": cpu} if cpu else {}),
    }), flush=True)


# C5: per layer (hidden 2048) attn-in 2048->8192, attn-out 4096->2048, gate/up 2048->6144, down
# 6144->2048; 24 layers; LoRA rank 16 alpha 32 on every projection; T = 32768 tokens
C5_PROJ = [(8192, 2048), (2048, 4096), (6144, 2048), (2048, 6144)]  # (N, K)
C5_LAYERS, C5_T, C5_R, C5_ALPHA = 24, 32768, 16, 32.0
# BASELINE's configs of several projections, each one whole LoRA step:
# name: (projections (N, K) of a layer, layers, T, rank, alpha, metric, description)
STACKS = {
    "c3_block": ([(12288, 4096), (12288, 4096), (4096, 12288)], 1, 8192, 32, 64.0,
                 "C3 LoRA-step tokens/s (one MLP block: gate, up, down; fwd + bwd + AdamW on the adapters)",
                 "C3: MLP block, hidden 4096, intermediate 12288: gate and up (4096->12288), down (12288->4096), "
                 "b5 trellis.mad, LoRA r32 alpha 64 on all three, T=8192, Y/dX f32 (the SiLU gate between "
                 "them is not this path)"),
    "c4_attn": ([(8192, 2048), (2048, 4096)], 1, 16384, 64, 128.0,
                "C4 LoRA-step tokens/s (attention projections: qkv+gate in, out; fwd + bwd + AdamW on the adapters)",
                "C4: attention projections, hidden 2048: qkv+gate 2048->8192, out 4096->2048, b5 trellis.mad, "
                "LoRA r64 alpha 128 on both, T=16384, Y/dX f32"),
    "c5_stack": (C5_PROJ, C5_LAYERS, C5_T, C5_R, C5_ALPHA,
                 "C5 LoRA-step tokens/s (24-layer stack, fwd + bwd + AdamW on the adapters)",
                 "C5: 24 layers x (2048->8192, 4096->2048, 2048->6144, 6144->2048) b5 trellis.mad, "
                 "LoRA r16 alpha 32 on every projection, T=32768, Y/dX f32"),
}


def coded_fwd_bench(args):
    """gemm_nt_q's twin (r97q_gemm_nt_q_fwd) at C2's square layer: int8 activation codes a [4096, 4096]
    with f32 scales per 128-column group, and a stored weight in the reference's two grids (int8
    codes [4096, 4096], bf16 scales [4096, 32]); Y f32. One step = one launch."""
    import torch

    from r9700training_amd import R97Q_F32, _ptr, _stream, check, lib

    dev = torch.device("cuda:0")
    T, N, K, _r, _alpha = CONFIGS["c2"]
    g = torch.Generator(device="cuda").manual_seed(args.seed)
    a = torch.randint(-127, 128, (T, K), dtype=torch.int8, device=dev, generator=g)
    a_scale = 0.01 + 0.05 * torch.rand((T, K // 128), device=dev, generator=g)
    codes = torch.randint(-126, 127, (N, K), dtype=torch.int8, device=dev, generator=g)
    scale = (0.0002 + 0.0004 * torch.rand((N, K // 128), device=dev, generator=g)).to(torch.bfloat16)
    Y = torch.empty((T, N), dtype=torch.float32, device=dev)
    L = lib()
    st = _stream(torch.cuda.current_stream())

    def step():
        check(L.r97q_gemm_nt_q_fwd(_ptr(codes), _ptr(scale), N, K, _ptr(a), _ptr(a_scale), T, _ptr(Y), R97Q_F32, st),
              "gemm_nt_q_fwd")

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ops = 2 * T * N * K
    tops = ops / (ms * 1e-3) / 1e12
    cpu = None
    if args.cpu_seconds > 0:
        import numpy as np

        from oracle import oracle as O

        a_h, as_h = a.cpu().numpy().astype(np.float64), a_scale.cpu().numpy().astype(np.float64)
        codes_h, scale_h = codes.cpu().numpy(), scale.view(torch.int16).cpu().numpy().view(np.uint16)
        cpu = rows_cpu_baseline(
            lambda idx: O.gemm_nt_q_twin(a_h[idx], as_h[idx], codes_h, scale_h, use_ref=O.ref() is not None),
            T, args.cpu_seconds, min(8, host_cores()), ops, "TOP/s", what=" through the gemm_nt_q twin")
    print(json.dumps({
        "metric": "coded forward (gemm_nt_q twin) TOP/s at C2's square layer",
        "value": round(tops, 3), "unit": "TOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "i8", "data": "synthetic: activation codes uniform in [-127, 127] with scales U(0.01, 0.06); "
                               "weight codes uniform in [-126, 126] with bf16 scales U(2e-4, 6e-4)",
        "config": {"workload": f"coded_fwd: Y = sum_g (a . codes^T)_g * a_scale * scale, T={T}, N={N}, K={K}, "
                               "group 128, Y f32", "T": T, "N": N, "K": K},
        "roofline": {"bound": "mfma", "kernel": "qlinear_q_kernel", "achieved": round(tops, 3),
                     "peak": PEAK_INT8_TOPS, "unit": "TOP/s", "frac": round(tops / PEAK_INT8_TOPS, 4), "traffic": None},
        **({"cpu_baseline": cpu} if cpu else {}),
    }), flush=True)


# The shapes the reference publishes its gemm_nt device adjoint at (docs/kernels/linear.md:261-268):
# name, tokens M, outputs N, inputs K (dX[M, K] = dY[M, N] . W[N, K]; the twin Y[M, N] = X . W^T), and
# the reference's R9700 kernel time for the adjoint in ms (context only: another card and kernel).
REF_SHAPES = [
    ("attn_k/v", 4096, 1024, 5120, 1.06),
    ("attn_output", 4096, 5120, 6144, 5.73),
    ("attn_qg", 1024, 12288, 5120, 3.39),
    ("attn_qg", 4096, 12288, 5120, 21.34),
    ("ssm_inz", 4096, 16384, 5120, 35.00),
    ("ffn_down", 4096, 5120, 17408, 18.47),
    ("ffn_gate_up", 1024, 34816, 5120, 11.38),
    ("ffn_gate_up", 4096, 34816, 5120, 53.91),
]


def ref_shapes_bench(args):
    """The stored-weight gemm_nt twin (Y = X . W^T) and adjoint (dX = dY . W) alone, no adapter, at
    the reference's published shapes: each product timed by HIP events around `steps` launches after
    a clock settle, over a b5 trellis.mad weight with an f32 row scale and scale.col (random packed
    codes; every byte pattern is a valid code), X and dY bf16 N(0,1), outputs f32."""
    import ctypes as C

    import numpy as np
    import torch

    from r9700training_amd import R97Q_F32, _ptr, _stream, check, lib
    from r9700training_amd.qlinear import QWeight, bwd_workspace, device_desc, fwd_workspace

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L = lib()
    L.r97q_set_decode_once(DECODE_MODES[args.decode])
    g = torch.Generator(device="cuda").manual_seed(args.seed)
    rng = np.random.default_rng(args.seed)
    st = _stream(torch.cuda.current_stream())
    P = _ptr
    out = []
    for name, M, N, K, ref_ms in REF_SHAPES:
        codes = torch.randint(0, 256, (N, K * 5 // 8), dtype=torch.uint8, device=dev, generator=g)
        scale = torch.from_numpy((0.0005 + 0.01 * rng.random(N)).astype(np.float32).view(np.uint8)).to(dev)
        cf = torch.from_numpy((0.5 + rng.random(K // 128)).astype(np.float32)).to(dev)
        d = device_desc(dict(codes=codes, scale=scale), N, K, dict(
            bits=5, state_bits=16, run_rows=256, rb=1, mad=1, round_mad=1, mad_a=0x2F1E3D | 1,
            mad_b=0x9E3779B9, codes_row_bytes=K * 5 // 8, scale_dtype=0, scale_block_cols=0, scale_row_bytes=4))
        w = QWeight(d, scale_col=cf)
        X = torch.randn((M, K), dtype=torch.bfloat16, device=dev, generator=g)
        dY = torch.randn((M, N), dtype=torch.bfloat16, device=dev, generator=g)
        Y = torch.empty((M, N), dtype=torch.float32, device=dev)
        dX = torch.empty((M, K), dtype=torch.float32, device=dev)
        wsf, wsb = fwd_workspace(M, N, K, 0, dev), bwd_workspace(M, N, K, 0, dev)
        check(L.r97q_lora_fwd_prep(M, N, K, P(X), None, 0, 1.0, None, P(wsf), wsf.numel(), st), "fwd_prep")
        check(L.r97q_lora_bwd_prep(M, N, K, P(dY), None, None, None, 0, 1.0, P(wsb), wsb.numel(), st), "bwd_prep")

        def fwd():
            check(L.r97q_qlinear_fwd_base(C.byref(w.w), P(X), M, None, 0, P(Y), R97Q_F32, P(wsf), wsf.numel(), st),
                  "fwd_base")

        def dx():
            check(L.r97q_qlinear_dx_base(C.byref(w.w), P(dY), M, 0, P(dX), R97Q_F32, 0, P(wsb), wsb.numel(), st),
                  "dx_base")

        res = {"shape": f"{name} {M} x {N} x {K}", "M": M, "N": N, "K": K}
        for tag, f, out_cols in (("twin", fwd, N), ("adjoint", dx, K)):
            settle(f, 0.3, torch)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(args.steps):
                f()
            e1.record()
            e1.synchronize()
            ms = e0.elapsed_time(e1) / args.steps
            tf = 2 * M * N * K / (ms * 1e-3) / 1e12
            tiles = ((M + 511) // 512) * (out_cols // 128)
            res[tag] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1), "frac": round(tf / PEAK_BF16_TFLOPS, 4),
                        "tiles_512x128": tiles}
        res["reference_r9700_adjoint_kernel_ms"] = ref_ms
        if args.cpu_seconds > 0:
            from oracle import oracle as O

            wc, ws_, dec_s = ref_decode(codes.cpu().numpy(), scale.cpu().numpy().view(np.float32), cf.cpu().numpy(),
                                        N, K, 0x2F1E3D | 1, 0x9E3779B9)
            use_ref = O.ref() is not None
            x_h, dy_h = X.float().cpu().numpy().astype(np.float64), dY.float().cpu().numpy().astype(np.float64)

            def host(idx):
                O.gemm_nt_twin(x_h[idx], wc, ws_, use_ref=use_ref)
                O.gemm_nt_adjoint(dy_h[idx], wc, ws_, use_ref=use_ref)

            res["cpu_baseline"] = rows_cpu_baseline(host, M, args.cpu_seconds / len(REF_SHAPES), min(8, host_cores()),
                                                    4 * M * N * K, "TFLOP/s", fixed_s=dec_s,
                                                    what=" through the gemm_nt twin and adjoint", reps=1)
            del x_h, dy_h, wc, ws_
        out.append(res)
        print(json.dumps(res), file=sys.stderr, flush=True)
        del w, codes, scale, cf, X, dY, Y, dX, wsf, wsb
        torch.cuda.empty_cache()
    print(json.dumps({
        "metric": "stored-weight gemm_nt twin / adjoint TFLOP/s at the reference's published shapes",
        "value": round(sum(2 * r["M"] * r["N"] * r["K"] * 2 for r in out) /
                       sum((r["twin"]["ms"] + r["adjoint"]["ms"]) * 1e-3 for r in out) / 1e12, 3),
        "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "higher_is_better": True, "dtype": "bf16",
        "data": "synthetic: random b5 trellis.mad codes, f32 row scale + scale.col; X, dY ~ N(0,1) bf16",
        "config": {"workload": "ref_shapes: docs/kernels/linear.md:261-268, M x N x K, no adapter, outputs f32",
                   "decode": args.decode},
        "shapes": out,
        **({"cpu_baseline": {
            "value": round(sum(4 * r["M"] * r["N"] * r["K"] for r in out) /
                           sum(r["cpu_baseline"]["s_per_call"] for r in out) / 1e12, 6),
            "unit": "TFLOP/s", "cores": out[0]["cpu_baseline"]["cores"], "kind": out[0]["cpu_baseline"]["kind"],
            "sample": "each shape's twin and adjoint on the host over a sample of its token rows, one pass a "
                      "shape, extrapolated in rows, plus its weight's decode (the shapes' own lines hold each); "
                      "the shapes' operations over their summed host seconds"}}
           if out and "cpu_baseline" in out[0] else {}),
    }), flush=True)


# The fused quantiser producers at the live tape's widths (tests/gpu/adjoint_quant.cpp:61-67 and the
# projections around them): name, part, rows, n (the part's output width), group.
FUSED_SHAPES = [
    ("rmsnorm_had_quant_i8g", "rmsnorm", 4096, 5120, 128),
    ("gated_had_quant_i8g", "silu_mul", 4096, 17408, 128),
    ("gate_had_quant_i8g", "sigmoid_mul", 4096, 6144, 128),
]


def fused_quant_bytes(part, rows, n, group, bwd):
    """The algorithmic HBM bytes of one launch: every input, output and cotangent once (bf16
    inputs, int8 codes, f32 scales, a bf16 output beside the codes, f32 cotangents, f32 dx read and
    written)."""
    total = rows * n
    in0 = 2 * total if part == "silu_mul" else total
    in1 = n if part == "rmsnorm" else total if part == "sigmoid_mul" else 0
    scale = 4 * total // group
    if not bwd:
        return 2 * (in0 + in1) + total + scale + 2 * total
    dx = 8 * in0 + (8 * total if part == "sigmoid_mul" else 0)
    return 2 * (in0 + in1) + scale + 4 * total + 4 * total + dx


def fused_quant_bench(args):
    """rmsnorm_had_quant_i8g, gated_had_quant_i8g and gate_had_quant_i8g (r97q_fused_had_quant_i8g and
    its adjoint) at the live widths: each launch timed by HIP events around `steps` launches after a
    clock settle, bf16 inputs N(0,1), the part's output written beside the codes, the adjoint with
    the output's cotangent. Achieved = algorithmic bytes / launch time against HBM's 8 TB/s."""
    import torch

    from r9700training_amd.quant import fused_had_quant_i8g, fused_had_quant_i8g_bwd

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator(device="cuda").manual_seed(args.seed)
    out = []
    for name, part, rows, n, group in FUSED_SHAPES:
        w0 = 2 * n if part == "silu_mul" else n
        x0 = torch.randn((rows, w0), dtype=torch.bfloat16, device=dev, generator=g)
        x1 = (torch.randn(n, dtype=torch.bfloat16, device=dev, generator=g) * 0.3 if part == "rmsnorm" else
              torch.randn((rows, n), dtype=torch.bfloat16, device=dev, generator=g) if part == "sigmoid_mul" else None)
        kw = dict(eps=1e-6, wadd=1.0) if part == "rmsnorm" else {}
        codes, scale, y = fused_had_quant_i8g(part, x0, x1, group, want_y=True, **kw)
        gc = torch.randn((rows, n), dtype=torch.float32, device=dev, generator=g)
        go = torch.randn((rows, n), dtype=torch.float32, device=dev, generator=g)
        dx0 = torch.zeros((rows, w0), dtype=torch.float32, device=dev)
        dx1 = torch.zeros((rows, n), dtype=torch.float32, device=dev) if part == "sigmoid_mul" else None
        res = {"op": name, "rows": rows, "n": n, "group": group}
        for tag, f, bwd in (("forward", lambda: fused_had_quant_i8g(part, x0, x1, group, want_y=True, **kw), False),
                            ("adjoint", lambda: fused_had_quant_i8g_bwd(part, x0, x1, group, scale, gc, go, dx0=dx0,
                                                                        dx1=dx1, **kw), True)):
            settle(f, 0.3, torch)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(args.steps):
                f()
            e1.record()
            e1.synchronize()
            ms = e0.elapsed_time(e1) / args.steps
            gbs = fused_quant_bytes(part, rows, n, group, bwd) / (ms * 1e-3) / 1e9
            res[tag] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4),
                        "bytes": fused_quant_bytes(part, rows, n, group, bwd)}
        if args.cpu_seconds > 0:
            import numpy as np

            from oracle import oracle as O

            f64 = lambda t: None if t is None else t.float().cpu().numpy().astype(np.float64)
            x0_h, x1_h, gc_h, go_h = f64(x0), f64(x1), f64(gc), f64(go)

            def host(idx):  # the oracle's producer and adjoint (single-threaded C) over the rows idx
                x1_r = x1_h if part == "rmsnorm" else None if x1_h is None else x1_h[idx]
                _, _, sc = O.fused_quant(part, x0_h[idx], x1_r, group, **kw)
                O.fused_quant_adjoint(part, x0_h[idx], x1_r, group, sc, gc_h[idx], go_h[idx], **kw)

            res["cpu_baseline"] = rows_cpu_baseline(
                host, rows, args.cpu_seconds / len(FUSED_SHAPES), 1, res["forward"]["bytes"] + res["adjoint"]["bytes"],
                "GB/s", what=" through the producer and its adjoint", reps=1, div=1e9, kind="port")
        out.append(res)
        print(json.dumps(res), file=sys.stderr, flush=True)
        del x0, x1, codes, scale, y, gc, go, dx0, dx1
        torch.cuda.empty_cache()
    total_bytes = sum(r[t]["bytes"] for r in out for t in ("forward", "adjoint"))
    total_s = sum(r[t]["us"] * 1e-6 for r in out for t in ("forward", "adjoint"))
    gbs = total_bytes / total_s / 1e9
    print(json.dumps({
        "metric": "fused quantiser producers (forward + adjoint) GB/s at the live widths",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(total_s * 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f64", "data": "synthetic: bf16 inputs N(0,1), gain N(0,0.09); f32 cotangents N(0,1)",
        "config": {"workload": "fused_quant: rmsnorm / gated / gate _had_quant_i8g, 4096 rows, group 128"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None},
        "ops": out,
        **({"cpu_baseline": {
            "value": round(total_bytes / sum(r["cpu_baseline"]["s_per_call"] for r in out) / 1e9, 3),
            "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": "each op's producer and adjoint through the oracle's restatement (single-threaded C) over "
                      "a sample of its rows, one pass an op, extrapolated in rows (the ops' own lines hold each); "
                      "the ops' bytes over their summed host seconds"}}
           if out and "cpu_baseline" in out[0] else {}),
    }), flush=True)


def stack_bench(args):
    """One complete LoRA step of a STACKS workload (C5: the 24-layer stack) on one GPU: the forward
    of every projection, layer by layer, then the backward in reverse (dX, dA, dB, the adapters'
    gradients staged), then AdamW on every factor with its bf16 copy refreshed. Synthetic: the weights are random
    b5 trellis.mad codes (any bytes are valid codes) with an f32 row scale and scale.col, prepared
    on the card; each projection's X and dY are shared random bf16 buffers of its shape (the
    projections between them -- norms, attention, the gated product -- are not this path)."""
    import ctypes as C

    import numpy as np
    import torch

    from r9700training_amd import R97Q_F32, _ptr, _stream, check, lib
    from r9700training_amd.optim import DeviceAdamW, config
    from r9700training_amd.qlinear import QWeight, bwd_workspace, device_desc, fwd_workspace

    proj, layers, T, r, alpha, metric, what = STACKS[args.workload]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    s = alpha / r
    L = lib()
    L.r97q_set_decode_once(DECODE_MODES[args.decode])
    g = torch.Generator(device="cuda").manual_seed(args.seed)
    rng = np.random.default_rng(args.seed)
    weights, keep = [], []
    for _layer in range(layers):
        for N, K in proj:
            codes = torch.randint(0, 256, (N, K * 5 // 8), dtype=torch.uint8, device=dev, generator=g)
            scale = torch.from_numpy((0.0005 + 0.01 * rng.random(N)).astype(np.float32).view(np.uint8)).to(dev)
            cf = torch.from_numpy((0.5 + rng.random(K // 128)).astype(np.float32)).to(dev)
            d = device_desc(dict(codes=codes, scale=scale), N, K, dict(
                bits=5, state_bits=16, run_rows=256, rb=1, mad=1, round_mad=1, mad_a=0x2F1E3D | 1,
                mad_b=0x9E3779B9, codes_row_bytes=K * 5 // 8, scale_dtype=0, scale_block_cols=0, scale_row_bytes=4))
            weights.append(QWeight(d, scale_col=cf))
            keep += [codes, scale, cf]
    X = {K: torch.randn((T, K), dtype=torch.bfloat16, device=dev, generator=g) for _, K in proj}
    dY = {N: torch.randn((T, N), dtype=torch.bfloat16, device=dev, generator=g) for N, _ in proj}
    Y = {N: torch.empty((T, N), dtype=torch.float32, device=dev) for N, _ in proj}
    dX = {K: torch.empty((T, K), dtype=torch.float32, device=dev) for _, K in proj}
    A = [(0.01 * torch.randn((r, K), generator=g, device=dev)).to(torch.bfloat16)
         for _ in range(layers) for _, K in proj]
    B = [(0.01 * torch.randn((N, r), generator=g, device=dev)).to(torch.bfloat16)
         for _ in range(layers) for N, _ in proj]
    tt = [torch.empty((T, r), dtype=torch.float32, device=dev) for _ in A]
    dA = [torch.zeros((r, a.shape[1]), dtype=torch.float32, device=dev) for a in A]
    dB = [torch.zeros((b.shape[0], r), dtype=torch.float32, device=dev) for b in B]
    wsf = max((fwd_workspace(T, N, K, r, dev) for N, K in proj), key=lambda x: x.numel())
    wsb = max((bwd_workspace(T, N, K, r, dev) for N, K in proj), key=lambda x: x.numel())
    masters = [a.float().contiguous() for a in A] + [b.float().contiguous() for b in B]
    copies = A + B
    opt = DeviceAdamW(masters, config(lr=1e-4), bf16_out=copies)
    stream = torch.cuda.current_stream()
    st = _stream(stream)
    P = _ptr

    def lora_step():
        for i, w in enumerate(weights):
            N, K = proj[i % len(proj)]
            check(L.r97q_lora_fwd_prep(T, N, K, P(X[K]), P(A[i]), r, s, P(tt[i]), P(wsf), wsf.numel(), st), "prep")
            check(L.r97q_qlinear_fwd_base(C.byref(w.w), P(X[K]), T, P(B[i]), r, P(Y[N]), R97Q_F32, P(wsf),
                                          wsf.numel(), st), "fwd")
        for i in reversed(range(len(weights))):
            N, K = proj[i % len(proj)]
            w = weights[i]
            check(L.r97q_qlinear_lora_bwd(C.byref(w.w), P(X[K]), P(dY[N]), T, P(A[i]), P(B[i]), r, s, P(tt[i]),
                                          P(dX[K]), R97Q_F32, 0, P(dA[i]), P(dB[i]), P(wsb), wsb.numel(), st), "bwd")
        opt.step(dA + dB, stream=stream, staged=True)

    steps, warmup = max(1, min(args.steps, 5)), max(1, min(args.warmup, 2))
    clock_settle = settle(lora_step, args.settle_s, torch, chunk=1) if args.settle_s > 0 else None
    for _ in range(warmup):
        lora_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        lora_step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    total = layers * sum(flops(T, N, K, r) for N, K in proj)
    tf = total / (ms * 1e-3) / 1e12
    cpu = None
    if args.cpu_seconds > 0:
        # the reference's host rows over the first layer's projections (the same weights and inputs),
        # extrapolated to every layer
        projs = []
        for i, (N, K) in enumerate(proj):
            c_d, s_d, f_d = keep[3 * i], keep[3 * i + 1], keep[3 * i + 2]
            codes, scale, dec_s = ref_decode(c_d.cpu().numpy(), s_d.cpu().numpy().view(np.float32),
                                             f_d.cpu().numpy(), N, K, 0x2F1E3D | 1, 0x9E3779B9)
            cache = {}

            def rows(idx, K=K, N=N, cache=cache):
                key = (int(idx[0]), len(idx), int(idx[-1]))
                if key not in cache:
                    it = torch.from_numpy(np.asarray(idx)).to(dev)
                    cache.clear()
                    cache[key] = (X[K][it].float().cpu().numpy().astype(np.float64),
                                  dY[N][it].float().cpu().numpy().astype(np.float64))
                return cache[key]

            projs.append(dict(N=N, K=K, codes=codes, scale=scale, decode_s=dec_s,
                              A=A[i].float().cpu().numpy().astype(np.float64),
                              B=B[i].float().cpu().numpy().astype(np.float64), rows=rows))
        cpu = cpu_baseline(projs, T, r, s, args.cpu_seconds, min(8, host_cores()), layers=layers,
                           what=" (one layer)" if layers > 1 else "", unit="tokens/s")
    print(json.dumps({
        "metric": metric,
        "value": round(T / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 3), "higher_is_better": True, "dtype": "bf16", "data": "synthetic",
        "tflops": round(tf, 3),
        "config": {"workload": what, "T": T, "layers": layers, "rank": r,
                   "decode": decode_label([decodes_once(args.decode, T, N, K) for N, K in proj])},
        "roofline": {"bound": "mfma", "achieved": round(tf, 3), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf / PEAK_BF16_TFLOPS, 4), "traffic": None},
        "memory_gib": round(torch.cuda.max_memory_allocated() / 2 ** 30, 2),
        "clock_settle": clock_settle,
        **({"cpu_baseline": cpu} if cpu else {}),
    }), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import ctypes as C

    import torch

    if args.calibrate_copy_mib > 0:
        n = args.calibrate_copy_mib << 18  # int32 elements
        src = torch.ones(n, dtype=torch.int32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_mib": args.calibrate_copy_mib, "launches": 3}), flush=True)
        return

    if args.workload == "vocab_head":
        return vocab_head_bench(args)
    if args.workload in STACKS:
        return stack_bench(args)
    if args.workload == "coded_fwd":
        return coded_fwd_bench(args)
    if args.workload == "ref_shapes":
        return ref_shapes_bench(args)
    if args.workload == "fused_quant":
        return fused_quant_bench(args)

    from r9700training_amd import R97Q_BF16, R97Q_F32, _ptr, _stream, check, lib
    from r9700training_amd.qlinear import bwd_workspace, fwd_workspace

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    T, N, K, r, alpha = CONFIGS[args.config]
    s = alpha / r
    inp = make_inputs(T, N, K, r, args.seed, dev, args.weight_form)
    w = inp["w"]
    out_dt = torch.float32 if args.out_dtype == "f32" else torch.bfloat16
    code = R97Q_F32 if args.out_dtype == "f32" else R97Q_BF16
    Y = torch.empty((T, N), dtype=out_dt, device=dev)
    dX = torch.empty((T, K), dtype=out_dt, device=dev)
    t = torch.empty((T, r), dtype=torch.float32, device=dev)
    dA = torch.zeros((r, K), dtype=torch.float32, device=dev)
    dB = torch.zeros((N, r), dtype=torch.float32, device=dev)
    L = lib()
    L.r97q_set_decode_once(DECODE_MODES[args.decode])
    wsf = fwd_workspace(T, N, K, r, dev)
    wsb = bwd_workspace(T, N, K, r, dev)
    stream = torch.cuda.current_stream()
    st = _stream(stream)
    P = lambda x: _ptr(x)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(6)] for _ in range(args.steps)]

    # The step: the forward's two stages, then the fused backward (r97q_qlinear_lora_bwd: the down
    # product, dA's chunk sums, and the dX launch that also takes dB and adds dA's sums). With e,
    # events around the forward's product and the whole backward.
    def step(e=None):
        check(L.r97q_lora_fwd_prep(T, N, K, P(inp["X"]), P(inp["A"]), r, s, P(t), P(wsf), wsf.numel(), st), "fwd_prep")
        if e: e[0].record(stream)
        check(L.r97q_qlinear_fwd_base(C.byref(w.w), P(inp["X"]), T, P(inp["B"]), r, P(Y), code, P(wsf),
                                      wsf.numel(), st), "fwd_base")
        if e: e[1].record(stream)
        check(L.r97q_qlinear_lora_bwd(C.byref(w.w), P(inp["X"]), P(inp["dY"]), T, P(inp["A"]), P(inp["B"]), r, s,
                                      P(t), P(dX), code, 0, P(dA), P(dB), P(wsb), wsb.numel(), st), "bwd")
        if e: e[4].record(stream)

    # The backward in its stages (the down product, both factor gradients in one launch, the dX
    # product alone), with events around the dX product: its launch duration with no other work.
    def staged_bwd(e):
        e[5].record(stream)
        check(L.r97q_lora_bwd_prep(T, N, K, P(inp["dY"]), P(inp["A"]), P(inp["B"]), P(t), r, s, P(wsb),
                                   wsb.numel(), st), "bwd_prep")
        check(L.r97q_lora_bwd_grads(T, N, K, P(inp["X"]), P(inp["dY"]), r, P(dA), P(dB), P(wsb), wsb.numel(), st),
              "bwd_grads")
        e[2].record(stream)
        check(L.r97q_qlinear_dx_base(C.byref(w.w), P(inp["dY"]), T, r, P(dX), code, 0, P(wsb), wsb.numel(), st),
              "dx_base")
        e[3].record(stream)

    clock_settle = settle(step, args.settle_s, torch) if args.settle_s > 0 else None
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_step = elapsed * 1e3 / args.steps
    # the same steps again with events around the forward's product and the backward, and the staged
    # backward with events around the dX product, for their launch durations
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(ev[i])
    torch.cuda.synchronize()
    ms_step_ev = (time.perf_counter() - t0) * 1e3 / args.steps
    for i in range(args.steps):
        staged_bwd(ev[i])
    torch.cuda.synchronize()
    fwd_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / args.steps
    bwd_ms = sum(e[1].elapsed_time(e[4]) for e in ev) / args.steps
    dx_ms = sum(e[2].elapsed_time(e[3]) for e in ev) / args.steps
    staged_ms = sum(e[5].elapsed_time(e[3]) for e in ev) / args.steps
    # The whole LoRA step: the same steps, then the factors' AdamW on the card (f32 master weights,
    # the reference Optimiser's update) taking dA, dB as the step's staged gradients (the grad-stage
    # flush's bf16 rounding, the buffers cleared for the next step) and writing the bf16 copies the
    # next step's kernels read: one launch.
    from r9700training_amd.optim import DeviceAdamW, config

    masters = [inp["A"].float().contiguous(), inp["B"].float().contiguous()]
    A_next, B_next = torch.empty_like(inp["A"]), torch.empty_like(inp["B"])
    opt = DeviceAdamW(masters, config(lr=1e-4), bf16_out=[A_next, B_next])
    dA.zero_()
    dB.zero_()

    def lora_step():
        step()
        opt.step([dA, dB], stream=stream, staged=True)

    for _ in range(args.warmup // 5 + 1):
        lora_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        lora_step()
    torch.cuda.synchronize()
    ms_lora_step = (time.perf_counter() - t0) * 1e3 / args.steps
    total_flops = flops(T, N, K, r)
    value = total_flops / (ms_step * 1e-3) / 1e12
    # the dominant kernel and its algorithmic work per launch (with the weight decoded once a call,
    # the event pair holds the decode launch and the product over its tiles)
    once = decodes_once(args.decode, T, N, K)
    kf, kd = ("predecode+qlinear_pd_kernel<fwd>", "predecode+qlinear_pd_kernel<dx>") if once else \
        ("qlinear_rt_kernel<fwd>", "qlinear_rt_kernel<dx>")
    kern = {kf: (fwd_ms, 2 * T * N * K + 2 * T * N * r),
            kd: (dx_ms, 2 * T * N * K + 2 * T * K * r)}
    name = max(kern, key=lambda k: kern[k][0])
    kms, kfl = kern[name]
    achieved = kfl / (kms * 1e-3) / 1e12
    traffic = profiled_traffic(name, args.config) if args.weight_form == "trellis" else None
    # the packed weight as the kernel reads it: every 512-token panel's workgroups walk the whole
    # stream (the panels sit on different XCDs, each with its own L2), so it is fetched once a panel
    packed_bytes = N * K if args.weight_form == "codes8" else N * K * 5 // 8
    panels = (T + 511) // 512
    line = {
        "metric": "qlinear+LoRA fwd+bwd TFLOP/s, % MFMA/HBM roofline; LoRA-step tokens/s",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: W ~ N(0,0.02) quantized by this repo's trellis quantizer; X, dY ~ N(0,1) bf16; "
                "A, B ~ N(0,0.01) bf16",
        "config": {"workload": f"{args.config.upper()}: IQR linear {N}x{K} (b5 trellis.mad L16, 256-row runs, "
                               f"f32 row scale + scale.col) + LoRA r{r} alpha {alpha:g}, T={T}, fwd+bwd, "
                               f"Y/dX {args.out_dtype}"
                               + (", weight in the int8-code form" if args.weight_form == "codes8" else ""),
                   "T": T, "N": N, "K": K, "rank": r, "alpha": alpha, "out_dtype": args.out_dtype,
                   "weight_form": args.weight_form, "decode": "once" if once else "fused"},
        "tokens_per_s": round(T / (ms_step * 1e-3), 1),
        "lora_step": {"tokens_per_s": round(T / (ms_lora_step * 1e-3), 1), "ms": round(ms_lora_step, 4),
                      "what": "fwd+bwd + the staged dA/dB flushed into AdamW on A, B (device, f32 masters) + their bf16 copies"},
        "flops_per_step": total_flops,
        "kernels_ms": {kf: round(fwd_ms, 4), kd + " (staged, alone)": round(dx_ms, 4),
                       "bwd (r97q_qlinear_lora_bwd)": round(bwd_ms, 4), "bwd (staged entries)": round(staged_ms, 4),
                       "other": round(ms_step_ev - fwd_ms - bwd_ms, 4), "ms_per_step_with_events": round(ms_step_ev, 4)},
        "roofline": {"bound": "mfma", "kernel": name, "achieved": round(achieved, 3),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic,
                     "hbm_GBs": None if traffic is None else round(traffic / (kms * 1e-3) / 1e9, 1),
                     "weight_stream_fetched_GBs": round(panels * packed_bytes / (kms * 1e-3) / 1e9, 1),
                     "weight_stream_note": f"the {packed_bytes / 1e6:.1f} MB packed weight fetched once by each "
                                           f"of the {panels} token panels' workgroups"},
        "quantizer_rel_err": round(inp["q"]["rel_err"], 4),
        "clock_settle": clock_settle,
    }
    # the rate the card sustains on MFMAs alone (power-limited: its clock falls well below the peak's
    # 2.4 GHz under a full matrix load): the nearer bar for the fused kernels
    ceil = mfma_ceiling(L, torch)
    line["roofline"]["ceiling_measured"] = dict(
        ceil, unit="TFLOP/s",
        what="v_mfma_f32_32x32x16_bf16 alone, operands in registers, 256 workgroups x 8 waves, ~40 ms a launch")
    line["roofline"]["frac_of_measured_ceiling"] = round(achieved / ceil["random_operands"], 4)
    if args.cpu_seconds > 0:
        pj = [c2_projection(inp, T, N, K, r)]
        line["cpu_baseline"] = cpu_baseline(pj, T, r, s, args.cpu_seconds, min(8, host_cores()))
        line["cpu_baseline_all_cores"] = (cpu_baseline(pj, T, r, s, args.cpu_seconds, host_cores())
                                          if host_cores() > 8 else line["cpu_baseline"])
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
