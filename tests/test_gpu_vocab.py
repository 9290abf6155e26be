"""The vocabulary head's transposed product on the card (r97q_vocab_head_transpose) against the
oracle's restatement of the reference's kernels (src/adjoint/device/vocab_head.hip:88-163, pinned in
tests/test_oracle.py), with the reference test's own checks (tests/gpu/vocab_head.cpp): a one-hot
cotangent row per class selects one weight row; chunking the token rows is additive; the cast
rounds like f32 -> bf16.

Bar: d_x within relative L2 1e-5 of the f64 restatement, the reference's own f32 level: each class
weight code * scale enters the MFMA as the exact sum of two bf16 values (two products, f32
accumulation), as the reference's kernel multiplies the exact int8 code in f32."""
import ctypes as C

import numpy as np
import pytest
import torch

import iqr_synth as S
from gpu_util import device_desc, dev, rel_l2
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-5

FORMS = {
    "trunk-b5": dict(bits=5, state_bits=16, run_rows=256, rb=1, mad=1, scale_dtype=S.F32, rowf=True),
    "stored-u4": dict(bits=4, state_bits=16, run_rows=128, rb=1, mad=0, scale_dtype=S.BF16, rowf=False),
    "embedding": dict(bits=4, state_bits=12, run_rows=256, rb=1, mad=0, scale_dtype=S.E4M3, rowf=False, second=True),
}


def make_class(rng, form, rows, K, ids, keep, seed):
    """A class: its planes on the card (the decode description), ids, scale.col; and the oracle's
    view of it (decoded codes, the settled bf16 scale, ids, scale.col)."""
    cf = (0.5 + rng.random(K // 128)).astype(np.float32)
    p = S.trellis(rows=rows, cols=K, seed=seed, **FORMS[form])
    p.scale_col = None  # the head multiplies its scale.col after the product; the decode does not fold it
    d = device_desc(p, keep)
    codes, gscale = O.decode(p.desc())
    ids_d, cf_d = dev(ids.astype(np.int32)), dev(cf)
    keep += [ids_d, cf_d]
    return (d, ids_d, cf_d), (codes, gscale.astype(np.uint16), ids.astype(np.int32), cf)


def head_and_oracle(rng, K, sizes, forms, vocab_offset=0, stray=0, transform=128):
    from r9700training_amd.vocab_head import VocabHead

    vocab = sum(sizes)
    perm = rng.permutation(vocab) + vocab_offset
    keep, dev_cls, orc_cls, at = [], [], [], 0
    for i, (n, form) in enumerate(zip(sizes, forms)):
        ids = perm[at:at + n].copy()
        at += n
        if stray:
            ids[:stray] = vocab_offset + vocab + rng.integers(0, 9, stray)
        dc, oc = make_class(rng, form, n, K, ids, keep, seed=100 + i)
        dev_cls.append(dc)
        orc_cls.append(oc)
    head = VocabHead(K, vocab, dev_cls, vocab_offset=vocab_offset, transform=transform)
    head._keep += keep
    return head, orc_cls, vocab


@pytest.mark.parametrize("rows,K,sizes,forms,offset,transform", [
    (37, 256, [1000, 700], ["trunk-b5", "stored-u4"], 0, 128),
    (300, 512, [1500, 333, 900], ["trunk-b5", "embedding", "trunk-b5"], 4096, 128),
    (600, 384, [2048], ["trunk-b5"], 0, 0),
])
def test_vocab_head_matches_oracle(rows, K, sizes, forms, offset, transform):
    print(f"case vocab head rows={rows} K={K} sizes={sizes} forms={forms} offset={offset} transform={transform}",
          flush=True)
    rng = np.random.default_rng(rows + K)
    head, orc_cls, vocab = head_and_oracle(rng, K, sizes, forms, offset, stray=5, transform=transform)
    dy = S.f32_to_bf16_bits(rng.standard_normal((rows, vocab)).astype(np.float32))
    d0 = rng.standard_normal((rows, K)).astype(np.float32)
    d_x = torch.tensor(d0, device="cuda")
    head.transpose(torch.from_numpy(dy.view(np.int16)).cuda().view(torch.bfloat16), d_x)
    torch.cuda.synchronize()
    want = O.vocab_head_transpose(dy, orc_cls, vocab_offset=offset, transform=transform, d_x=d0)
    base = O.fwht128(d0) if transform else d0.astype(np.float64)
    e = rel_l2(d_x.cpu().numpy() - base, want - base)
    print(f"  rel L2 {e:.3e}", flush=True)
    assert e <= TOL


def test_vocab_head_ranges_and_padding():
    """A class of several 4096-row decode ranges (20077 rows: four whole, one short) whose short last
    range is padded to a multiple of 128 rows; the ranges split over several product slices."""
    print("case vocab head ranges", flush=True)
    rng = np.random.default_rng(4)
    rows, K = 64, 128
    head, orc_cls, vocab = head_and_oracle(rng, K, [20000 + 77], ["trunk-b5"], transform=0)
    dy = S.f32_to_bf16_bits(rng.standard_normal((rows, vocab)).astype(np.float32))
    d_x = torch.zeros((rows, K), device="cuda")
    head.transpose(torch.from_numpy(dy.view(np.int16)).cuda().view(torch.bfloat16), d_x)
    torch.cuda.synchronize()
    want = O.vocab_head_transpose(dy, orc_cls)
    e = rel_l2(d_x.cpu().numpy(), want)
    print(f"  rel L2 {e:.3e}", flush=True)
    assert e <= TOL


def test_vocab_head_two_row_blocks():
    """Token rows past one block (4096 + 4 = 4100 rows): the weights are decoded once, beside the first
    block's gather, and the second block's gather and product reuse them; d_x is added into."""
    print("case vocab head rows=4100 (two token-row blocks)", flush=True)
    rng = np.random.default_rng(4100)
    rows, K = 4100, 256
    head, orc_cls, vocab = head_and_oracle(rng, K, [1000, 700], ["trunk-b5", "stored-u4"], transform=128)
    dy = S.f32_to_bf16_bits(rng.standard_normal((rows, vocab)).astype(np.float32))
    d0 = rng.standard_normal((rows, K)).astype(np.float32)
    d_x = torch.tensor(d0, device="cuda")
    head.transpose(torch.from_numpy(dy.view(np.int16)).cuda().view(torch.bfloat16), d_x)
    torch.cuda.synchronize()
    want = O.vocab_head_transpose(dy, orc_cls, transform=128, d_x=d0)
    base = O.fwht128(d0)
    got = d_x.cpu().numpy()
    e, e2 = rel_l2(got - base, want - base), rel_l2(got[4096:] - base[4096:], want[4096:] - base[4096:])
    print(f"  rel L2 {e:.3e}, the second block's 4 rows {e2:.3e}", flush=True)
    assert e <= TOL and e2 <= TOL


def test_vocab_head_one_hot_and_chunking():
    """The reference test's checks: one-hot rows against the class rows they select (row scale,
    scale.col, then the transform); the same rows in two calls equal one call."""
    print("case vocab head one-hot", flush=True)
    rng = np.random.default_rng(8)
    K, rows = 256, 8
    head, orc_cls, vocab = head_and_oracle(rng, K, [768, 512], ["trunk-b5", "trunk-b5"], transform=128)
    dy = np.zeros((rows, vocab), np.uint16)
    want = np.zeros((rows, K))
    for m in range(rows):
        for c, (codes, gscale, ids, cf) in enumerate(orc_cls):
            r = 32 * c + 8 * m + 1
            dy[m, ids[r]] = 0x3F80
            want[m] += (codes[r].astype(np.float64) * np.repeat(S.bf16_bits_to_f32(gscale[r]).astype(np.float64), 128)
                        * np.repeat(cf.astype(np.float64), 128))
    want = O.fwht128(want)
    dyt = torch.from_numpy(dy.view(np.int16)).cuda().view(torch.bfloat16)
    one = torch.zeros((rows, K), device="cuda")
    head.transpose(dyt, one)
    two = torch.zeros((rows, K), device="cuda")
    head.transpose(dyt[:3].contiguous(), two[:3])
    rest = torch.zeros((rows - 3, K), device="cuda")
    head.transpose(dyt[3:].contiguous(), rest)
    torch.cuda.synchronize()
    two[3:] = rest
    got = one.cpu().numpy()
    e = rel_l2(got, want)
    print(f"  one-hot rel L2 {e:.3e}", flush=True)
    assert e <= TOL
    assert torch.equal(one, two)
    assert rel_l2(got, 2 * want) > 0.3  # teeth: a doubled transform misses


def test_vocab_head_full_size():
    """The benchmark's head at its full size: four b5 trellis.mad classes of 32768, 65536, 98304 and
    51712 rows (248320 in all, ids ascending within a class, a random partition of the vocabulary),
    n_embd 2048, fwht128, 4096 token rows -- 61 ranges, 8 product slices. Checked against float64
    products of the oracle's decoded weights: 8 sampled token rows (the first, tile edges, the last),
    and every row at once through the column sum (the head is linear in its token rows:
    sum_m d_x[m] = H . sum_c ((sum_m dy[m, ids_c]) . W_c) * scale.col_c). The rows within TOL (1e-5;
    measured 1.7e-6), the column sum within 1e-4 (measured 1.0e-5: the 4096 rows' f32 results,
    each rounded on its own, summed against a sum taken before the product, with much
    cancellation); a dropped low half misses by ~2e-3."""
    from r9700training_amd.vocab_head import VocabHead

    print("case vocab head full size: 248320 rows, n_embd 2048, 4096 token rows", flush=True)
    sizes, K, rows = [32768, 65536, 98304, 51712], 2048, 4096
    vocab = sum(sizes)
    rng = np.random.default_rng(248320)
    perm = rng.permutation(vocab)
    keep, dev_cls, orc, at = [], [], [], 0
    for i, n in enumerate(sizes):
        p = S.trellis(rows=n, cols=K, bits=5, state_bits=16, run_rows=256, rb=1, mad=1, scale_dtype=S.F32,
                      rowf=True, seed=700 + i, packed=True)
        p.scale_col = None  # the head multiplies its scale.col after the product
        ids = np.sort(perm[at:at + n]).astype(np.int32)
        at += n
        cf = (0.5 + rng.random(K // 128)).astype(np.float32)
        d = device_desc(p, keep)
        ids_d, cf_d = dev(ids), dev(cf)
        keep += [ids_d, cf_d]
        dev_cls.append((d, ids_d, cf_d))
        codes, gscale = O.decode(p.desc())
        orc.append((codes, S.bf16_bits_to_f32(gscale.astype(np.uint16)).astype(np.float64), ids, cf.astype(np.float64)))
    head = VocabHead(K, vocab, dev_cls, transform=128)
    head._keep += keep
    gen = torch.Generator(device="cuda").manual_seed(248320)
    dy = torch.randn((rows, vocab), generator=gen, device="cuda").to(torch.bfloat16)
    d_x = torch.zeros((rows, K), device="cuda")
    head.transpose(dy, d_x)
    torch.cuda.synchronize()
    sample = np.array([0, 1, 511, 512, 2047, 2048, 4094, 4095])
    ridx = torch.from_numpy(sample).cuda()
    dys = dy.index_select(0, ridx).double().cpu().numpy()
    dysum = dy.sum(0, dtype=torch.float64).cpu().numpy()[None]
    got, gotsum = d_x.index_select(0, ridx).double().cpu().numpy(), d_x.sum(0, dtype=torch.float64).cpu().numpy()[None]
    del dy, d_x
    torch.cuda.empty_cache()

    def reference(y):  # float64: sum over classes and 128-column blocks of (y[:, ids] * scale) . codes * cf
        out = np.zeros((y.shape[0], K))
        for codes, scale, ids, cf in orc:
            yc = y[:, ids]
            for kb in range(K // 128):
                blk = slice(128 * kb, 128 * kb + 128)
                out[:, blk] += ((yc * scale[:, kb]) @ codes[:, blk].astype(np.float64)) * cf[kb]
        return O.fwht128(out)

    e, es = rel_l2(got, reference(dys)), rel_l2(gotsum, reference(dysum))
    print(f"  rows {sample.tolist()}: rel L2 {e:.3e}; column sums rel L2 {es:.3e}", flush=True)
    assert e <= TOL and es <= 1e-4


def test_vocab_head_in_a_graph():
    """The head captured in a HIP graph and replayed: a call forks its weights' decode onto the
    device's side stream (beside the gather on the caller's stream) and joins it back before the
    products, which a capture records as a branch of the graph. Each replay, with eager work and
    synchronisation between replays, equals the eager call bit for bit (the arithmetic's order is
    fixed)."""
    print("case vocab head in a graph rows=300 K=256", flush=True)
    rng = np.random.default_rng(12)
    K, rows = 256, 300
    head, _, vocab = head_and_oracle(rng, K, [1500, 900], ["trunk-b5", "stored-u4"])
    gen = torch.Generator(device="cuda").manual_seed(12)
    dy = torch.randn((rows, vocab), generator=gen, device="cuda").to(torch.bfloat16)
    ws = torch.empty(head.workspace_bytes(rows), dtype=torch.uint8, device="cuda")
    d_x = torch.zeros((rows, K), device="cuda")
    head.transpose(dy, d_x, ws)  # eager first: the side stream is made outside the capture
    torch.cuda.synchronize()
    eager = d_x.clone()
    assert float(eager.abs().sum()) > 0
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        d_x.zero_()  # a fill kernel, not a memset node
        head.transpose(dy, d_x, ws, stream=torch.cuda.current_stream())
    for i in range(4):
        d_x.fill_(float("nan"))  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(d_x, eager), i


def test_vocab_head_on_a_caller_stream():
    """The head on a stream of the caller's own (not the default one): the decode forks from that
    stream and joins back into it, so work the caller enqueues after the call on the same stream
    sees the whole result; bit-equal to the call on the default stream."""
    print("case vocab head on a caller stream rows=300 K=256", flush=True)
    rng = np.random.default_rng(13)
    K, rows = 256, 300
    head, _, vocab = head_and_oracle(rng, K, [1500, 900], ["trunk-b5", "stored-u4"])
    gen = torch.Generator(device="cuda").manual_seed(13)
    dy = torch.randn((rows, vocab), generator=gen, device="cuda").to(torch.bfloat16)
    want = torch.zeros((rows, K), device="cuda")
    head.transpose(dy, want)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    got = torch.zeros((rows, K), device="cuda")
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        head.transpose(dy, got, stream=side)
        copy = got.clone()  # enqueued after the call on the same stream
    torch.cuda.synchronize()
    assert torch.equal(copy, want) and torch.equal(got, want)


def test_vocab_head_cast():
    from r9700training_amd.vocab_head import cast

    x = torch.randn(5000, device="cuda") * 100
    x[:4] = torch.tensor([0.0, -0.0, 1.0 / 16384.0, float("nan")], device="cuda")
    y = cast(x)
    torch.cuda.synchronize()
    want = x.cpu().to(torch.bfloat16)
    assert torch.equal(y.cpu()[4:].view(torch.int16), want[4:].view(torch.int16))
    assert torch.equal(y.cpu()[:3].view(torch.int16), want[:3].view(torch.int16)) and torch.isnan(y.cpu()[3])


def test_vocab_head_refusals():
    from r9700training_amd import R97qError, VocabPlan, lib

    rng = np.random.default_rng(1)
    head, _, vocab = head_and_oracle(rng, 128, [256], ["trunk-b5"])
    L = lib()
    bad = VocabPlan.from_buffer_copy(head.plan)
    bad.cls[0].scale_col = None
    assert L.r97q_vocab_head_workspace_bytes(C.byref(bad), 4) == -1
    assert b"incomplete" in L.r97q_last_error()
    bad = VocabPlan.from_buffer_copy(head.plan)
    bad.transform = 64
    assert L.r97q_vocab_head_workspace_bytes(C.byref(bad), 4) == -1
    dy = torch.zeros((4, vocab), dtype=torch.bfloat16, device="cuda")
    d_x = torch.zeros((4, 128), device="cuda")
    with pytest.raises(R97qError, match="workspace"):
        head.transpose(dy, d_x, workspace=torch.empty(16, dtype=torch.uint8, device="cuda"))
