"""AdamW on the card (r97q_adamw_step) against the reference's own Optimiser (src/optim.cpp), bit for
bit: the golden runs (tests/golden/adamw_runs.npz, written by the reference's optimiser over
LoRA-shaped parameters, six gradient sets, three configurations: defaults; warm-up + cosine with
weight decay, a no-decay parameter and a clip that bites; accumulation over two calls) replayed
through the device optimiser give the same master weights, moments and buffers.

The fused forms (one launch over many parameters, the bf16 copies written by the update, the device
rows' staged gradients taken through the flush's bf16 rounding) are held to the oracle's optimiser
(oracle/oracle.c orc_adamw_step, pinned to the reference's runs by the CPU tests), bit for bit."""
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CONFIGS = {
    "plain": dict(),
    "schedule_clip_decay": dict(lr=1e-2, warmup_steps=2, total_steps=5, lr_floor_frac=0.1, weight_decay=0.05,
                                clip_norm=1.0),
    "accumulate": dict(lr=3e-3, accum_steps=2, clip_norm=1e3),
}


@pytest.mark.parametrize("name", list(CONFIGS))
def test_adamw_matches_reference_bits(name):
    from r9700training_amd.optim import DeviceAdamW, config

    print(f"case adamw {name}", flush=True)
    z = np.load(os.path.join(G, "adamw_runs.npz"))
    params = [torch.tensor(z[f"w{i}"], device="cuda") for i in range(3)]
    outs = [torch.empty(p.shape, dtype=torch.bfloat16, device="cuda") for p in params]
    opt = DeviceAdamW(params, config(**CONFIGS[name]), decay=list(z["decay"]), bf16_out=outs)
    applied = []
    for s in range(6):
        applied.append(opt.step([torch.tensor(z[f"g{s}_{i}"], device="cuda") for i in range(3)]))
    torch.cuda.synchronize()
    for i in range(3):
        for k, t in (("w", params[i]), ("m", opt.m[i]), ("v", opt.v[i]), ("acc", opt.acc[i])):
            got = t.cpu().numpy()
            want = z[f"{name}_{k}{i}"]
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, k, i, np.abs(got - want).max())
        assert torch.equal(outs[i].cpu(), params[i].cpu().to(torch.bfloat16)), (name, "bf16 copy", i)
    assert opt.updates.value == z[f"{name}_updates"] and opt.pending.value == z[f"{name}_pending"]
    assert applied == ([True] * 6 if name != "accumulate" else [False, True] * 3)


def test_bf16_copies_round_to_nearest_even():
    from r9700training_amd.optim import bf16_copies

    x = torch.randn(100000, device="cuda") * 3.0
    x[:4] = torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, float("inf"), float("nan")], device="cuda")
    (y,) = bf16_copies([x])
    torch.cuda.synchronize()
    want = x.cpu().to(torch.bfloat16)
    got = y.cpu()
    assert torch.equal(got[2:3], want[2:3]) and torch.isnan(got[3])
    assert torch.equal(got[4:], want[4:]) and torch.equal(got[:2], want[:2])


def _bits(t):
    return t.cpu().numpy().view(np.uint32)


def _bf16_rounded(a):
    return torch.tensor(a).to(torch.bfloat16).to(torch.float32).numpy()


@pytest.mark.parametrize("staged", [False, True])
@pytest.mark.parametrize("cfg", [dict(lr=2e-3, weight_decay=0.01, clip_norm=0.5),
                                 dict(lr=1e-3, accum_steps=3, clip_norm=2.0, warmup_steps=2, total_steps=6),
                                 dict(lr=5e-3, accum_steps=2)])
def test_many_parameters_match_oracle(cfg, staged):
    """37 parameters (three launch tables; sizes that leave norm chunks spanning parameters and
    tables), against the oracle's optimiser on the same gradients (staged: the flush's bf16 value)."""
    from r9700training_amd.optim import DeviceAdamW, config
    from oracle import oracle as O

    print(f"case adamw many {cfg} staged={staged}", flush=True)
    rng = np.random.default_rng(11 + staged)
    sizes = [int(x) for x in rng.integers(1, 9000, 37)]
    sizes[5], sizes[20] = 4096, 12289
    w0 = [(0.1 * rng.standard_normal(n)).astype(np.float32) for n in sizes]
    decay = [int(x) for x in rng.integers(0, 2, 37)]
    params = [torch.tensor(w, device="cuda") for w in w0]
    outs = [torch.empty(n, dtype=torch.bfloat16, device="cuda") for n in sizes]
    opt = DeviceAdamW(params, config(**cfg), decay=decay, bf16_out=outs)
    ref = O.AdamW(O.AdamWConfig.make(**cfg), [w.copy() for w in w0], decay=decay)
    for s in range(7):
        g = [(rng.standard_normal(n) * (0.3 + s)).astype(np.float32) for n in sizes]
        gd = [torch.tensor(x, device="cuda") for x in g]
        got = opt.step(gd, staged=staged)
        want = ref.step([_bf16_rounded(x) for x in g] if staged else g)
        assert got == want
        if staged:
            torch.cuda.synchronize()
            assert all(not x.any() for x in gd), "the staging buffers are cleared"
    torch.cuda.synchronize()
    for i in range(37):
        for k, t, r in (("w", params[i], ref.w[i]), ("m", opt.m[i], ref.m[i]), ("v", opt.v[i], ref.v[i]),
                        ("acc", opt.acc[i], ref.acc[i])):
            assert np.array_equal(_bits(t), r.view(np.uint32)), (k, i)
        assert torch.equal(outs[i].cpu(), params[i].cpu().to(torch.bfloat16))
    assert opt.updates.value == ref.step_count.value and opt.pending.value == ref.pending.value


def test_step_refusals():
    from r9700training_amd import R97qError
    from r9700training_amd.optim import DeviceAdamW, config

    p = [torch.zeros(10, device="cuda")]
    opt = DeviceAdamW(p, config())
    with pytest.raises(ValueError):
        opt.step([torch.zeros(11, device="cuda")])
    with pytest.raises(ValueError):
        DeviceAdamW(p, config(), bf16_out=[torch.zeros(10, device="cuda")])
    opt.cfg.accum_steps = 0
    with pytest.raises(R97qError, match="accum_steps"):
        opt.step([torch.zeros(10, device="cuda")])
