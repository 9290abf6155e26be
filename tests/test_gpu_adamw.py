"""AdamW on the card (r97q_adamw_step) against the reference's own Optimiser (src/optim.cpp), bit for
bit: the golden runs (tests/golden/adamw_runs.npz, written by the reference's optimiser over
LoRA-shaped parameters, six gradient sets, three configurations: defaults; warm-up + cosine with
weight decay, a no-decay parameter and a clip that bites; accumulation over two calls) replayed
through the device optimiser give the same master weights, moments and buffers."""
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
    opt = DeviceAdamW(params, config(**CONFIGS[name]), decay=list(z["decay"]))
    applied = []
    for s in range(6):
        applied.append(opt.step([torch.tensor(z[f"g{s}_{i}"], device="cuda") for i in range(3)]))
    torch.cuda.synchronize()
    for i in range(3):
        for k, t in (("w", params[i]), ("m", opt.m[i]), ("v", opt.v[i]), ("acc", opt.acc[i])):
            got = t.cpu().numpy()
            want = z[f"{name}_{k}{i}"]
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, k, i, np.abs(got - want).max())
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
