"""r97_iqr_decode on the card: the reference's own decode, bit for bit (the reference's device test
tests/gpu/iqr_decode.cpp holds device bytes == host bytes exactly; here the host bytes are the golden
vectors the reference's r97_iqr_decode_host wrote, and the oracle)."""
import glob
import hashlib
import os

import numpy as np
import pytest
import torch

import iqr_synth as S
from test_oracle import planes_from

pytestmark = pytest.mark.gpu

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FILES = [f for f in sorted(glob.glob(os.path.join(G, "decode_*.npz"))) if "digest" not in f]


def run_decode(p, row0=0, rows=None):
    from gpu_util import device_desc
    from r9700training_amd import iqr_decode

    keep = []
    d = device_desc(p, keep, row0=row0, rows=rows)
    oc = torch.zeros((int(d.rows), p.cols), dtype=torch.int8, device="cuda")
    os_ = torch.zeros((int(d.rows), p.cols // 128), dtype=torch.int16, device="cuda")
    iqr_decode(d, oc, os_)
    torch.cuda.synchronize()
    return oc.cpu().numpy(), os_.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("path", FILES, ids=lambda p: os.path.basename(p)[7:-4])
def test_device_decode_golden(path):
    print(f"case {os.path.basename(path)}", flush=True)
    z = np.load(path)
    p = planes_from(z)
    codes, scale = run_decode(p)
    assert np.array_equal(codes, z["out_codes"])
    assert np.array_equal(scale, z["out_scale"])
    if p.affine:
        c = run_decode(p, row0=128, rows=100)
    else:
        c = run_decode(p, row0=p.run_rows, rows=p.run_rows)
    assert np.array_equal(c[0], z["chunk_codes"]) and np.array_equal(c[1], z["chunk_scale"])


def test_device_decode_trunk256():
    z = np.load(os.path.join(G, "decode_trunk256_digest.npz"))
    p = S.trellis(rows=768, cols=512, bits=5, state_bits=16, run_rows=256, rb=1, mad=1,
                  scale_dtype=S.F32, rowf=True, seed=int(z["seed"]))
    codes, scale = run_decode(p)
    assert hashlib.sha256(codes.tobytes()).hexdigest() == str(z["codes_sha"])
    assert hashlib.sha256(scale.tobytes()).hexdigest() == str(z["scale_sha"])


def test_device_decode_refuses_invalid():
    from gpu_util import device_desc
    from r9700training_amd import R97qError, iqr_decode

    p = S.trellis(rows=128, cols=256, bits=5, run_rows=64, seed=3)
    keep = []
    d = device_desc(p, keep)
    d.cols = 200  # not a multiple of 128
    oc = torch.zeros((128, 256), dtype=torch.int8, device="cuda")
    os_ = torch.zeros((128, 2), dtype=torch.int16, device="cuda")
    with pytest.raises(R97qError):
        iqr_decode(d, oc, os_)
