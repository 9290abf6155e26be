"""This build's device rows inside the reference's own registry (CPU only).

The reference's walk finds a device row through its registry (src/adjoint_registry.cpp:53-113). Its
executable exports that registry and loads plugin rows into the same symbol scope; libr97rows.so's
registry definitions are weak, so there its static registrations land in the reference's registry.
This test shows it with the reference's own registry compiled from its sources (oracle/_ref, the
checker's build of src/adjoint_registry.cpp and the host rows): loaded first into the global scope,
then libr97rows.so, the reference's adjoint_find returns this build's rows for the device side, with
this build's frozen positions, and still its own host rows for the host side. It runs in a child
process so the load order is the one stated (an earlier test may have loaded libr97rows.so alone)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.path.join(ROOT, "oracle", "_ref", "libr97ref.so")
ROWS = os.path.join(ROOT, "r9700training_amd", "libr97rows.so")

CHILD = r'''
import ctypes as C, sys
ref = C.CDLL(sys.argv[1], mode=C.RTLD_GLOBAL)
rows = C.CDLL(sys.argv[2], mode=C.RTLD_GLOBAL)
ref.ref_adjoint_find.restype = C.c_void_p
ref.ref_adjoint_find.argtypes = [C.c_char_p, C.c_int32, C.c_char_p, C.c_int64]
ref.ref_adjoint_frozen.restype = C.c_int32
ref.ref_adjoint_frozen.argtypes = [C.c_char_p, C.c_int32, C.c_char_p, C.c_int64, C.POINTER(C.c_int32)]

class DlInfo(C.Structure):
    _fields_ = [("fname", C.c_char_p), ("fbase", C.c_void_p), ("sname", C.c_char_p), ("saddr", C.c_void_p)]
libc = C.CDLL(None)
libc.dladdr.argtypes = [C.c_void_p, C.POINTER(DlInfo)]

def where(p):
    if not p:
        return "none"
    info = DlInfo()
    assert libc.dladdr(C.c_void_p(p), C.byref(info)) != 0
    return info.fname.decode().rsplit("/", 1)[-1]

def frozen(op, dev, dt, g):
    f = (C.c_int32 * 4)()
    n = ref.ref_adjoint_frozen(op.encode(), dev, dt.encode(), g, f)
    return list(f[:min(n, 4)])

ref.ref_adjoint_find_spec.restype = C.c_void_p
ref.ref_adjoint_find_spec.argtypes = [C.c_char_p, C.c_int32, C.c_char_p]
ref.ref_adjoint_frozen_spec.restype = C.c_int32
ref.ref_adjoint_frozen_spec.argtypes = [C.c_char_p, C.c_int32, C.c_char_p, C.POINTER(C.c_int32)]

def frozen_spec(op, dev, spec):
    f = (C.c_int32 * 4)()
    n = ref.ref_adjoint_frozen_spec(op.encode(), dev, spec.encode(), f)
    return list(f[:min(n, 4)])

for op, spec in [("had_quant_act_i8g", "n=256;group=128"), ("rmsnorm_had_quant_i8g", "n=5120;group=128;eps=1e-6"),
                 ("gated_had_quant_i8g", "n=256;group=128"), ("gated_had_quant_i8g", "n=256;group=128;act=silu"),
                 ("gate_had_quant_i8g", "n=256;group=128;act=sigmoid"), ("gate_had_quant_i8g", "n=256;group=128"),
                 ("gated_had_quant_i8g", "n=256;group=128;act=sigmoid"), ("rmsnorm_had_quant_i8g", "n=4096;group=2048")]:
    print("spec", op, spec, where(ref.ref_adjoint_find_spec(op.encode(), 1, spec.encode())), frozen_spec(op, 1, spec))

for op, dev, dt, g in [("gemm_nt", 1, "bf16", 0), ("lora_shrink", 1, "bf16", 0), ("lora_shrink", 1, "i8", 128),
                       ("lora_shrink", 1, "fp8_e4m3", 128), ("lora_expand", 1, "bf16", 0),
                       ("lora_expand_mm", 1, "bf16", 0), ("lora_expand_mm", 0, "bf16", 0),
                       ("gemm_nt_q", 1, "i8a8h", 128), ("gemm_nt", 0, "bf16", 0), ("lora_shrink", 0, "bf16", 0),
                       ("lora_expand", 0, "bf16", 0)]:
    print(op, dev, dt, where(ref.ref_adjoint_find(op.encode(), dev, dt.encode(), g)), frozen(op, dev, dt, g))
'''


def test_rows_register_into_the_reference_registry():
    if not os.path.exists(REF):
        pytest.skip("oracle/_ref is built only where the reference's sources are present")
    if not os.path.exists(ROWS):
        pytest.fail(f"{ROWS} is not built (run __graft_entry__.build())")
    out = subprocess.run([sys.executable, "-c", CHILD, REF, ROWS], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    lines = out.stdout.strip().splitlines()
    spec = {tuple(line.split(" ", 3)[1:3]): line.split(" ", 3)[3] for line in lines if line.startswith("spec ")}
    got = {tuple(line.split(" ", 3)[:3]): line.split(" ", 3)[3] for line in lines if not line.startswith("spec ")}
    # the quantiser's rows: this build's on the device side, keyed by the reference's predicates
    # (src/adjoint/device/quant.hip:129-159): the gated row for silu or no act, the gate for sigmoid
    # only, no row for a group wider than 1024; the norm's gain frozen
    assert spec[("had_quant_act_i8g", "n=256;group=128")].startswith("libr97rows.so")
    assert spec[("rmsnorm_had_quant_i8g", "n=5120;group=128;eps=1e-6")] == "libr97rows.so [1]"
    assert spec[("gated_had_quant_i8g", "n=256;group=128")] == "libr97rows.so []"
    assert spec[("gated_had_quant_i8g", "n=256;group=128;act=silu")] == "libr97rows.so []"
    assert spec[("gate_had_quant_i8g", "n=256;group=128;act=sigmoid")] == "libr97rows.so []"
    assert spec[("gate_had_quant_i8g", "n=256;group=128")].startswith("none")
    assert spec[("gated_had_quant_i8g", "n=256;group=128;act=sigmoid")].startswith("none")
    assert spec[("rmsnorm_had_quant_i8g", "n=4096;group=2048")].startswith("none")
    # device rows: this build's, with this build's (the reference's) frozen positions
    assert got[("gemm_nt", "1", "bf16")] == "libr97rows.so [1]"
    assert got[("lora_shrink", "1", "bf16")] == "libr97rows.so [1, 2, 3]"
    assert got[("lora_shrink", "1", "i8")] == "libr97rows.so [2, 3]"
    assert got[("lora_shrink", "1", "fp8_e4m3")] == "libr97rows.so [2, 3]"
    assert got[("lora_expand", "1", "bf16")] == "libr97rows.so [1, 2, 3]"
    assert got[("lora_expand_mm", "1", "bf16")] == "libr97rows.so [1, 2, 3]"
    assert got[("gemm_nt_q", "1", "i8a8h")] == "libr97rows.so [1, 2, 3]"
    # host rows: still the reference's own
    for op in ("gemm_nt", "lora_shrink", "lora_expand", "lora_expand_mm"):
        assert got[(op, "0", "bf16")].startswith("libr97ref.so"), got[(op, "0", "bf16")]
