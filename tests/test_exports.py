"""The libraries load and export every function their headers declare (no GPU needed: nothing is
called). include/r97q.h is the C ABI of libr97q.so; include/r97/*.h the C++ contract of
libr97rows.so (the adjoint registry, the family table and the device weight store)."""
import ctypes as C
import os
import re
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "r9700training_amd")


def declared_c_functions(header):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M)
    return sorted({n for n in names if n.startswith(("r97q_", "r97_"))})


def test_c_abi_exports_every_declared_function():
    names = declared_c_functions(os.path.join(ROOT, "include", "r97q.h"))
    assert len(names) >= 19, names
    lib = C.CDLL(os.path.join(PKG, "libr97q.so"))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    from r9700training_amd import SIGNATURES
    unbound = [n for n in names if n not in SIGNATURES]
    assert not unbound, f"declared in r97q.h but not bound in r9700training_amd/__init__.py: {unbound}"


def test_rows_library_exports_the_contract():
    so = os.path.join(PKG, "libr97rows.so")
    C.CDLL(so)  # loads (its rows register at load)
    out = subprocess.run(["nm", "-D", "--defined-only", "-C", so], capture_output=True, text=True, check=True).stdout
    for fn in ["r97::twin_register", "r97::adjoint_register", "r97::twin_find", "r97::adjoint_find",
               "r97::adjoint_frozen", "r97::ops_registered", "r97::op_rows", "r97::family_register",
               "r97::family_find", "r97::adjoint_family_name", "r97::device_weight_get",
               "r97::device_weight_find", "r97::device_weight_count", "r97::device_weight_bytes",
               "r97::device_weight_clear"]:
        assert re.search(re.escape(fn) + r"(\[abi:cxx11\])?\(", out), fn
    # the registry's definitions are weak, so a host executable's own registry takes precedence
    weak = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True, check=True).stdout
    reg = [l for l in weak.splitlines() if "adjoint_register" in l]
    assert reg and all(l.split()[1] in ("W", "V") for l in reg), reg
