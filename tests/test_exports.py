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
               "r97::device_weight_clear", "r97::device::scratch_stats", "r97::device::scratch_reset",
               "r97::device::scratch_alloc", "r97::device::scratch_free", "r97::device::grad_stage_slot"]:
        assert re.search(re.escape(fn) + r"(\[abi:cxx11\])?\(", out), fn
    # the registry's definitions are weak, so a host executable's own registry takes precedence
    weak = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True, check=True).stdout
    reg = [l for l in weak.splitlines() if "adjoint_register" in l]
    assert reg and all(l.split()[1] in ("W", "V") for l in reg), reg
    led = [l for l in weak.splitlines() if "scratch_alloc" in l or "scratch_free" in l]
    assert len(led) == 2 and all(l.split()[1] in ("W", "V") for l in led), led


def test_plugin_table():
    """The kernel-plugin exports radiance's loader reads (the reference's
    src/adjoint/device/plugin.hip:38-80): the plugin's identity, and empty op-schema and kernel
    tables (the rows register into r97's registry instead)."""
    from_header = declared_c_functions_rad(os.path.join(ROOT, "include", "r97", "rad_plugin_abi.h"))
    assert from_header == ["rad_kernel_at", "rad_kernel_count", "rad_kernel_schema_at", "rad_kernel_schema_count",
                           "rad_plugin_abi_version", "rad_plugin_info"], from_header
    lib = C.CDLL(os.path.join(PKG, "libr97rows.so"))

    class Info(C.Structure):
        _fields_ = [("kind", C.c_int32), ("name", C.c_char_p), ("version", C.c_char_p),
                    ("description", C.c_char_p), ("target", C.c_char_p)]

    lib.rad_plugin_abi_version.restype = C.c_uint32
    lib.rad_plugin_info.restype = C.POINTER(Info)
    lib.rad_kernel_schema_at.restype = C.c_void_p
    lib.rad_kernel_at.restype = C.c_void_p
    info = lib.rad_plugin_info().contents
    assert info.name == b"r97" and info.target == b"gfx950" and info.version and info.description
    assert lib.rad_plugin_abi_version() == 0  # no radiance header in this tree: set at build time
    assert lib.rad_kernel_schema_count() == 0 and lib.rad_kernel_count() == 0
    assert lib.rad_kernel_schema_at(0) is None and lib.rad_kernel_at(0) is None


def declared_c_functions_rad(header):
    text = re.sub(r"/\*.*?\*/|//[^\n]*", " ", open(header).read(), flags=re.S)
    return sorted(set(re.findall(r"\b(rad_[a-z_]+)\s*\(", text)))
