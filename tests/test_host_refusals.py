"""Argument refusals of the C ABI that happen on the host before any GPU work (no GPU needed: each
call returns its status before touching a device pointer or the HIP runtime)."""
import ctypes as C
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
R97Q_EINVAL = 1  # include/r97q.h


def test_bwd_prep_needs_t_with_a_rank():
    """r97q_lora_bwd_prep writes dB's operand from t: without t a later r97q_lora_bwd_grads could not
    tell that operand is missing, so the prep refuses (rank 0 needs no t)."""
    lib = C.CDLL(os.path.join(ROOT, "r9700training_amd", "libr97q.so"))
    f = lib.r97q_lora_bwd_prep
    f.restype = C.c_int
    f.argtypes = [C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32,
                  C.c_float, C.c_void_p, C.c_int64, C.c_void_p]
    lib.r97q_last_error.restype = C.c_char_p
    fake = C.c_void_p(0x1000)  # never dereferenced: the refusal comes first
    rc = f(256, 256, 256, fake, fake, fake, None, 16, 2.0, fake, 1 << 30, None)
    assert rc == R97Q_EINVAL
    assert b"t" in lib.r97q_last_error()


def test_mfma_probe_refuses_a_short_out_buffer():
    """r97q_mfma_probe writes 256 * 512 floats: an out_count below that is refused before the launch."""
    lib = C.CDLL(os.path.join(ROOT, "r9700training_amd", "libr97q.so"))
    f = lib.r97q_mfma_probe
    f.restype = C.c_int
    f.argtypes = [C.c_int32, C.c_int32, C.c_void_p, C.c_int64, C.c_void_p]
    lib.r97q_last_error.restype = C.c_char_p
    fake = C.c_void_p(0x1000)  # never dereferenced: the refusal comes first
    assert f(100, 0, fake, 256 * 512 - 1, None) == R97Q_EINVAL
    assert b"out_count" in lib.r97q_last_error()
    assert f(0, 0, fake, 256 * 512, None) == R97Q_EINVAL
