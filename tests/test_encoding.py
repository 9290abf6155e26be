"""The stored weight's encoding and the description derived from it (libr97q.so's
r97_iqr_desc_from_encoding / r97_iqr_scale_col / r97_enc_plane_offsets), on the CPU.

The derivation restates the role rules of the reference's src/iqr_form.h:87-217. Two things pin it:
  * the assertions of the reference's own test of that derivation (tests/host/iqr_form.cpp:185-342),
    restated over this build's plane table: the trunk form, the stored bf16 form, the affine grid and
    the refusals, on planes built as that test builds them (:55-180);
  * every form the decode's case list holds (tests/host/iqr_decode.cpp:465-492, the affine grids
    :341-461): the description derived from the encoding equals the one the synthetic builder states,
    field for field, and decodes (through the oracle) to the same bytes.
The oracle only decodes here; the derivation under test is the product's."""
import ctypes as C

import numpy as np
import pytest

import iqr_synth as S
import r9700training_amd as R
from oracle import oracle as O


def lib():
    return R.lib()


def stored(planes):
    arr = (R.StoredPlane * R.R97_ENC_MAX_PLANES)()
    for i, a in enumerate(planes):
        if a is None:
            continue
        arr[i].data = a.ctypes.data
        arr[i].bytes = a.size
    return arr


def derive(enc, planes, rows, cols):
    d = R.Desc()
    ok = lib().r97_iqr_desc_from_encoding(C.byref(enc), stored(planes), rows, cols, C.byref(d))
    return d if ok else None


def scale_col(enc, planes, rows, cols):
    f = C.POINTER(C.c_float)()
    ok = lib().r97_iqr_scale_col(C.byref(enc), stored(planes), rows, cols, C.byref(f))
    return ok, (C.cast(f, C.c_void_p).value if f else None)


def oracle_decode(d):
    return O.decode(O.Desc.from_buffer_copy(d))


def plane_bytes(enc, i, rows, cols):
    return lib().r97_enc_plane_bytes(C.byref(enc.plane[i]), rows, cols)


def role_index(enc, role):
    for i in range(enc.n_planes):
        if enc.plane[i].role.decode() == role:
            return i
    return -1


# ---------------------------------------------------------------- the reference test's forms
def trunk_form(rows, cols, with_mad, with_scale_col):
    """tests/host/iqr_form.cpp:55-115: codes=u6[1x1], scale=f32[1x*], trellis=i8{65536x1} with a
    256-row run, trellis.mad=u32{2x1}, scale.col=f32[*x128]."""
    nkb = cols // 128
    e = R.Encoding()
    e.scheme, e.transform = b"trellis", b"fwht128"
    e.add("codes", R.R97_PLANE_TILED, R.R97_DT_U[6], block=(1, 1))
    e.add("scale", R.R97_PLANE_TILED, R.R97_DT_F32, block=(1, 0))
    e.add("trellis", R.R97_PLANE_TABLE, R.R97_DT_I8, block=(256, 1), extent=(65536, 1))
    if with_mad:
        e.add("trellis.mad", R.R97_PLANE_TABLE, R.R97_DT_U32, extent=(2, 1))
    if with_scale_col:
        e.add("scale.col", R.R97_PLANE_TILED, R.R97_DT_F32, block=(0, 128))
    planes = [np.zeros(plane_bytes(e, i, rows, cols), np.uint8) for i in range(e.n_planes)]
    it = role_index(e, "trellis")
    planes[it][:] = (np.arange(planes[it].size) * 37 + 11).astype(np.uint8)
    if with_mad:
        planes[role_index(e, "trellis.mad")][:] = np.array([0x00ABCDEF, 7], np.uint32).view(np.uint8)
    vals = ((np.arange(rows)[:, None] * 13 + np.arange(cols)[None, :] * 7) % 64).astype(np.uint32)
    planes[0][:] = S.pack_rows(vals, 6).reshape(-1)
    planes[1][:] = (0.0001 * (np.arange(rows) + 1)).astype(np.float32).view(np.uint8)
    if with_scale_col:
        planes[role_index(e, "scale.col")][:] = (2.0 + np.arange(nkb)).astype(np.float32).view(np.uint8)
    return e, planes


def bf16_form(rows, cols):
    """tests/host/iqr_form.cpp:117-145: codes=u6, scale=bf16[1x128], trellis, trellis.mad."""
    nkb = cols // 128
    e = R.Encoding()
    e.scheme, e.transform = b"trellis", b"fwht128"
    e.add("codes", R.R97_PLANE_TILED, R.R97_DT_U[6], block=(1, 1))
    e.add("scale", R.R97_PLANE_TILED, R.R97_DT_BF16, block=(1, 128))
    e.add("trellis", R.R97_PLANE_TABLE, R.R97_DT_I8, block=(256, 1), extent=(65536, 1))
    e.add("trellis.mad", R.R97_PLANE_TABLE, R.R97_DT_U32, extent=(2, 1))
    planes = [np.zeros(plane_bytes(e, i, rows, cols), np.uint8) for i in range(e.n_planes)]
    planes[2][:] = (np.arange(planes[2].size) * 29 + 5).astype(np.uint8)
    planes[1][:] = S.f32_to_bf16_bits((0.5 + 0.25 * np.arange(rows * nkb)).astype(np.float32)).view(np.uint8)
    return e, planes


def affine_form(rows, cols):
    """tests/host/iqr_form.cpp:147-180: codes=u4, scale=bf16[1x128], zero=u8[1x128]."""
    nkb = cols // 128
    e = R.Encoding()
    e.scheme = b"affine"
    e.add("codes", R.R97_PLANE_TILED, R.R97_DT_U[4], block=(1, 1))
    e.add("scale", R.R97_PLANE_TILED, R.R97_DT_BF16, block=(1, 128))
    e.add("zero", R.R97_PLANE_TILED, R.R97_DT_U[8], block=(1, 128))
    planes = [np.zeros(plane_bytes(e, i, rows, cols), np.uint8) for i in range(e.n_planes)]
    vals = ((np.arange(rows)[:, None] * 5 + np.arange(cols)[None, :] * 3) & 15).astype(np.uint32)
    planes[0][:] = S.pack_rows(vals, 4).reshape(-1)
    planes[2][:] = np.tile((np.arange(nkb) + 1).astype(np.uint8), rows)
    planes[1][:] = S.f32_to_bf16_bits((0.125 * (np.arange(rows * nkb) + 1)).astype(np.float32)).view(np.uint8)
    return e, planes, vals


def test_trunk_form():
    """tests/host/iqr_form.cpp:185-257 (check_trunk)."""
    rows, cols = 512, 256
    e, planes = trunk_form(rows, cols, True, True)
    d = derive(e, planes, rows, cols)
    assert d is not None, "the trunk form is a description"
    assert d.bits == 6 and d.state_bits == 16 and d.run_rows == 256 and d.rb == 1
    assert d.mad == 1 and d.round_mad == 1 and (d.mad_a, d.mad_b) == (0x00ABCDEF, 7)
    assert d.scale_dtype == S.F32 and d.scale_block_cols == 0 and not d.scale2 and d.affine == 0
    assert d.codes == planes[0].ctypes.data and d.scale == planes[1].ctypes.data
    assert d.lut == planes[2].ctypes.data
    out = oracle_decode(d)
    assert out is not None and out[0].shape == (rows, cols) and out[1].shape == (rows, cols // 128)
    # the factor the description cannot carry: the scale.col plane, handed to the preparation's fold
    ok, f = scale_col(e, planes, rows, cols)
    assert ok and f == planes[role_index(e, "scale.col")].ctypes.data
    # a computed codebook without scale.col still rounds; a stored one beside scale.col rounds too
    e2, p2 = trunk_form(rows, cols, True, False)
    d2 = derive(e2, p2, rows, cols)
    assert d2.round_mad == 1 and scale_col(e2, p2, rows, cols) == (1, None)
    e3, p3 = trunk_form(rows, cols, False, True)
    d3 = derive(e3, p3, rows, cols)
    assert d3.mad == 0 and d3.round_mad == 1 and d3.lut == p3[2].ctypes.data


def test_bf16_form():
    """tests/host/iqr_form.cpp:259-288 (check_bf16)."""
    rows, cols = 512, 256
    e, planes = bf16_form(rows, cols)
    d = derive(e, planes, rows, cols)
    assert d is not None
    assert d.scale_dtype == S.BF16 and d.scale_block_cols == 128 and d.scale_row_bytes == (cols // 128) * 2
    assert d.affine == 0 and not d.scale2
    codes, scale = oracle_decode(d)
    assert np.array_equal(scale.view(np.uint8).reshape(-1), planes[1]), "the stored form's scales are its own"
    assert codes.min() >= -127 and codes.max() <= 127


def test_affine_form():
    """tests/host/iqr_form.cpp:290-318 (check_affine): every code is its stored code less the block's
    zero."""
    rows, cols = 256, 256
    e, planes, vals = affine_form(rows, cols)
    d = derive(e, planes, rows, cols)
    assert d is not None
    assert d.affine == 1 and d.bits == 4 and d.zero_bits == 8 and d.zero_row_bytes == cols // 128
    assert d.run_rows == 1 and d.rb == 1 and not d.scale2
    codes, _ = oracle_decode(d)
    zero = (np.arange(cols)[None, :] // 128 + 1).astype(np.int32)
    assert np.array_equal(codes.astype(np.int32), vals.astype(np.int32) - zero)


def test_affine_zero_i8():
    """src/iqr_form.h:110-124: the zero plane may be any dtype of 1-8 bits (rad_dtype_bits), so an i8
    zero plane is the same grid as the u8 one, read as 8 unsigned bits; a 12-bit or f32 zero is
    refused."""
    rows, cols = 256, 256
    e, planes, vals = affine_form(rows, cols)
    iz = role_index(e, "zero")
    e.plane[iz].dtype = R.R97_DT_I8
    d = derive(e, planes, rows, cols)
    assert d is not None, "an i8 zero plane is an affine description"
    assert d.affine == 1 and d.zero_bits == 8 and d.zero_row_bytes == cols // 128
    codes, _ = oracle_decode(d)
    zero = (np.arange(cols)[None, :] // 128 + 1).astype(np.int32)
    assert np.array_equal(codes.astype(np.int32), vals.astype(np.int32) - zero)
    for dt in (R.R97_DT_U[12], R.R97_DT_F32):
        e, planes, _ = affine_form(rows, cols)
        e.plane[role_index(e, "zero")].dtype = dt
        planes[iz] = np.zeros(plane_bytes(e, iz, rows, cols), np.uint8)
        assert derive(e, planes, rows, cols) is None, dt


def test_refusals():
    """tests/host/iqr_form.cpp:320-342 (check_refusals)."""
    rows, cols = 256, 256
    e, planes = trunk_form(rows, cols, True, True)
    e.n_planes = 2  # codes and scale only: no trellis and no zero
    assert derive(e, planes, rows, cols) is None
    e, planes = trunk_form(rows, cols, True, True)
    e.plane[role_index(e, "trellis")].extent[0] = 1000  # not a power of two
    assert derive(e, planes, rows, cols) is None
    # a bf16 block scale beside scale.col: derivable, but the fold refuses the pair
    e, planes = bf16_form(rows, cols)
    e.add("scale.col", R.R97_PLANE_TILED, R.R97_DT_F32, block=(0, 128))
    planes.append(np.zeros(cols // 128 * 4, np.uint8))
    assert derive(e, planes, rows, cols) is not None
    assert scale_col(e, planes, rows, cols)[0] == 0
    # a short codes plane
    e, planes = trunk_form(rows, cols, True, True)
    planes[0] = planes[0][: planes[0].size // 2]
    assert derive(e, planes, rows, cols) is None
    # a column count the decode does not tile, and no encoding at all
    e, planes = trunk_form(rows, cols, True, True)
    assert derive(e, planes, rows, 250) is None
    d = R.Desc()
    assert lib().r97_iqr_desc_from_encoding(None, stored(planes), rows, cols, C.byref(d)) == 0


FIELDS = ["rows_all", "cols", "row0", "rows", "bits", "state_bits", "run_rows", "rb", "mad", "round_mad", "mad_a",
          "mad_b", "codes_row_bytes", "scale_dtype", "scale_block_cols", "scale_row_bytes", "affine", "zero_bits",
          "zero_row_bytes", "scale2_dtype", "scale2_row_bytes", "scale2_block_rows", "scale2_block_cols"]


@pytest.mark.parametrize("name,kw", S.decode_cases() + [("affine-" + n, dict(kw, affine=True))
                                                         for n, kw in S.AFFINE_CASES])
def test_every_decode_form_derives_its_description(name, kw):
    """Each form of the decode's case list, written as an encoding over its planes (joined at the
    library's offsets), derives the description the builder states, and decodes to the same bytes."""
    kw = dict(kw)
    p = S.affine(**{k: v for k, v in kw.items() if k != "affine"}) if kw.pop("affine", False) else S.trellis(**kw)
    e, buf = S.joined(p)
    off = (C.c_int64 * R.R97_ENC_MAX_PLANES)()
    total = lib().r97_enc_plane_offsets(C.byref(e), p.rows, p.cols, off)
    assert total == buf.size and all(off[i] % 256 == 0 for i in range(e.n_planes))
    planes = [buf[off[i]:off[i] + plane_bytes(e, i, p.rows, p.cols)] for i in range(e.n_planes)]
    d = derive(e, planes, p.rows, p.cols)
    assert d is not None, name
    want = p.desc()
    for f in FIELDS:
        if f in ("mad_a", "mad_b") and not p.mad:
            continue  # the builder draws A and B for a stored codebook too; the decode never reads them
        assert getattr(d, f) == getattr(want, f), (name, f, getattr(d, f), getattr(want, f))
    got, ref = oracle_decode(d), O.decode(want)
    assert np.array_equal(got[0], ref[0]) and np.array_equal(got[1], ref[1]), name
    ok, f = scale_col(e, planes, p.rows, p.cols)
    assert ok and (f is None) == (p.scale_col is None)


# radiance's plane dtypes by name -> this build's codes: the mapping a caller applies when it copies
# a RadEncoding into an R97Encoding (each packed width to its bit count, the rest one to one;
# radiance's own numeric values are not in this tree)
RAD_TO_R97 = dict({f"RAD_U{b}": R.R97_DT_U[b] for b in range(1, 13)},
                  RAD_I8=R.R97_DT_I8, RAD_U32=R.R97_DT_U32, RAD_F32=R.R97_DT_F32, RAD_BF16=R.R97_DT_BF16,
                  RAD_F16=R.R97_DT_F16, RAD_F8E4M3=R.R97_DT_F8E4M3)


def from_rad(scheme, planes):
    """An R97Encoding copied field for field from a RadEncoding written as (role, kind, RAD dtype
    name, block, extent) tuples, the dtype mapped by name."""
    e = R.Encoding()
    e.scheme = scheme.encode()
    for role, kind, dt, block, extent in planes:
        e.add(role, R.R97_PLANE_TILED if kind == "tiled" else R.R97_PLANE_TABLE, RAD_TO_R97[dt], block=block,
              extent=extent)
    return e


@pytest.mark.parametrize("form", ["f32-row+scale.col", "bf16-128", "f16-128", "e4m3-128", "bf16-128+scale.1"])
def test_rad_mapping_scale_forms(form):
    """Each scale form a stored weight's RadEncoding can carry, copied through the name mapping,
    derives the description the synthetic builder states for the same planes (scale dtype, block,
    row bytes, scale.1, the scale.col factor) and decodes to the same bytes."""
    rows, cols = 256, 256
    kind = {"f32-row+scale.col": dict(rowf=True, scale_col=np.linspace(0.5, 1.5, cols // 128).astype(np.float32)),
            "bf16-128": dict(scale_dtype=S.BF16), "f16-128": dict(scale_dtype=S.F16),
            "e4m3-128": dict(scale_dtype=S.E4M3), "bf16-128+scale.1": dict(scale_dtype=S.BF16, second=True)}[form]
    p = S.trellis(rows=rows, cols=cols, bits=4, run_rows=128, seed=3, **kind)
    rad_scale = {S.F32: "RAD_F32", S.BF16: "RAD_BF16", S.F16: "RAD_F16", S.E4M3: "RAD_F8E4M3"}[p.scale_dtype]
    planes = [("codes", "tiled", "RAD_U4", (1, 1), (0, 0)),
              ("scale", "tiled", rad_scale, (1, p.scale_block_cols), (0, 0)),
              ("trellis", "table", "RAD_I8", (p.run_rows, p.rb), (1 << p.state_bits, 1)),
              ("trellis.mad", "table", "RAD_U32", (0, 0), (2, 1))]
    data = [p.codes, p.scale, p.lut.view(np.uint8), np.array([p.mad_a, p.mad_b], np.uint32).view(np.uint8)]
    if p.scale2 is not None:
        planes.append(("scale.1", "tiled", "RAD_F32", (0, 0), (0, 0)))
        data.append(p.scale2)
    if p.scale_col is not None:
        planes.append(("scale.col", "tiled", "RAD_F32", (0, 128), (0, 0)))
        data.append(p.scale_col.view(np.uint8))
    e = from_rad("trellis", planes)
    data = [np.ascontiguousarray(a).view(np.uint8).reshape(-1) for a in data]
    d = derive(e, data, rows, cols)
    assert d is not None, form
    want = p.desc()
    for f in FIELDS:
        assert getattr(d, f) == getattr(want, f), (form, f, getattr(d, f), getattr(want, f))
    got, ref = oracle_decode(d), O.decode(want)
    assert np.array_equal(got[0], ref[0]) and np.array_equal(got[1], ref[1]), form
    ok, fcol = scale_col(e, data, rows, cols)
    assert ok and (fcol is None) == (p.scale_col is None), form
