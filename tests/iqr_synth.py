"""Synthetic canonical IQR planes for the tests (host numpy arrays + a description).

The forms follow the case list the reference's decode test builds (tests/host/iqr_decode.cpp:82-212,
465-492): a computed `trellis.mad` codebook or a stored LUT, f32/bf16/e4m3 scales, a per-row f32
scale with `scale.col`, a `scale.1` second level, rb row blocks, a short last run, and the affine
grid (:341-461). Codes and scales are drawn from a seeded numpy generator; the planes are packed
LSB first along each row (src/iqr_decode.h:191-200).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

F32, BF16, E4M3, F16 = 0, 1, 2, 3


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """RNE with NaN quieting (src/iqr_decode.h:118-124), vectorised."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    q = ((u >> 16) | 0x40) & 0xFFFF
    return np.where(nan, q, r).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def pack_rows(vals: np.ndarray, bits: int) -> np.ndarray:
    """[rows, n] unsigned values < 2^bits -> [rows, ceil(n*bits/8)] bytes, LSB first."""
    rows, n = vals.shape
    nbytes = (n * bits + 7) // 8
    bitarr = ((vals.astype(np.uint32)[:, :, None] >> np.arange(bits, dtype=np.uint32)) & 1).astype(np.uint8)
    bitarr = bitarr.reshape(rows, n * bits)
    pad = nbytes * 8 - n * bits
    if pad:
        bitarr = np.concatenate([bitarr, np.zeros((rows, pad), np.uint8)], axis=1)
    return np.packbits(bitarr.reshape(rows, nbytes, 8), axis=2, bitorder="little").reshape(rows, nbytes)


def unpack_rows(packed: np.ndarray, bits: int, n: int) -> np.ndarray:
    rows = packed.shape[0]
    bitarr = np.unpackbits(packed.reshape(rows, -1, 1), axis=2, bitorder="little").reshape(rows, -1)
    bitarr = bitarr[:, : n * bits].reshape(rows, n, bits).astype(np.uint32)
    return (bitarr << np.arange(bits, dtype=np.uint32)).sum(axis=2).astype(np.uint32)


def mad_lut(A: int, B: int, state_bits: int) -> np.ndarray:
    st = np.arange(1 << state_bits, dtype=np.uint64)
    h = ((st & 0xFFFFFF) * (A & 0xFFFFFF) + B) & 0xFFFFFFFF
    h &= 0x3F3F3F3F
    v = (h & 0xFF) + ((h >> 8) & 0xFF) + ((h >> 16) & 0xFF) + ((h >> 24) & 0xFF)
    return (v.astype(np.int64) - 126).astype(np.int8)


@dataclass
class Planes:
    """Host planes of one weight and the fields of its description."""
    rows: int
    cols: int
    bits: int
    state_bits: int = 16
    run_rows: int = 256
    rb: int = 1
    mad: int = 1
    round_mad: int = 1
    mad_a: int = 0
    mad_b: int = 0
    scale_dtype: int = F32
    scale_block_cols: int = 0
    codes: np.ndarray = None          # uint8 [rows, codes_row_bytes]
    scale: np.ndarray = None          # uint8 bytes [rows, scale_row_bytes]
    lut: np.ndarray = None            # int8 [2^state_bits]
    scale2: np.ndarray = None         # uint8 bytes
    scale2_dtype: int = F32
    scale2_row_bytes: int = 0
    scale_col: np.ndarray = None      # f32 [cols/128] or None
    affine: int = 0
    zero: np.ndarray = None
    zero_bits: int = 0
    raw_codes: np.ndarray = field(default=None, repr=False)  # uint32 [rows, cols]

    @property
    def codes_row_bytes(self):
        return self.codes.shape[1]

    @property
    def scale_row_bytes(self):
        return self.scale.shape[1]

    def desc(self, row0: int = 0, rows: int | None = None):
        """The description over host memory (pointers into these arrays; keep `self` alive)."""
        from oracle.oracle import Desc

        rows = self.rows - row0 if rows is None else rows
        d = Desc()
        d.rows_all, d.cols, d.row0, d.rows = self.rows, self.cols, row0, rows
        d.bits, d.state_bits, d.run_rows, d.rb = self.bits, self.state_bits, self.run_rows, self.rb
        d.mad, d.round_mad, d.mad_a, d.mad_b = self.mad, self.round_mad, self.mad_a, self.mad_b
        d.lut = self.lut.ctypes.data if self.lut is not None else None
        d.codes = self.codes.ctypes.data + row0 * self.codes_row_bytes
        d.codes_row_bytes = self.codes_row_bytes
        d.scale = self.scale.ctypes.data + row0 * self.scale_row_bytes
        d.scale_dtype = self.scale_dtype
        d.scale_block_cols = self.scale_block_cols
        d.scale_row_bytes = self.scale_row_bytes
        d.affine = self.affine
        if self.affine:
            d.zero = self.zero.ctypes.data + row0 * self.zero.shape[1]
            d.zero_bits = self.zero_bits
            d.zero_row_bytes = self.zero.shape[1]
        if self.scale2 is not None:
            d.scale2 = self.scale2.ctypes.data
            d.scale2_dtype = self.scale2_dtype
            d.scale2_row_bytes = self.scale2_row_bytes
        return d


def trellis(rows, cols, bits, state_bits=16, run_rows=256, rb=1, mad=1, scale_dtype=F32,
            rowf=False, second=False, seed=0, scale_col=None, packed=False) -> Planes:
    """A trellis weight as tests/host/iqr_decode.cpp's Synth builds one (:100-211).

    rowf: one f32 scale a row plus a scale.col plane (ones unless `scale_col` given);
    otherwise one scale a 128-column block in `scale_dtype`. second: a scale.1 of 0.625.
    packed: draw the packed code bytes themselves (uniform bytes are uniform codes; fast at full
    layer sizes) and leave raw_codes unset."""
    rng = np.random.default_rng(seed)
    nkb = cols // 128
    raw = None if packed else rng.integers(0, 1 << bits, size=(rows, cols), dtype=np.uint32)
    p = Planes(rows=rows, cols=cols, bits=bits, state_bits=state_bits, run_rows=run_rows, rb=rb,
               mad=mad, round_mad=int(bool(mad or rowf)), scale_dtype=scale_dtype,
               scale_block_cols=0 if rowf else 128)
    p.raw_codes = raw
    if packed:
        p.codes = rng.integers(0, 256, size=(rows, (cols * bits + 7) // 8), dtype=np.uint8)
        if (cols * bits) % 8:  # the last byte's unused high bits stay clear, as pack_rows leaves them
            p.codes[:, -1] &= (1 << ((cols * bits) % 8)) - 1
    else:
        p.codes = pack_rows(raw, bits)
    A = (int(rng.integers(0, 1 << 32)) & 0xFFFFFF) | 1
    B = int(rng.integers(0, 1 << 32))
    p.mad_a, p.mad_b = A, B
    if mad:
        p.lut = mad_lut(A, B, state_bits)
    else:
        p.lut = (rng.integers(0, 253, size=1 << state_bits) - 126).astype(np.int8)
    n = 1 if rowf else nkb
    vals = (0.0005 + rng.integers(0, 1000, size=(rows, n)) * 0.00001).astype(np.float32)
    if scale_dtype == F32:
        p.scale = vals.view(np.uint8).reshape(rows, n * 4).copy()
    elif scale_dtype == BF16:
        p.scale = f32_to_bf16_bits(vals).view(np.uint8).reshape(rows, n * 2).copy()
    elif scale_dtype == E4M3:
        p.scale = (0x20 | rng.integers(0, 32, size=(rows, n))).astype(np.uint8)
    else:
        p.scale = vals.astype(np.float16).view(np.uint8).reshape(rows, n * 2).copy()
    if second:
        p.scale2 = np.array([0.625], np.float32).view(np.uint8).copy()
        p.scale2_dtype = F32
        p.scale2_row_bytes = 4
    if rowf:
        p.scale_col = (np.ones(nkb, np.float32) if scale_col is None
                       else np.ascontiguousarray(scale_col, np.float32))
    return p


def affine(rows, cols, bits, zero_bits, scale_dtype, seed=0) -> Planes:
    """The affine grid of tests/host/iqr_decode.cpp:344-391."""
    rng = np.random.default_rng(seed)
    nkb = cols // 128
    raw = rng.integers(0, 1 << bits, size=(rows, cols), dtype=np.uint32)
    zero = rng.integers(0, 1 << bits, size=(rows, nkb), dtype=np.uint32)
    vals = (0.0004 + rng.integers(0, 997, size=(rows, nkb)) * 2.0e-5).astype(np.float32)
    p = Planes(rows=rows, cols=cols, bits=bits, state_bits=0, run_rows=1, rb=1, mad=0, round_mad=0,
               scale_dtype=scale_dtype, scale_block_cols=128, affine=1, zero_bits=zero_bits)
    p.raw_codes = raw
    p.codes = pack_rows(raw, bits)
    p.zero = pack_rows(zero, zero_bits)
    if scale_dtype == F16:
        p.scale = vals.astype(np.float16).view(np.uint8).reshape(rows, nkb * 2).copy()
    else:
        p.scale = f32_to_bf16_bits(vals).view(np.uint8).reshape(rows, nkb * 2).copy()
    return p


# The decode case list: tests/host/iqr_decode.cpp:465-492, with a smaller run where the fixture
# would otherwise be large (the run length is a parameter of every form).
def decode_cases(run_rows=64):
    cases = []
    for bits in (3, 4, 5, 6):
        cases.append((f"trunk-u{bits}", dict(bits=bits, state_bits=16, rb=1, mad=1, scale_dtype=F32,
                                             rowf=True, second=False, cols=256, partial=False)))
        cases.append((f"stored-u{bits}", dict(bits=bits, state_bits=16, rb=1, mad=0, scale_dtype=BF16,
                                              rowf=False, second=False, cols=256, partial=False)))
    cases += [
        ("embedding", dict(bits=4, state_bits=12, rb=1, mad=0, scale_dtype=E4M3, rowf=False, second=True, cols=256, partial=False)),
        ("f32-128", dict(bits=4, state_bits=16, rb=1, mad=1, scale_dtype=F32, rowf=False, second=False, cols=512, partial=False)),
        ("e4m3-128", dict(bits=5, state_bits=12, rb=1, mad=0, scale_dtype=E4M3, rowf=False, second=True, cols=128, partial=False)),
        ("mad-rb", dict(bits=4, state_bits=16, rb=8, mad=1, scale_dtype=F32, rowf=True, second=False, cols=256, partial=False)),
        ("lut-rb", dict(bits=5, state_bits=16, rb=16, mad=0, scale_dtype=BF16, rowf=False, second=False, cols=256, partial=False)),
        ("rb-f32-row", dict(bits=4, state_bits=16, rb=8, mad=0, scale_dtype=F32, rowf=True, second=False, cols=256, partial=False)),
        ("short-last-mad", dict(bits=4, state_bits=16, rb=1, mad=1, scale_dtype=F32, rowf=True, second=False, cols=256, partial=True)),
        ("short-last-embedding", dict(bits=4, state_bits=12, rb=1, mad=0, scale_dtype=E4M3, rowf=False, second=True, cols=256, partial=True)),
        ("partial-workgroup", dict(bits=4, state_bits=16, rb=1, mad=1, scale_dtype=F32, rowf=True, second=False, cols=640, partial=False)),
    ]
    out = []
    for i, (name, c) in enumerate(cases):
        rows = 3 * run_rows + (run_rows // 2 if c["partial"] else 0)
        out.append((name, dict(rows=rows, cols=c["cols"], bits=c["bits"], state_bits=c["state_bits"],
                               run_rows=run_rows, rb=c["rb"], mad=c["mad"], scale_dtype=c["scale_dtype"],
                               rowf=c["rowf"], second=c["second"], seed=1000 + i)))
    return out


AFFINE_CASES = [
    ("drafter", dict(rows=300, cols=512, bits=2, zero_bits=8, scale_dtype=F16, seed=77)),
    ("drafter-narrow-zero", dict(rows=300, cols=384, bits=2, zero_bits=4, scale_dtype=F16, seed=78)),
    ("drafter-bf16", dict(rows=300, cols=256, bits=4, zero_bits=8, scale_dtype=BF16, seed=79)),
]


# ---------------------------------------------------------------- the encoding of a weight
# The plane table a container would write for these planes (include/r97q.h, R97Encoding), the
# plane roles src/iqr_form.h:87-217 reads, and each plane's bytes in plane order.
def encoding(p: Planes):
    """(R97Encoding, [host bytes of each plane, in plane order]) for the planes of `p`."""
    import r9700training_amd as R

    dt_of = {F32: R.R97_DT_F32, BF16: R.R97_DT_BF16, E4M3: R.R97_DT_F8E4M3, F16: R.R97_DT_F16}
    e = R.Encoding()
    e.scheme = b"affine" if p.affine else b"trellis"
    planes = []
    e.add("codes", R.R97_PLANE_TILED, p.bits, block=(1, 1))
    planes.append(p.codes)
    e.add("scale", R.R97_PLANE_TILED, dt_of[p.scale_dtype], block=(1, p.scale_block_cols))
    planes.append(p.scale)
    if p.affine:
        e.add("zero", R.R97_PLANE_TILED, p.zero_bits, block=(1, 128))
        planes.append(p.zero)
    else:
        e.add("trellis", R.R97_PLANE_TABLE, R.R97_DT_I8, block=(p.run_rows, p.rb), extent=(1 << p.state_bits, 1))
        planes.append(p.lut.view(np.uint8))
        if p.mad:
            e.add("trellis.mad", R.R97_PLANE_TABLE, R.R97_DT_U32, extent=(2, 1))
            planes.append(np.array([p.mad_a, p.mad_b], np.uint32).view(np.uint8))
    if p.scale2 is not None:
        e.add("scale.1", R.R97_PLANE_TILED, dt_of[p.scale2_dtype], block=(0, 0))
        planes.append(p.scale2)
    if p.scale_col is not None:
        e.add("scale.col", R.R97_PLANE_TILED, R.R97_DT_F32, block=(0, 128))
        planes.append(p.scale_col.view(np.uint8))
    return e, [np.ascontiguousarray(a).view(np.uint8).reshape(-1) for a in planes]


def joined(p: Planes):
    """(R97Encoding, one host byte buffer holding every plane at the library's joined offsets)."""
    import r9700training_amd as R

    e, planes = encoding(p)
    off = (C.c_int64 * R.R97_ENC_MAX_PLANES)()
    total = R.lib().r97_enc_plane_offsets(C.byref(e), p.rows, p.cols, off)
    assert total > 0
    buf = np.zeros(total, np.uint8)
    for i, a in enumerate(planes):
        n = R.lib().r97_enc_plane_bytes(C.byref(e.plane[i]), p.rows, p.cols)
        assert n == a.size, (e.plane[i].role, n, a.size)
        buf[off[i]:off[i] + n] = a
    return e, buf
