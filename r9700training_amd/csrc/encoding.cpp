// encoding.cpp -- a stored weight's plane table (R97Encoding, include/r97q.h) and the decode's
// description derived from it: the role rules of the reference's src/iqr_form.h:87-217, stated over
// this build's own plane table.
//
// Which plane is what is read from the roles alone: "codes" (the packed values) and "scale" are
// required, and either a "trellis" table (the state codebook: its extent is the state count, its
// block the run and row-block lengths) or a "zero" plane (the affine grid, each row a run of its
// own). "trellis.mad" makes the codebook computed from its two u32 words; "scale.1" is the second
// scale level; "scale.col" is a per-128-column f32 factor the description cannot carry, applied by
// the preparation (r97q_weight_prepare) as bf16(row scale * factor). Anything else is refused, not
// decoded as some other shape.
#include <cstdint>
#include <cstring>

#include "../../include/r97q.h"

namespace {

int find_role(const R97Encoding& e, const char* role) {
    for (int i = 0; i < e.n_planes && i < R97_ENC_MAX_PLANES; ++i)
        if (std::strncmp(e.plane[i].role, role, R97_ENC_STR) == 0) return i;
    return -1;
}

// the plane i holds at least `need` bytes
bool holds(const R97IqrStoredPlane* plane, int i, int64_t need) {
    return i >= 0 && plane[i].data != nullptr && plane[i].bytes >= need;
}

// log2 of n when n is a power of two, else -1
int exact_log2(int64_t n) {
    if (n <= 0 || (n & (n - 1)) != 0) return -1;
    int l = 0;
    while ((int64_t(1) << l) < n) ++l;
    return l;
}

// the decode's scale element type for a plane dtype, or -1
int scale_type_of(uint32_t dt) {
    switch (dt) {
        case R97_DT_F32: return R97_IQR_F32;
        case R97_DT_BF16: return R97_IQR_BF16;
        case R97_DT_F8E4M3: return R97_IQR_F8E4M3;
        case R97_DT_F16: return R97_IQR_F16;
        default: return -1;
    }
}

// bytes of one row of a per-row scale-like plane: one element a 128-column block, or one a row
int64_t per_row_bytes(uint32_t dt, int64_t block_cols, int64_t nkb) {
    return r97_enc_row_bytes(dt, block_cols > 0 ? nkb : 1);
}

}  // namespace

extern "C" {

int32_t r97_enc_dtype_bits(uint32_t dtype) {
    if (dtype >= R97_DT_U1 && dtype <= R97_DT_U12) return (int32_t)dtype;
    switch (dtype) {
        case R97_DT_I8: case R97_DT_F8E4M3: return 8;
        case R97_DT_BF16: case R97_DT_F16: return 16;
        case R97_DT_U32: case R97_DT_F32: return 32;
        default: return 0;
    }
}

int64_t r97_enc_row_bytes(uint32_t dtype, int64_t n) { return (n * r97_enc_dtype_bits(dtype) + 7) / 8; }

void r97_enc_plane_dims(const R97EncPlane* p, int64_t rows, int64_t cols, int64_t* prows, int64_t* pcols) {
    int64_t r = 0, c = 0;
    if (p->kind == R97_PLANE_TABLE) {
        r = p->extent[1] > 0 ? p->extent[1] : 1;
        c = p->extent[0] > 0 ? p->extent[0] : 1;
    } else {
        r = p->block[0] > 0 ? (rows + p->block[0] - 1) / p->block[0] : 1;
        c = p->block[1] > 0 ? (cols + p->block[1] - 1) / p->block[1] : 1;
    }
    if (prows) *prows = r;
    if (pcols) *pcols = c;
}

int64_t r97_enc_plane_bytes(const R97EncPlane* p, int64_t rows, int64_t cols) {
    int64_t r = 0, c = 0;
    r97_enc_plane_dims(p, rows, cols, &r, &c);
    return r * r97_enc_row_bytes(p->dtype, c);
}

int64_t r97_enc_plane_offsets(const R97Encoding* enc, int64_t rows, int64_t cols, int64_t* offsets) {
    if (enc == nullptr || enc->n_planes <= 0 || enc->n_planes > R97_ENC_MAX_PLANES) return -1;
    int64_t at = 0;
    for (int i = 0; i < enc->n_planes; ++i) {
        if (offsets) offsets[i] = at;
        at += (r97_enc_plane_bytes(&enc->plane[i], rows, cols) + 255) / 256 * 256;
    }
    return at;
}

int r97_iqr_desc_from_encoding(const R97Encoding* enc, const R97IqrStoredPlane* plane, int64_t rows, int64_t cols,
                               R97IqrDecodeDesc* out) {
    if (enc == nullptr || plane == nullptr || out == nullptr || rows <= 0 || cols <= 0) return 0;
    if (enc->n_planes <= 0 || enc->n_planes > R97_ENC_MAX_PLANES || cols % 128 != 0) return 0;
    const int64_t nkb = cols / 128;
    const int ic = find_role(*enc, "codes"), is = find_role(*enc, "scale");
    const int it = find_role(*enc, "trellis"), iz = find_role(*enc, "zero");
    if (ic < 0 || is < 0 || (it < 0 && iz < 0)) return 0;
    const R97EncPlane &cp = enc->plane[ic], &sp = enc->plane[is];

    R97IqrDecodeDesc d;
    std::memset(&d, 0, sizeof d);
    d.rows_all = rows;
    d.cols = cols;
    d.rows = rows;
    // the codes: an unsigned packed width
    d.bits = cp.dtype >= R97_DT_U1 && cp.dtype <= R97_DT_U12 ? (int32_t)cp.dtype : 0;
    if (d.bits <= 0) return 0;
    d.codes_row_bytes = r97_enc_row_bytes(cp.dtype, cols);
    if (!holds(plane, ic, rows * d.codes_row_bytes)) return 0;

    if (iz >= 0) {
        // the affine grid: a zero a block beside the scale, no trellis; every row its own run
        if (it >= 0) return 0;
        const R97EncPlane& zp = enc->plane[iz];
        // any plane dtype of 1-8 bits (an unsigned packed width, or an 8-bit one such as i8): the
        // decode reads the zero as that many unsigned bits
        d.zero_bits = r97_enc_dtype_bits(zp.dtype);
        if (d.zero_bits < 1 || d.zero_bits > 8) return 0;
        if (zp.block[0] != sp.block[0] || zp.block[1] != sp.block[1]) return 0;
        d.affine = 1;
        d.run_rows = 1;
        d.rb = 1;
        d.zero_row_bytes = per_row_bytes(zp.dtype, zp.block[1], nkb);
        if (!holds(plane, iz, rows * d.zero_row_bytes)) return 0;
        d.zero = plane[iz].data;
    } else {
        // the trellis: 2^state_bits states, run_rows rows a run (block[0]), rb rows a block (block[1])
        const R97EncPlane& tp = enc->plane[it];
        d.state_bits = exact_log2(tp.extent[0]);
        if (d.state_bits < 1) return 0;
        d.run_rows = (int32_t)tp.block[0];
        d.rb = tp.block[1] > 0 ? (int32_t)tp.block[1] : 1;
        if (d.run_rows < 1 || d.rb < 1) return 0;
    }

    d.scale_dtype = scale_type_of(sp.dtype);
    if (d.scale_dtype < 0) return 0;
    d.scale_block_cols = sp.block[1];
    d.scale_row_bytes = per_row_bytes(sp.dtype, d.scale_block_cols, nkb);
    if (!holds(plane, is, rows * d.scale_row_bytes)) return 0;

    const int is2 = find_role(*enc, "scale.1");
    if (is2 >= 0) {
        if (iz >= 0) return 0;  // the affine grid has no second level
        const R97EncPlane& s2 = enc->plane[is2];
        d.scale2_dtype = scale_type_of(s2.dtype);
        if (d.scale2_dtype < 0) return 0;
        d.scale2_block_rows = s2.block[0];
        d.scale2_block_cols = s2.block[1];
        d.scale2_row_bytes = per_row_bytes(s2.dtype, d.scale2_block_cols, nkb);
        const int64_t rows2 = d.scale2_block_rows > 0 ? (rows + d.scale2_block_rows - 1) / d.scale2_block_rows : 1;
        if (!holds(plane, is2, rows2 * d.scale2_row_bytes)) return 0;
        d.scale2 = plane[is2].data;
    }

    // a computed codebook rounds its codes; so does a stored one beside a scale.col factor
    const int im = find_role(*enc, "trellis.mad");
    d.mad = im >= 0;
    d.round_mad = d.mad || find_role(*enc, "scale.col") >= 0;
    if (it >= 0) {
        if (!holds(plane, it, enc->plane[it].extent[0])) return 0;  // one int8 a state
        d.lut = reinterpret_cast<const int8_t*>(plane[it].data);
        if (d.mad) {
            if (!holds(plane, im, 8)) return 0;
            // the codebook's A and B, read here: this plane is a host one even where the others are
            // device planes (8 bytes; the caller copies it out)
            uint32_t ab[2];
            std::memcpy(ab, plane[im].data, sizeof ab);
            d.mad_a = ab[0];
            d.mad_b = ab[1];
        }
    }
    d.codes = plane[ic].data;
    d.scale = plane[is].data;
    *out = d;
    return 1;
}

int r97_iqr_scale_col(const R97Encoding* enc, const R97IqrStoredPlane* plane, int64_t rows, int64_t cols,
                      const float** factor) {
    if (factor) *factor = nullptr;
    if (enc == nullptr || plane == nullptr || factor == nullptr || cols % 128 != 0) return 0;
    const int icf = find_role(*enc, "scale.col");
    if (icf < 0) return 1;
    const int is = find_role(*enc, "scale");
    if (is < 0) return 0;
    // one f32 a row times one f32 a 128-column block: the only pair the fold has a meaning for
    if (enc->plane[icf].dtype != R97_DT_F32 || !holds(plane, icf, cols / 128 * 4)) return 0;
    if (enc->plane[is].dtype != R97_DT_F32 || enc->plane[is].block[1] > 0) return 0;
    (void)rows;
    *factor = reinterpret_cast<const float*>(plane[icf].data);
    return 1;
}

}  // extern "C"
