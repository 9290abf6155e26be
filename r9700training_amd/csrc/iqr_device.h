// iqr_device.h -- the IQR format on gfx950: scalar conversions, the trellis state value, and the
// column-stream layout the fused kernels read.
//
// Format arithmetic follows the reference's host header bit for bit (src/iqr_decode.h:118-315):
// bf16 RNE with NaN quieting, the f16 / OCP E4M3 readers, LSB-first packed code rows, the
// computed `trellis.mad` codebook, the tail-biting seam, the two-level block scale.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/r97q.h"

#define R97Q_HD __host__ __device__ inline

namespace r97q {

// ---------------------------------------------------------------- scalar formats
R97Q_HD uint16_t f32_to_bf16(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

R97Q_HD float bf16_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

R97Q_HD float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, u;
    if (e == 0) {
        if (m == 0) {
            u = sign;
        } else {
            int32_t ex = 127 - 15 + 1;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                --ex;
            }
            u = sign | ((uint32_t)ex << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        u = sign | 0x7F800000u | (m << 13);
    } else {
        u = sign | ((e + 112u) << 23) | (m << 13);
    }
    return __builtin_bit_cast(float, u);
}

R97Q_HD float e4m3_to_f32(uint8_t b) {
    const uint32_t s = (uint32_t)(b >> 7) << 31;
    uint32_t e = ((uint32_t)b >> 3) & 0xFu, m = (uint32_t)b & 0x7u, u;
    if (e == 0u) {
        if (m == 0u) {
            u = s;
        } else {
            int sh = 0;
            while (!(m & 0x8u)) {
                m <<= 1;
                ++sh;
            }
            u = s | ((uint32_t)(121 - sh) << 23) | ((m & 0x7u) << 20);
        }
    } else if (e == 0xFu && m == 0x7u) {
        u = s | 0x7FC00000u;
    } else {
        u = s | ((e + 120u) << 23) | (m << 20);
    }
    return __builtin_bit_cast(float, u);
}

R97Q_HD float load_scalar(const uint8_t* base, int32_t dtype, int64_t i) {
    switch (dtype) {
        case R97_IQR_F32: return __builtin_bit_cast(float, ((const uint32_t*)base)[i]);
        case R97_IQR_BF16: return bf16_to_f32(((const uint16_t*)base)[i]);
        case R97_IQR_F8E4M3: return e4m3_to_f32(base[i]);
        case R97_IQR_F16: return f16_to_f32(((const uint16_t*)base)[i]);
        default: return 0.0f;
    }
}

// element i of a packed code row, lowest bits first
R97Q_HD uint32_t load_bits(const uint8_t* row, int32_t bits, int64_t i) {
    const int64_t o = i * (int64_t)bits;
    const int64_t byte = o >> 3;
    const int sh = (int)(o & 7);
    uint32_t w = row[byte];
    if (sh + bits > 8) w |= (uint32_t)row[byte + 1] << 8;
    if (sh + bits > 16) w |= (uint32_t)row[byte + 2] << 16;
    if (sh + bits > 24) w |= (uint32_t)row[byte + 3] << 24;
    return (w >> sh) & ((1u << bits) - 1u);
}

// The byte-sum of the masked affine hash of a state: trellis.mad's computed codebook. The
// -126 offset rides in the dot's accumulator (0xFFFFFF82 is -126 in two's complement).
R97Q_HD int32_t mad_value(uint32_t st, uint32_t a24, uint32_t b) {
    const uint32_t h = (st * a24 + b) & 0x3F3F3F3Fu;
#if defined(__HIP_DEVICE_COMPILE__)
    return (int32_t)__builtin_amdgcn_udot4(h, 0x01010101u, 0xFFFFFF82u, false);
#else
    return (int32_t)((h & 0xFFu) + ((h >> 8) & 0xFFu) + ((h >> 16) & 0xFFu) + (h >> 24)) - 126;
#endif
}

// ---------------------------------------------------------------- the block scale
// The scale of row r's 128-column block kb, scale.1 settled to bf16 (src/iqr_decode.h:216-235).
R97Q_HD float block_scale(const R97IqrDecodeDesc& d, int64_t r, int64_t kb) {
    const int64_t bc = d.scale_block_cols > 0 ? d.scale_block_cols : d.cols;
    const int64_t gb = bc == d.cols ? 0 : (kb * 128) / bc;
    float v = load_scalar(d.scale + (r - d.row0) * d.scale_row_bytes, d.scale_dtype, gb);
    if (d.scale2) {
        const int64_t i2 = d.scale2_block_rows > 0 ? (r / d.scale2_block_rows) : 0;
        const int64_t j2 = d.scale2_block_cols > 0 ? (gb * bc) / d.scale2_block_cols : 0;
        const float s2 = load_scalar(d.scale2 + i2 * d.scale2_row_bytes, d.scale2_dtype, j2);
        v = bf16_to_f32(f32_to_bf16(v * s2));
    }
    return v;
}

// ---------------------------------------------------------------- the column-stream layout
//
// Rows are grouped in 32-row segments (segment g = rows 32g..32g+31). Within a trellis run
// [r0, r1), a column's codes are laid out in DESCENDING row order, LSB first: row 32g+i's code sits
// at bit bits*(31-i) of segment g's `bits` dwords, and the bits after segment g's last code are
// the first codes of the segment below it -- rows 32g-1, 32g-2, ... -- or, for the run's lowest
// segment, of the run's top segment: exactly the rows the tail-biting seam wraps to. So the
// trellis state of row n (its own code in the low bits, the previous ceil(L/b)-1 codes above it,
// masked to L bits) is the L-bit window at row n's code, read across into the next segment's first
// dword when it runs past the segment's end. No halo is stored: the plane is a permutation of the
// canonical code bits.
//
// Dword d of segment g for the 4 columns 4q..4q+3 is one 16-byte unit, so a wave reading dword d
// of 64 consecutive column groups issues one coalesced 1 KiB load:
//     stream[((g * bits + d) * (cols / 4) + q) * 4 + (col % 4)]
R97Q_HD int64_t stream_index(int64_t g, int32_t bits, int32_t d, int64_t cols, int64_t col) {
    return ((g * bits + d) * (cols >> 2) + (col >> 2)) * 4 + (col & 3);
}

// The segment whose first dword continues segment g's window: the one below it in the same run,
// or the run's top segment for the run's lowest one (the seam). `rows` is the weight's row count.
R97Q_HD int64_t halo_segment(int64_t g, int64_t run_rows, int64_t rows) {
    const int64_t r = g * 32;
    const int64_t r0 = (r / run_rows) * run_rows;
    if (r != r0) return g - 1;
    int64_t r1 = r0 + run_rows;
    if (r1 > rows) r1 = rows;
    return r1 / 32 - 1;
}

}  // namespace r97q
