// act_tiles.h -- the token operand of the register-fed fused kernels, laid out in MFMA fragment
// order.
//
// An activation [T, R] (T tokens, R the reduction length: K for the forward's X, N for dX's dY),
// bf16, is stored as blocks of 32 token rows x 64 reduction values (4 KiB). Block (rb, s) holds
// rows 32rb..32rb+31 and values 64s..64s+63; blocks are ordered s-major, rb-minor, so the blocks
// every workgroup of an XCD reads in one step are contiguous (spread over all L2 channels, where
// a row-major order puts them a whole row apart, on few channels). Inside a block, slice j
// (1 KiB, j = 0..3) is what one v_mfma_f32_32x32x16_bf16 takes as its A operand: lane
// l = 32h + i holds row 32rb + i, values 64s + 32h + 8j .. +8 (16 bytes). So one wave loads a
// fragment with one fully coalesced 1 KiB global_load_dwordx4, with no LDS staging; the weight
// tile the kernels decode into LDS uses the same order of the reduction values (chunk 4h + j of
// a 64-value row), so the products pair up.
//
// Rows past T up to the next multiple of 32 are zero (the producer writes them). The layout holds
// exactly the activation's bytes (plus that row padding).
#pragma once

#include <stdint.h>

#include "iqr_device.h"

namespace r97q {

// row blocks of the tiled copy of a T-row operand
R97Q_HD int64_t act_tile_blocks(int64_t T) { return (T + 31) >> 5; }

// element offset of activation value (m, k) in the tiled layout of a T-row operand
R97Q_HD int64_t act_tile_index(int64_t m, int64_t k, int64_t T) {
    const int64_t rb = m >> 5, i = m & 31, s = k >> 6;
    const int64_t kk = k & 63;
    const int64_t h = kk >> 5, j = (kk >> 3) & 3, e = kk & 7;
    return (((s * act_tile_blocks(T) + rb) * 4 + j) * 64 + 32 * h + i) * 8 + e;
}

// bytes of the tiled copy of a [T, R] bf16 operand
R97Q_HD int64_t act_tile_bytes(int64_t T, int64_t R) { return (T + 31) / 32 * 32 * R * 2; }

}  // namespace r97q
