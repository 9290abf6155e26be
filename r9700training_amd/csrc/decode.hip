// decode.hip -- the standalone IQR decode (canonical planes -> int8 grid + bf16 scale) and the
// one-time preparation of a weight for the fused kernels (canonical planes -> column streams +
// transposed effective scale), with their C-ABI entry points.
//
// The decode is the reference's r97_iqr_decode (src/iqr_decode.h:278-386): same rules, same
// values, bit for bit. It is not the reference's schedule: instead of one thread walking a whole
// 256-row run of one column, each thread decodes an 8-row chunk of a column and seeds its state
// from the ceil(L/b) codes above the chunk (wrapping inside the run, which is exactly the
// tail-biting seam), so a launch has rows/8 x cols independent threads and consecutive threads
// write consecutive columns. The common form (trellis.mad, L = 16, rb = 1, bits 3-6) runs on a
// kernel with its code width compiled in, alone or several row ranges a launch.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "iqr_device.h"
#include "status.h"

namespace r97q {

namespace {
thread_local std::string g_error;
}

void set_error(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
}

void clear_error() { g_error.clear(); }

const char* last_error() { return g_error.c_str(); }

// ---------------------------------------------------------------- the description's rules
// src/iqr_decode.h:321-349
int32_t validate(const R97IqrDecodeDesc& d) {
    if (!d.codes || !d.out_codes || !d.out_scale) return 1;
    if (d.rows <= 0 || d.row0 < 0 || d.rows_all <= 0 || d.rows > d.rows_all - d.row0) return 1;
    if (d.cols <= 0 || (d.cols & 127) != 0) return 1;
    if (d.run_rows <= 0 || d.rb <= 0 || d.run_rows % d.rb != 0) return 1;
    if (d.row0 % d.run_rows != 0) return 1;
    if (d.rows % d.run_rows != 0 && d.row0 + d.rows != d.rows_all) return 1;
    const int64_t bc = d.scale_block_cols > 0 ? d.scale_block_cols : d.cols;
    if (bc != 128 && bc != d.cols) return 1;
    if (d.affine) {
        if (!d.zero || d.bits < 1 || d.bits > 7 || d.zero_bits < 1 || d.zero_bits > 8) return 1;
        if (d.run_rows != 1 || d.rb != 1 || d.scale2) return 1;
        return 0;
    }
    if (d.bits < 1 || d.bits > 16 || d.state_bits < 1 || d.state_bits > 24) return 1;
    if (!d.mad && !d.lut) return 1;
    if (d.scale2 && (d.scale2_block_rows < 0 || d.scale2_block_cols < 0)) return 1;
    if (d.scale2 && d.scale2_block_cols > 0 && d.scale2_block_cols % 128 != 0) return 1;
    const int32_t c = (d.state_bits + d.bits - 1) / d.bits;
    for (int64_t r0 = d.row0; r0 < d.row0 + d.rows; r0 += d.run_rows) {
        int64_t r1 = r0 + d.run_rows;
        if (r1 > d.rows_all) r1 = d.rows_all;
        if (r1 - r0 < c) return 1;
    }
    return 0;
}

namespace {

// ---------------------------------------------------------------- the decode kernel
constexpr int kDecodeThreads = 256;

__device__ inline int32_t state_value(const R97IqrDecodeDesc& d, uint32_t st) {
    if (d.mad) return mad_value(st & 0xFFFFFFu, d.mad_a & 0xFFFFFFu, d.mad_b);
    return (int32_t)d.lut[st];
}

// src/iqr_decode.h:239-250
__device__ float block_max(const R97IqrDecodeDesc& d, int64_t r, int64_t kb) {
    const int64_t r0 = (r / d.rb) * d.rb;
    int64_t r1 = r0 + d.rb;
    if (r1 > d.rows_all) r1 = d.rows_all;
    float m = 0.0f;
    for (int64_t q = r0; q < r1; ++q) {
        const float v = block_scale(d, q, kb);
        m = v > m ? v : m;
    }
    return m;
}

// src/iqr_decode.h:253-256
__device__ inline int32_t rb_round(int32_t v, float ratio, int32_t mad) {
    if (mad) return (int32_t)(__builtin_fmaf((float)v, ratio, 12582912.0f) - 12582912.0f);
    return (int32_t)__builtin_rintf((float)v * ratio);
}

// Where the decode writes (rows counted from the description's row0). Canonical: out_codes
// [rows, cols] int8 row-major and out_scale [rows, cols/128] bf16 (the reference's grids). TILED:
// the int8-code form the fused kernels read (out_codes holds 32-byte units of 8 rows x 4 columns
// -- byte 16*(c>>1) + 2*i + (c&1) is row i, column c -- ordered [rows/8][cols/4]) and the scale
// transposed to [cols/128][ld] (ld >= rows).
template <bool TILED>
struct DecodeOut {
    __device__ static int64_t code(const R97IqrDecodeDesc& d, int64_t q, int64_t j) {
        q -= d.row0;
        if (!TILED) return q * d.cols + j;
        return ((q >> 3) * (d.cols >> 2) + (j >> 2)) * 32 + 16 * ((j >> 1) & 1) + 2 * (q & 7) + (j & 1);
    }
    __device__ static int64_t scale(const R97IqrDecodeDesc& d, int64_t q, int64_t kb, int64_t ld) {
        q -= d.row0;
        if (!TILED) return q * (d.cols >> 7) + kb;
        return kb * ld + q;
    }
};

// One thread: column j, rows [r, r_end) of the run [run_start, run_end).
template <bool TILED>
__global__ __launch_bounds__(kDecodeThreads) void decode_kernel(const R97IqrDecodeDesc d,
                                                                int64_t chunk_rows,
                                                                int64_t chunks, int64_t scale_ld) {
    using O = DecodeOut<TILED>;
    const int64_t j = (int64_t)blockIdx.x * kDecodeThreads + threadIdx.x;
    const int64_t ch = blockIdx.y + (int64_t)blockIdx.z * gridDim.y;
    if (j >= d.cols || ch >= chunks) return;
    const int64_t r = d.row0 + ch * chunk_rows;
    const int64_t run_start = (r / d.run_rows) * d.run_rows;
    int64_t run_end = run_start + d.run_rows;
    if (run_end > d.rows_all) run_end = d.rows_all;
    int64_t r_end = r + chunk_rows;
    if (r_end > run_end) r_end = run_end;
    if (r_end > d.row0 + d.rows) r_end = d.row0 + d.rows;
    const int64_t kb = j >> 7;
    const bool first = (j & 127) == 0;

    if (d.affine) {
        for (int64_t q = r; q < r_end; ++q) {
            const uint32_t code = load_bits(d.codes + (q - d.row0) * d.codes_row_bytes, d.bits, j);
            const int64_t bc = d.scale_block_cols > 0 ? d.scale_block_cols : d.cols;
            const int64_t gb = bc == d.cols ? 0 : (kb * 128) / bc;
            const uint32_t zero = load_bits(d.zero + (q - d.row0) * d.zero_row_bytes, d.zero_bits, gb);
            d.out_codes[O::code(d, q, j)] = (int8_t)((int32_t)code - (int32_t)zero);
            if (first) d.out_scale[O::scale(d, q, kb, scale_ld)] = f32_to_bf16(block_scale(d, q, kb));
        }
        return;
    }

    // The state before row r: the c codes above it, wrapping inside the run (the seam when r is
    // the run's first row, the plain shift register otherwise).
    const int32_t c = (d.state_bits + d.bits - 1) / d.bits;
    const uint32_t mask = (1u << d.state_bits) - 1u;
    const int64_t len = run_end - run_start;
    uint32_t st = 0;
    for (int32_t q = c; q >= 1; --q) {
        int64_t t = r - q;
        if (t < run_start) t += len;
        st = ((st << d.bits) | load_bits(d.codes + (t - d.row0) * d.codes_row_bytes, d.bits, j)) & mask;
    }
    // rb > 1: the block's shared scale is set at the block's first row; a chunk that starts inside
    // a block takes the block's value, which is what the serial walk carried there.
    float cur = 0.0f;
    if (d.rb > 1 && (r % d.rb) != 0) cur = block_max(d, (r / d.rb) * d.rb, kb);
    // the code row and the output byte advance by fixed steps down the chunk (a TILED chunk never
    // leaves its 8-row unit: it is 8 rows from a multiple of 8, or 1 row)
    const uint8_t* row = d.codes + (r - d.row0) * d.codes_row_bytes;
    int8_t* dst = d.out_codes + O::code(d, r, j);
    const int64_t dst_step = TILED ? 2 : d.cols;
    for (int64_t q = r; q < r_end; ++q, row += d.codes_row_bytes, dst += dst_step) {
        st = ((st << d.bits) | load_bits(row, d.bits, j)) & mask;
        const int32_t v = state_value(d, st);
        int32_t out = v;
        if (d.rb > 1) {
            if (q % d.rb == 0) cur = block_max(d, q, kb);
            const float sr = block_scale(d, q, kb);
            out = cur <= 0.0f ? 0 : rb_round(v, sr / cur, d.round_mad);
            if (first) d.out_scale[O::scale(d, q, kb, scale_ld)] = f32_to_bf16(cur);
        }
        *dst = (int8_t)out;
    }
    // rb == 1: the chunk's scales of the 128-column block, one row a lane of the block's first
    // lanes (a wave that ran the generic scale read for one lane on every row spent most of the
    // launch there)
    const int64_t i = j & 127;
    if (d.rb == 1 && i < r_end - r) {
        const int64_t q = r + i;
        d.out_scale[O::scale(d, q, kb, scale_ld)] = f32_to_bf16(block_scale(d, q, kb));
    }
}

// The common form -- trellis.mad, L = 16, rb = 1, bits 3..6 -- with the code width a compile-time
// constant. One thread: the 4 columns 4q..4q+3 (their codes are 4 BITS consecutive bits of a row:
// one or two dword loads and a funnel shift) over the ROWS rows of chunk ch (8: the chunks never
// straddle a run: the launch checks that runs, rows and row0 are whole chunks, and that code rows
// are 4-byte aligned; 16-row chunks measured slower, 13.3 against 10.0 µs, with half the threads);
// the state walk, the hash and the byte sum are a handful of VALU a value with no per-value form
// branches. TILED: each 8 x 4 codes of the thread are one 32-byte unit of the
// int8-code form, written as two 16-byte stores; canonical: one 4-byte store a row. The same values as
// decode_kernel, bit for bit.
template <int BITS, bool TILED, int ROWS>
__device__ __forceinline__ void mad_rows(const R97IqrDecodeDesc& d, int64_t ch, int64_t chunks, int64_t scale_ld) {
    using O = DecodeOut<TILED>;
    constexpr int C = (16 + BITS - 1) / BITS;  // codes above a chunk that seed its state
    const int64_t q4 = (int64_t)blockIdx.x * kDecodeThreads + threadIdx.x;
    if (ch >= chunks || 4 * q4 >= d.cols) return;
    const int64_t j = 4 * q4;  // the thread's first column
    const int64_t r = d.row0 + ch * ROWS;
    const int64_t run_start = (r / d.run_rows) * d.run_rows;
    int64_t run_end = run_start + d.run_rows;
    if (run_end > d.rows_all) run_end = d.rows_all;
    const int64_t len = run_end - run_start;
    const int64_t w = (j * BITS) >> 5;
    const int sh = (int)((j * BITS) & 31);
    const bool straddle = sh + 4 * BITS > 32;
    // the 4 codes of row q, column 4q4 + c at bits BITS c
    auto codes4 = [&](int64_t q) -> uint32_t {
        const uint32_t* row = reinterpret_cast<const uint32_t*>(d.codes + (q - d.row0) * d.codes_row_bytes);
        const uint32_t lo = row[w];
        const uint32_t hi = straddle ? row[w + 1] : 0u;
        return __builtin_amdgcn_alignbit(hi, lo, (uint32_t)sh);
    };
    constexpr uint32_t kMask = (1u << BITS) - 1u;
    uint32_t st[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int q = C; q >= 1; --q) {
        int64_t t = r - q;
        if (t < run_start) t += len;
        const uint32_t c4 = codes4(t);
#pragma unroll
        for (int c = 0; c < 4; ++c) st[c] = ((st[c] << BITS) | ((c4 >> (BITS * c)) & kMask)) & 0xFFFFu;
    }
    const uint32_t a24 = d.mad_a & 0xFFFFFFu;
#pragma unroll
    for (int u = 0; u < ROWS / 8; ++u) {
        const int64_t ru = r + 8 * u;
        uint32_t v[8][4];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t c4 = codes4(ru + i);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                st[c] = ((st[c] << BITS) | ((c4 >> (BITS * c)) & kMask)) & 0xFFFFu;
                v[i][c] = (uint32_t)mad_value(st[c], a24, d.mad_b) & 0xFFu;
            }
        }
        if constexpr (TILED) {
            // byte 16 (c >> 1) + 2 i + (c & 1) of the unit is row i, column c
            uint32_t o[8];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    o[4 * h + k] = v[2 * k][2 * h] | (v[2 * k][2 * h + 1] << 8) | (v[2 * k + 1][2 * h] << 16) |
                                   (v[2 * k + 1][2 * h + 1] << 24);
            uint4* dst = reinterpret_cast<uint4*>(d.out_codes + O::code(d, ru, j));
            dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
            dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                *reinterpret_cast<uint32_t*>(d.out_codes + O::code(d, ru + i, j)) =
                    v[i][0] | (v[i][1] << 8) | (v[i][2] << 16) | (v[i][3] << 24);
        }
    }
    // the chunk's scales of the thread's 128-column block: the block's first thread
    if ((j & 127) == 0) {
        const int64_t kb = j >> 7;
#pragma unroll
        for (int i = 0; i < ROWS; ++i)
            d.out_scale[O::scale(d, r + i, kb, scale_ld)] = f32_to_bf16(block_scale(d, r + i, kb));
    }
}

template <int BITS, bool TILED, int ROWS>
__global__ __launch_bounds__(kDecodeThreads) void decode_mad_kernel(const R97IqrDecodeDesc d, int64_t chunks,
                                                                    int64_t scale_ld) {
    mad_rows<BITS, TILED, ROWS>(d, blockIdx.y + (int64_t)blockIdx.z * gridDim.y, chunks, scale_ld);
}

// Several row ranges of the common form in one launch (blockIdx.z: the range), into the int8-code
// form: each range as decode_mad_kernel decodes it alone, the same bits.
constexpr int kDecodeBatch = 8;
struct DecodeBatch {
    R97IqrDecodeDesc d[kDecodeBatch];
};
template <int BITS>
__global__ __launch_bounds__(kDecodeThreads) void decode_mad_batch_kernel(const DecodeBatch b, int64_t scale_ld) {
    const R97IqrDecodeDesc& d = b.d[blockIdx.z];
    mad_rows<BITS, true, 8>(d, blockIdx.y, d.rows / 8, scale_ld);
}

// ---------------------------------------------------------------- preparation
// One workgroup per (segment g, 256 columns): the segment's 32 packed rows over those columns are
// staged in LDS (each row's bytes contiguous; every load of the workgroup issued before any LDS
// write, so the loads are in flight together), then each thread assembles its column's 32 codes
// into the `BITS` stream dwords (row 32g+i's code at bit BITS*(31-i)), written coalesced:
// consecutive columns are consecutive dwords. Rows whose stride and start are dword-aligned (every
// packed row of a multiple of 128 columns) are staged a dword a load, others a byte a load.
constexpr int kPrepCols = 256;
template <int BITS>
__global__ __launch_bounds__(kPrepCols) void prepare_stream_kernel(const R97IqrDecodeDesc d,
                                                                   uint32_t* __restrict__ stream) {
    constexpr int kSpan = kPrepCols * BITS / 8 + 1;  // a row's bytes over the block's columns (+ a straddle)
    constexpr int kRow = kSpan + 3;                  // LDS bytes a row: 32 BITS + 4, a whole number of dwords
    __shared__ __attribute__((aligned(4))) uint8_t rows[32][kRow];
    const int64_t c0 = (int64_t)blockIdx.x * kPrepCols;
    const int64_t g = blockIdx.y;
    const int64_t byte0 = c0 * BITS / 8;  // c0 is a multiple of 256: the block starts on a dword
    const int64_t avail = d.codes_row_bytes - byte0;
    const int span = (int)(avail < kSpan ? avail : kSpan);
    if (d.codes_row_bytes % 4 == 0 && reinterpret_cast<uintptr_t>(d.codes) % 4 == 0) {
        // a row's dwords: ceil(span / 4), within the row (avail is a multiple of 4; a full block's
        // last dword reaches 3 bytes into the next block's)
        const int sd = (span + 3) / 4;
        constexpr int kLoads = (32 * (kRow / 4) + kPrepCols - 1) / kPrepCols;
        uint32_t v[kLoads];
#pragma unroll
        for (int u = 0; u < kLoads; ++u) {
            const int idx = (int)threadIdx.x + kPrepCols * u, i = idx / sd, q = idx - i * sd;
            v[u] = idx < 32 * sd ? *reinterpret_cast<const uint32_t*>(d.codes + (g * 32 + i) * d.codes_row_bytes + byte0 +
                                                                      4 * q)
                                 : 0u;
        }
#pragma unroll
        for (int u = 0; u < kLoads; ++u) {
            const int idx = (int)threadIdx.x + kPrepCols * u, i = idx / sd, q = idx - i * sd;
            if (idx < 32 * sd) *reinterpret_cast<uint32_t*>(&rows[i][4 * q]) = v[u];
        }
    } else {
        for (int idx = threadIdx.x; idx < 32 * span; idx += kPrepCols) {
            const int i = idx / span, b = idx - i * span;
            rows[i][b] = d.codes[(g * 32 + i) * d.codes_row_bytes + byte0 + b];
        }
    }
    __syncthreads();
    const int64_t col = c0 + threadIdx.x;
    if (col >= d.cols) return;
    const int o = (int)threadIdx.x * BITS;  // the column's bit offset in the staged rows
    const int byte = o >> 3, sh = o & 7;
    uint32_t w[BITS];
#pragma unroll
    for (int q = 0; q < BITS; ++q) w[q] = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        // a code spans at most two bytes (sh + BITS <= 13); the second is read only when it holds bits
        uint32_t v = rows[i][byte];
        if (sh + BITS > 8) v |= (uint32_t)rows[i][byte + 1] << 8;
        const uint32_t code = (v >> sh) & ((1u << BITS) - 1u);
        const int pos = BITS * (31 - i);
        const int wi = pos >> 5, bs = pos & 31;
        w[wi] |= code << bs;
        if (bs + BITS > 32) w[wi + 1] |= code >> (32 - bs);
    }
#pragma unroll
    for (int q = 0; q < BITS; ++q) stream[stream_index(g, BITS, q, d.cols, col)] = w[q];
}

// One thread per 32-byte unit (8 rows x 4 columns) of a decoded int8 grid [rows, cols]: the unit in
// the fused kernels' int8-code form (the TILED layout of decode_kernel).
__global__ __launch_bounds__(256) void tile_codes_kernel(const int8_t* __restrict__ codes, int64_t rows,
                                                         int64_t cols, int8_t* __restrict__ tiled) {
    const int64_t k4 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t n8 = blockIdx.y;
    if (k4 >= cols / 4) return;
    uint32_t row[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) row[i] = *reinterpret_cast<const uint32_t*>(codes + (n8 * 8 + i) * cols + 4 * k4);
    // byte b of the unit: column 2*(b>>4) + (b&1), row (b&15)>>1
    uint32_t out[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        uint32_t v = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int b = 4 * q + t;
            const int c = 2 * (b >> 4) + (b & 1), i = (b & 15) >> 1;
            v |= ((row[i] >> (8 * c)) & 0xFFu) << (8 * t);
        }
        out[q] = v;
    }
    uint4* dst = reinterpret_cast<uint4*>(tiled + (n8 * (cols / 4) + k4) * 32);
    dst[0] = make_uint4(out[0], out[1], out[2], out[3]);
    dst[1] = make_uint4(out[4], out[5], out[6], out[7]);
}

// [rows, nkb] bf16 -> [nkb, rows]
__global__ __launch_bounds__(256) void transpose_scale_kernel(const uint16_t* __restrict__ scale, int64_t rows,
                                                              int64_t nkb, uint16_t* __restrict__ scale_t) {
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t kb = blockIdx.y;
    if (n < rows) scale_t[kb * rows + n] = scale[n * nkb + kb];
}

// One thread per (row, 128-column block): the effective bf16 scale, transposed to [cols/128][rows].
__global__ __launch_bounds__(256) void prepare_scale_kernel(const R97IqrDecodeDesc d,
                                                            const float* __restrict__ scale_col,
                                                            uint16_t* __restrict__ scale_t) {
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t kb = blockIdx.y;
    if (n >= d.rows_all) return;
    uint16_t s;
    if (scale_col) {
        // src/iqr_form.h:203-216: one f32 a row times one f32 a block, rounded once
        const float row = __builtin_bit_cast(float, ((const uint32_t*)(d.scale + n * d.scale_row_bytes))[0]);
        s = f32_to_bf16(row * scale_col[kb]);
    } else {
        s = f32_to_bf16(block_scale(d, n, kb));
    }
    scale_t[kb * d.rows_all + n] = s;
}

}  // namespace

// the common form on whole 8-row chunks and aligned rows: decode_mad_kernel
template <bool TILED>
bool mad_fast(const R97IqrDecodeDesc& d) {
    return !d.affine && d.mad && d.rb == 1 && d.state_bits == 16 && d.bits >= 3 && d.bits <= 6 &&
           d.run_rows % 8 == 0 && d.row0 % 8 == 0 && d.rows % 8 == 0 && d.codes_row_bytes % 4 == 0 &&
           (reinterpret_cast<uintptr_t>(d.codes) & 3) == 0 &&
           (reinterpret_cast<uintptr_t>(d.out_codes) & (TILED ? 15 : 3)) == 0;
}

template <bool TILED>
void launch_decode(const R97IqrDecodeDesc& d, hipStream_t s, int64_t scale_ld = 0) {
    if (mad_fast<TILED>(d)) {
        const int64_t chunks = d.rows / 8;
        const int64_t gy = chunks < 65535 ? chunks : 65535;
        const int64_t gz = (chunks + gy - 1) / gy;
        const dim3 grid((unsigned)((d.cols / 4 + kDecodeThreads - 1) / kDecodeThreads), (unsigned)gy, (unsigned)gz);
        const dim3 block(kDecodeThreads);
        switch (d.bits) {
            case 3: hipLaunchKernelGGL((decode_mad_kernel<3, TILED, 8>), grid, block, 0, s, d, chunks, scale_ld); break;
            case 4: hipLaunchKernelGGL((decode_mad_kernel<4, TILED, 8>), grid, block, 0, s, d, chunks, scale_ld); break;
            case 5: hipLaunchKernelGGL((decode_mad_kernel<5, TILED, 8>), grid, block, 0, s, d, chunks, scale_ld); break;
            default: hipLaunchKernelGGL((decode_mad_kernel<6, TILED, 8>), grid, block, 0, s, d, chunks, scale_ld); break;
        }
        return;
    }
    const int64_t chunk_rows = (d.run_rows % 8 == 0) ? 8 : 1;
    // chunks never straddle a run: runs start at multiples of run_rows and chunk_rows divides it
    const int64_t chunks = (d.rows + chunk_rows - 1) / chunk_rows;
    const int64_t gy = chunks < 65535 ? chunks : 65535;
    const int64_t gz = (chunks + gy - 1) / gy;
    dim3 grid((unsigned)((d.cols + kDecodeThreads - 1) / kDecodeThreads), (unsigned)gy, (unsigned)gz);
    hipLaunchKernelGGL(decode_kernel<TILED>, grid, dim3(kDecodeThreads), 0, s, d, chunk_rows, chunks, scale_ld);
}

// The rows [row0, row0 + rows) of a valid description, decoded into the int8-code form at
// d.out_codes / d.out_scale (row row0 first; the scale with leading dimension scale_ld).
int decode_tiled(const R97IqrDecodeDesc& d, int64_t scale_ld, hipStream_t s) {
    launch_decode<true>(d, s, scale_ld);
    return launch_status("decode_kernel (int8-code form)");
}

// n valid descriptions (the same scale_ld), each decoded as decode_tiled decodes it: one launch when
// all n are the common form with the same code width and columns, else one a description
int decode_tiled_batch(const R97IqrDecodeDesc* ds, int n, int64_t scale_ld, hipStream_t s) {
    bool one = n >= 1 && n <= kDecodeBatch;
    int64_t chunks = 0;
    for (int i = 0; one && i < n; ++i) {
        one = mad_fast<true>(ds[i]) && ds[i].bits == ds[0].bits && ds[i].cols == ds[0].cols &&
              ds[i].rows / 8 <= 65535;
        chunks = ds[i].rows / 8 > chunks ? ds[i].rows / 8 : chunks;
    }
    if (!one || chunks == 0) {
        for (int i = 0; i < n; ++i)
            if (int e = decode_tiled(ds[i], scale_ld, s)) return e;
        return R97Q_OK;
    }
    DecodeBatch b{};
    for (int i = 0; i < n; ++i) b.d[i] = ds[i];
    const dim3 grid((unsigned)((ds[0].cols / 4 + kDecodeThreads - 1) / kDecodeThreads), (unsigned)chunks, (unsigned)n);
    const dim3 block(kDecodeThreads);
    switch (ds[0].bits) {
        case 3: hipLaunchKernelGGL(decode_mad_batch_kernel<3>, grid, block, 0, s, b, scale_ld); break;
        case 4: hipLaunchKernelGGL(decode_mad_batch_kernel<4>, grid, block, 0, s, b, scale_ld); break;
        case 5: hipLaunchKernelGGL(decode_mad_batch_kernel<5>, grid, block, 0, s, b, scale_ld); break;
        default: hipLaunchKernelGGL(decode_mad_batch_kernel<6>, grid, block, 0, s, b, scale_ld); break;
    }
    return launch_status("decode_mad_batch_kernel (int8-code form)");
}

// Whether `d` is a form the fused kernels serve; the reason goes to the error message.
bool fused_form(const R97IqrDecodeDesc& d, const float* scale_col) {
    if (d.affine) {
        set_error("fused path: the affine grid has no trellis (decode it with r97_iqr_decode)");
        return false;
    }
    if (!d.mad) {
        set_error("fused path: a stored-LUT codebook is not served (trellis.mad only)");
        return false;
    }
    if (d.rb != 1) {
        set_error("fused path: rb = %d row blocks are not served (rb = 1 only)", (int)d.rb);
        return false;
    }
    if (d.state_bits != 16 || d.bits < 3 || d.bits > 6) {
        set_error("fused path: bits %d state_bits %d not served (bits 3..6, L = 16)", (int)d.bits,
                  (int)d.state_bits);
        return false;
    }
    if (d.rows_all % 32 != 0 || d.run_rows % 32 != 0 || d.cols % 128 != 0) {
        set_error("fused path: rows %lld / run %d must be multiples of 32, cols %lld of 128",
                  (long long)d.rows_all, (int)d.run_rows, (long long)d.cols);
        return false;
    }
    if (scale_col && (d.scale_dtype != R97_IQR_F32 || d.scale_block_cols > 0)) {
        set_error("fused path: scale.col needs one f32 scale a row (src/iqr_form.h:209)");
        return false;
    }
    return true;
}

// Whether `d` (valid) can take the int8-code form: every form the decode reads, with whole 8-row
// units and 128-column blocks.
bool codes8_form(const R97IqrDecodeDesc& d, const float* scale_col) {
    if (d.rows_all % 8 != 0 || d.cols % 128 != 0) {
        set_error("int8-code form: rows %lld must be a multiple of 8, cols %lld of 128", (long long)d.rows_all,
                  (long long)d.cols);
        return false;
    }
    if (scale_col && (d.scale_dtype != R97_IQR_F32 || d.scale_block_cols > 0)) {
        set_error("int8-code form: scale.col needs one f32 scale a row (src/iqr_form.h:209)");
        return false;
    }
    return true;
}

}  // namespace r97q

using namespace r97q;

extern "C" {

const char* r97q_last_error(void) { return r97q::last_error(); }

int r97q_iqr_validate(const R97IqrDecodeDesc* desc) { return desc ? r97q::validate(*desc) : 1; }

int r97_iqr_decode(const R97IqrDecodeDesc* desc, R97IqrStream stream) {
    clear_error();
    if (!desc || validate(*desc)) {
        set_error("r97_iqr_decode: the description is outside the decode's rules");
        return 1;
    }
    const R97IqrDecodeDesc& d = *desc;
    launch_decode<false>(d, (hipStream_t)stream);
    return launch_status("r97_iqr_decode") == R97Q_OK ? 0 : 1;
}

int64_t r97q_weight_stream_bytes(const R97IqrDecodeDesc* desc) {
    clear_error();
    if (!desc) {
        set_error("r97q_weight_stream_bytes: null description");
        return -1;
    }
    if (fused_form(*desc, nullptr)) return desc->rows_all / 32 * desc->bits * desc->cols * 4;
    // the other forms: the int8-code form (the description's own rules still apply)
    R97IqrDecodeDesc d = *desc;
    int8_t probe_codes = 0;
    uint16_t probe_scale = 0;
    d.out_codes = &probe_codes;
    d.out_scale = &probe_scale;
    if (validate(d)) {
        set_error("r97q_weight_stream_bytes: the description is outside the decode's rules");
        return -1;
    }
    if (!codes8_form(d, nullptr)) return -1;
    clear_error();
    return d.rows_all * d.cols;
}

int r97q_weight_prepare(const R97IqrDecodeDesc* desc, const float* scale_col,
                        uint32_t* stream_out, uint16_t* scale_t_out, R97qWeight* w,
                        R97IqrStream stream) {
    clear_error();
    if (!desc || !stream_out || !scale_t_out || !w) {
        set_error("r97q_weight_prepare: null argument");
        return R97Q_EINVAL;
    }
    R97IqrDecodeDesc d = *desc;
    if (d.row0 != 0 || d.rows != d.rows_all) {
        set_error("r97q_weight_prepare: the whole weight is prepared at once (row0 0, rows = rows_all)");
        return R97Q_EINVAL;
    }
    // the rules need output pointers; preparation writes its own planes instead
    d.out_codes = reinterpret_cast<int8_t*>(stream_out);
    d.out_scale = scale_t_out;
    if (validate(d)) {
        set_error("r97q_weight_prepare: the description is outside the decode's rules");
        return R97Q_EINVAL;
    }
    if (!fused_form(d, scale_col)) {
        // every other form the decode reads: decoded once into the int8-code form
        clear_error();
        return r97q_weight_prepare_codes8(desc, scale_col, reinterpret_cast<int8_t*>(stream_out), scale_t_out, w,
                                          stream);
    }
    const hipStream_t s = (hipStream_t)stream;
    const dim3 pgrid((unsigned)((d.cols + kPrepCols - 1) / kPrepCols), (unsigned)(d.rows_all / 32));
    switch (d.bits) {
        case 3: hipLaunchKernelGGL(prepare_stream_kernel<3>, pgrid, dim3(kPrepCols), 0, s, d, stream_out); break;
        case 4: hipLaunchKernelGGL(prepare_stream_kernel<4>, pgrid, dim3(kPrepCols), 0, s, d, stream_out); break;
        case 5: hipLaunchKernelGGL(prepare_stream_kernel<5>, pgrid, dim3(kPrepCols), 0, s, d, stream_out); break;
        default: hipLaunchKernelGGL(prepare_stream_kernel<6>, pgrid, dim3(kPrepCols), 0, s, d, stream_out); break;
    }
    if (int e = launch_status("prepare_stream_kernel")) return e;
    hipLaunchKernelGGL(prepare_scale_kernel,
                       dim3((unsigned)((d.rows_all + 255) / 256), (unsigned)(d.cols / 128)),
                       dim3(256), 0, s, d, scale_col, scale_t_out);
    if (int e = launch_status("prepare_scale_kernel")) return e;
    R97qWeight out{};
    out.rows = d.rows_all;
    out.cols = d.cols;
    out.bits = d.bits;
    out.state_bits = d.state_bits;
    out.run_rows = d.run_rows;
    out.mad = d.mad;
    out.mad_a = d.mad_a;
    out.mad_b = d.mad_b;
    out.lut = d.lut;
    out.stream = stream_out;
    out.scale_t = scale_t_out;
    *w = out;
    return R97Q_OK;
}

}  // extern "C"

extern "C" {

int r97q_weight_prepare_codes8(const R97IqrDecodeDesc* desc, const float* scale_col, int8_t* codes_out,
                               uint16_t* scale_t_out, R97qWeight* w, R97IqrStream stream) {
    clear_error();
    const char* who = "r97q_weight_prepare_codes8";
    if (!desc || !codes_out || !scale_t_out || !w) {
        set_error("%s: null argument", who);
        return R97Q_EINVAL;
    }
    R97IqrDecodeDesc d = *desc;
    if (d.row0 != 0 || d.rows != d.rows_all) {
        set_error("%s: the whole weight is prepared at once (row0 0, rows = rows_all)", who);
        return R97Q_EINVAL;
    }
    d.out_codes = codes_out;
    d.out_scale = scale_t_out;
    if (validate(d)) {
        set_error("%s: the description is outside the decode's rules", who);
        return R97Q_EINVAL;
    }
    if (!codes8_form(d, scale_col)) return R97Q_EUNSUPPORTED;
    const hipStream_t s = (hipStream_t)stream;
    // the decode writes the codes in the tiled form and the scale transposed
    launch_decode<true>(d, s, d.rows_all);
    if (int e = launch_status("decode_kernel (int8-code form)")) return e;
    if (scale_col) {
        // src/iqr_form.h:203-216: the scale.col fold replaces the decoded scale
        hipLaunchKernelGGL(prepare_scale_kernel,
                           dim3((unsigned)((d.rows_all + 255) / 256), (unsigned)(d.cols / 128)), dim3(256), 0, s, d,
                           scale_col, scale_t_out);
        if (int e = launch_status("prepare_scale_kernel")) return e;
    }
    R97qWeight out{};
    out.rows = d.rows_all;
    out.cols = d.cols;
    out.bits = R97Q_CODES8;
    out.stream = reinterpret_cast<const uint32_t*>(codes_out);
    out.scale_t = scale_t_out;
    *w = out;
    return R97Q_OK;
}

int r97q_weight_from_decoded(const int8_t* codes, const uint16_t* scale, int64_t rows, int64_t cols,
                             int8_t* codes_out, uint16_t* scale_t_out, R97qWeight* w, R97IqrStream stream) {
    clear_error();
    const char* who = "r97q_weight_from_decoded";
    if (!codes || !scale || !codes_out || !scale_t_out || !w) {
        set_error("%s: null argument", who);
        return R97Q_EINVAL;
    }
    if (rows <= 0 || cols <= 0 || rows % 8 != 0 || cols % 128 != 0) {
        set_error("%s: rows %lld must be a positive multiple of 8, cols %lld of 128", who, (long long)rows,
                  (long long)cols);
        return R97Q_EINVAL;
    }
    const hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(tile_codes_kernel, dim3((unsigned)((cols / 4 + 255) / 256), (unsigned)(rows / 8)), dim3(256),
                       0, s, codes, rows, cols, codes_out);
    if (int e = launch_status("tile_codes_kernel")) return e;
    hipLaunchKernelGGL(transpose_scale_kernel, dim3((unsigned)((rows + 255) / 256), (unsigned)(cols / 128)),
                       dim3(256), 0, s, scale, rows, cols / 128, scale_t_out);
    if (int e = launch_status("transpose_scale_kernel")) return e;
    R97qWeight out{};
    out.rows = rows;
    out.cols = cols;
    out.bits = R97Q_CODES8;
    out.stream = reinterpret_cast<const uint32_t*>(codes_out);
    out.scale_t = scale_t_out;
    *w = out;
    return R97Q_OK;
}

}  // extern "C"
