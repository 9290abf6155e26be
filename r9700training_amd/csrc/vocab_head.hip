// vocab_head.hip -- the vocabulary head's transposed product on gfx950 (the reference's
// src/vocab_head.h:27-99 contract, its kernels src/adjoint/device/vocab_head.hip:82-238):
//
//   d_x[rows, n_embd] += H . sum over classes c of (dy[:, ids_c] . W_c) * scale.col_c
//
// The reference runs it as a gather, a per-token-row GEMV over the decoded int8 grid with f32
// fmas, and the un-rotation. Here it is the fused dX kernel's product. A class's rows go in ranges
// of about 4096 (whole trellis runs), a batch of up to kBatch ranges at a time: the batch's ranges
// are decoded into the int8-code form in the workspace (the standalone decode's kernel writing
// tiled, one launch for the batch when the form allows), and one batched
// qlinear_dx_kernel<R97Q_CODES8> launch (a grid slice a range, so a head with few
// token rows or a narrow n_embd still fills the chip) writes each range's (gathered . W) *
// scale.col -- the class's scale.col in its epilogue, one factor a 128-column tile -- into its own
// f32 partial; the partials are then added into d_x in range order (deterministic). Ranges are
// padded to Np (a multiple of 128) rows with zero codes, zero scales and zero cotangent columns.
// The products' operands -- the cotangent's columns of every class's rows, bf16 [range][rows][Np] a
// class -- are gathered first, for all classes in one launch whose token rows vary slowest, so the
// workgroups in flight cover a few token rows of every class and each cotangent line is fetched
// from memory about once (the classes split the vocabulary at random: a class on its own touches
// almost every line). Token rows go in blocks of at most kRowBlock, each block's operands held at
// once. Once every class is in, the unnormalised 128-wide Hadamard runs over each 128 columns of
// d_x.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/r97q.h"
#include "iqr_device.h"
#include "qlinear_fused.h"
#include "status.h"

namespace r97q {
namespace {

constexpr int64_t kRangeRows = 4096;  // rows of a range (whole trellis runs)
constexpr int kBatch = 8;             // ranges a batched launch
constexpr int kFillWorkgroups = 512;  // a batch large enough for this many workgroups (256 CUs)
constexpr int64_t kRowBlock = 4096;   // token rows a pass (every class's gathered operands held for them)

int64_t round_up(int64_t n, int64_t m) { return (n + m - 1) / m * m; }
int64_t row_block(int64_t rows) { return rows < kRowBlock ? rows : kRowBlock; }

// the rows one range takes: whole runs (the decode's rule for a row range), about kRangeRows
int64_t range_rows(const R97qVocabClass& c) {
    const int64_t run = c.decode.affine ? 1 : (c.decode.run_rows > 0 ? c.decode.run_rows : 1);
    int64_t r = kRangeRows / run * run;
    if (r < run) r = run;
    return r < c.rows ? r : c.rows;
}

int64_t ranges_of(const R97qVocabClass& c) {
    const int64_t R = range_rows(c);
    return (c.rows + R - 1) / R;
}

// ranges a batch takes: enough for kFillWorkgroups workgroups, at most kBatch
int batch_of(int64_t rows, int64_t K) {
    const int64_t wgs = (rows + kBM - 1) / kBM * (K / kBN);
    const int64_t b = (kFillWorkgroups + wgs - 1) / wgs;
    return (int)(b < 1 ? 1 : b > kBatch ? kBatch : b);
}

struct VocabWs {
    int64_t codes, scale, gather, part, part_lo, cf, total;
};

VocabWs vocab_ws(const R97qVocabPlan& plan, int64_t rows) {
    int64_t Np = 0;
    for (int c = 0; c < plan.classes; ++c) {
        const int64_t s = round_up(range_rows(plan.cls[c]), 128);
        Np = s > Np ? s : Np;
    }
    const int64_t K = plan.n_embd, nkb = K / 128, rb = row_block(rows), Z = batch_of(rb, K);
    int64_t nranges = 0;
    for (int c = 0; c < plan.classes; ++c) nranges += ranges_of(plan.cls[c]);
    VocabWs w{};
    int64_t off = 0;
    auto take = [&](int64_t bytes) {
        const int64_t at = off;
        off += round_up(bytes, 256);
        return at;
    };
    w.codes = take(Z * Np * K);
    w.scale = take(Z * nkb * Np * 2);
    w.gather = take(nranges * rb * Np * 2);
    w.part = take(Z * rb * K * 4);
    w.part_lo = take(Z * rb * K * 4);
    w.cf = take(nkb * 4);
    w.total = off;
    return w;
}

// the padding rows [ns, ns_pad) of a range: zero codes (from the unit row that holds row ns on) and
// zero scales
__global__ __launch_bounds__(256) void vocab_pad_kernel(int8_t* __restrict__ codes, uint16_t* __restrict__ scale_t,
                                                        int64_t ns, int64_t ns_pad, int64_t K) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t c0 = (ns / 8) * (K / 4) * 32 / 4, c1 = ns_pad * K / 4;  // in dwords
    if (c0 + i < c1) reinterpret_cast<uint32_t*>(codes)[c0 + i] = 0u;
    const int64_t pad = ns_pad - ns, nkb = K / 128;
    if (i < pad * nkb) scale_t[(i / pad) * ns_pad + ns + i % pad] = 0;
}

// The gathered operands of one block of token rows: class c's range z is a[z][m][n] =
// dy[m, ids[z*R + n] - vocab_offset] for a class row z*R + n < rows and an id inside this
// vocabulary, else 0 (the range's padding columns up to Np included).
struct GatherClass {
    const int32_t* ids;
    int64_t rows, R;  // the class's rows; rows a range
    uint16_t* out;    // [ranges][rb][Np]
    int y0;           // the class's first range in the launch's grid
};
struct GatherAll {
    GatherClass cls[4];
    int classes, ny;   // ny: every class's ranges
    int64_t rb, vocab, vocab_offset, Np, nx, ngroups;  // nx: Np / 256; ngroups: token-row groups
};
// A workgroup: 256 columns of one range x a group of kGatherRows token rows; a column and
// kGatherRows token rows a thread (the id read once for them; measured: 8 columns a thread with one
// 16-byte store is 40% slower -- fewer loads in flight). The workgroups are dealt so that XCD x
// takes the token-row groups x, x + 8, .. whole, one after another, each for every class and range:
// a cotangent line is then fetched into one XCD's L2 while its few token rows are gathered, not
// into all eight (the hardware deals workgroup ids round-robin over the XCDs, in id order on each).
constexpr int kGatherRows = 8;
__global__ __launch_bounds__(256) void vocab_gather_kernel(const uint16_t* __restrict__ dy, const GatherAll g) {
    const int64_t xcd = blockIdx.x & 7, l = blockIdx.x >> 3;
    const int64_t per = g.nx * g.ny;  // workgroups a token-row group
    const int64_t grp = (l / per) * 8 + xcd;
    if (grp >= g.ngroups) return;
    const int y = (int)((l % per) / g.nx);
    int c = 0;
    while (c + 1 < g.classes && y >= g.cls[c + 1].y0) ++c;
    const GatherClass& k = g.cls[c];
    const int64_t z = y - k.y0;
    const int64_t n = (l % per % g.nx) * 256 + threadIdx.x;
    const int64_t mb = grp * kGatherRows;
    if (n >= g.Np) return;
    const int64_t r = z * k.R + n;
    int64_t col = -1;
    if (n < k.R && r < k.rows) {
        const int64_t id = k.ids[r];
        if (id >= g.vocab_offset && id < g.vocab_offset + g.vocab) col = id - g.vocab_offset;
    }
#pragma unroll
    for (int i = 0; i < kGatherRows; ++i) {
        const int64_t m = mb + i;
        if (m >= g.rb) break;
        k.out[(z * g.rb + m) * g.Np + n] = col >= 0 ? dy[m * g.vocab + col] : (uint16_t)0;
    }
}

// d_x[i] += (hi[0][i] + lo[0][i]) + (hi[1][i] + lo[1][i]) + ... (the ranges in order; a range's
// product over the weights' high halves plus its product over their low halves)
__global__ __launch_bounds__(256) void vocab_reduce_kernel(float* __restrict__ d_x, const float* __restrict__ hi,
                                                           const float* __restrict__ lo, int64_t n, int Z) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float v = d_x[i];
    for (int z = 0; z < Z; ++z) v += hi[z * n + i] + lo[z * n + i];
    d_x[i] = v;
}

__global__ __launch_bounds__(64) void vocab_cf_kernel(const uint8_t* __restrict__ cf, int32_t dtype, int64_t nkb,
                                                      float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (i < nkb) out[i] = load_scalar(cf, dtype, i);
}

// The unnormalised Hadamard of one 128-column block of one row, in place: the seven butterfly
// stages (pairs j, j + h for h = 1, 2, .., 64; sum in j, difference in j + h) -- the natural-order
// Sylvester matrix, as src/adjoint/device/vocab_head.hip:145-163 applies it.
__global__ __launch_bounds__(128) void vocab_unrotate_kernel(float* __restrict__ d_x, int64_t K) {
    __shared__ float v[128];
    const int t = threadIdx.x;
    float* p = d_x + (int64_t)blockIdx.x * K + (int64_t)blockIdx.y * 128;
    v[t] = p[t];
    __syncthreads();
    for (int h = 1; h < 128; h <<= 1) {
        if (t < 64) {
            const int j = (t / h) * 2 * h + t % h;
            const float a = v[j], b = v[j + h];
            v[j] = a + b;
            v[j + h] = a - b;
        }
        __syncthreads();
    }
    p[t] = v[t];
}

__global__ __launch_bounds__(256) void vocab_cast_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst,
                                                         int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = f32_to_bf16(src[i]);
}

unsigned blocks(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

// the reference's rules for the plan and the buffers (src/adjoint/device/vocab_head.hip:170-211)
bool plan_ok(const R97qVocabPlan* plan, int64_t rows, const char* who) {
    if (!plan || rows <= 0 || plan->classes <= 0 || plan->classes > 4 || plan->n_embd <= 0 ||
        plan->n_embd % 128 != 0 || plan->vocab <= 0 || plan->vocab_offset < 0 ||
        (plan->transform != 0 && plan->transform != 128)) {
        set_error("%s: the plan or the buffers are outside the kernel's rules", who);
        return false;
    }
    for (int c = 0; c < plan->classes; ++c) {
        const R97qVocabClass& k = plan->cls[c];
        if (k.rows <= 0 || !k.ids || !k.scale_col || k.decode.rows_all != k.rows || k.decode.cols != plan->n_embd) {
            set_error("%s: the plan's class %d is incomplete", who, c);
            return false;
        }
    }
    return true;
}

}  // namespace
}  // namespace r97q

using namespace r97q;

extern "C" {

int64_t r97q_vocab_head_workspace_bytes(const R97qVocabPlan* plan, int64_t rows) {
    clear_error();
    if (!plan_ok(plan, rows, "r97q_vocab_head_workspace_bytes")) return -1;
    return vocab_ws(*plan, rows).total;
}

int r97q_vocab_head_transpose(const R97qVocabPlan* plan, const uint16_t* dy, int64_t rows, float* d_x,
                              void* workspace, int64_t workspace_bytes, R97IqrStream stream) {
    clear_error();
    const char* who = "r97q_vocab_head_transpose";
    if (!dy || !d_x) {
        set_error("%s: the plan or the buffers are outside the kernel's rules", who);
        return R97Q_EINVAL;
    }
    if (!plan_ok(plan, rows, who)) return R97Q_EINVAL;
    const VocabWs ws = vocab_ws(*plan, rows);
    if (!workspace || workspace_bytes < ws.total) {
        set_error("%s: workspace %lld bytes, needs %lld", who, (long long)workspace_bytes, (long long)ws.total);
        return R97Q_EWORKSPACE;
    }
    uint8_t* wsb = static_cast<uint8_t*>(workspace);
    int8_t* codes = reinterpret_cast<int8_t*>(wsb + ws.codes);
    uint16_t* scale_t = reinterpret_cast<uint16_t*>(wsb + ws.scale);
    uint16_t* gathered = reinterpret_cast<uint16_t*>(wsb + ws.gather);
    float* part = reinterpret_cast<float*>(wsb + ws.part);
    float* part_lo = reinterpret_cast<float*>(wsb + ws.part_lo);
    float* cf = reinterpret_cast<float*>(wsb + ws.cf);
    const hipStream_t s = (hipStream_t)stream;
    const int64_t K = plan->n_embd, nkb = K / 128;

    const int64_t rbmax = row_block(rows);
    const int Zmax = batch_of(rbmax, K);  // the partials' workspace holds this many ranges
    for (int64_t m0 = 0; m0 < rows; m0 += rbmax) {
        const int64_t rb = rows - m0 < rbmax ? rows - m0 : rbmax;
        // every class's gathered operands for token rows [m0, m0 + rb)
        int64_t Np = 0;
        for (int c = 0; c < plan->classes; ++c) {
            const int64_t np = round_up(range_rows(plan->cls[c]), 128);
            Np = np > Np ? np : Np;
        }
        GatherAll g{};
        g.classes = plan->classes;
        g.rb = rb;
        g.vocab = plan->vocab;
        g.vocab_offset = plan->vocab_offset;
        g.Np = Np;
        int ny = 0;
        int64_t goff = 0;
        for (int c = 0; c < plan->classes; ++c) {
            const R97qVocabClass& cls = plan->cls[c];
            const int64_t nr = ranges_of(cls);
            g.cls[c] = GatherClass{static_cast<const int32_t*>(cls.ids), cls.rows, range_rows(cls), gathered + goff, ny};
            ny += (int)nr;
            goff += nr * rb * Np;
        }
        g.ny = ny;
        g.nx = blocks(Np, 256);
        g.ngroups = blocks(rb, kGatherRows);
        const int64_t nwg = (g.ngroups + 7) / 8 * 8 * g.nx * ny;  // every XCD's share whole
        if (nwg > INT32_MAX) {
            set_error("%s: %d ranges of %lld rows are more than a launch's grid takes", who, ny, (long long)kRangeRows);
            return R97Q_EUNSUPPORTED;
        }
        hipLaunchKernelGGL(vocab_gather_kernel, dim3((unsigned)nwg), dim3(256), 0, s, dy + m0 * plan->vocab, g);
        if (int e = launch_status("vocab_gather_kernel")) return e;

        for (int c = 0; c < plan->classes; ++c) {
            const R97qVocabClass& cls = plan->cls[c];
            hipLaunchKernelGGL(vocab_cf_kernel, dim3(blocks(nkb, 64)), dim3(64), 0, s,
                               static_cast<const uint8_t*>(cls.scale_col), cls.scale_col_dtype, nkb, cf);
            if (int e = launch_status("vocab_cf_kernel")) return e;
            const int64_t R = range_rows(cls);
            for (int64_t b0 = 0; b0 < cls.rows; b0 += Zmax * R) {
                const int64_t nb = Zmax * R < cls.rows - b0 ? Zmax * R : cls.rows - b0;  // the batch's class rows
                const int Z = (int)((nb + R - 1) / R);
                R97IqrDecodeDesc dz[kBatch];
                for (int z = 0; z < Z; ++z) {
                    const int64_t r0 = b0 + z * R;
                    const int64_t ns = R < cls.rows - r0 ? R : cls.rows - r0;
                    int8_t* zc = codes + z * Np * K;
                    uint16_t* zs = scale_t + z * nkb * Np;
                    R97IqrDecodeDesc d = cls.decode;
                    d.row0 = r0;
                    d.rows = ns;
                    d.codes = d.codes + r0 * d.codes_row_bytes;
                    d.scale = d.scale + r0 * d.scale_row_bytes;
                    d.zero = d.zero ? d.zero + r0 * d.zero_row_bytes : nullptr;
                    d.out_codes = zc;
                    d.out_scale = zs;
                    if (validate(d)) {
                        set_error("%s: the plan's class %d decode is outside the kernel's rules", who, c);
                        return R97Q_EINVAL;
                    }
                    if (Np != ns) {
                        const int64_t n = Np * K / 4 - (ns / 8) * (K / 4) * 8;
                        const int64_t m = (Np - ns) * nkb;
                        hipLaunchKernelGGL(vocab_pad_kernel, dim3(blocks(n > m ? n : m, 256)), dim3(256), 0, s, zc,
                                           zs, ns, Np, K);
                        if (int e = launch_status("vocab_pad_kernel")) return e;
                    }
                    dz[z] = d;
                }
                if (int e = decode_tiled_batch(dz, Z, Np, s)) return e;
                DxParams p{};
                p.dY = g.cls[c].out + (b0 / R) * rb * Np;
                p.T = rb;
                p.N = Np;
                p.K = K;
                p.stream = reinterpret_cast<const uint32_t*>(codes);
                p.scale_t = scale_t;
                p.rank = 0;
                p.dX = part;
                p.dx_f32 = 1;
                p.accumulate = 0;
                p.a_scale = cf;  // one factor a 128-column tile: every row reads cf[kt]
                p.a_scale_ld = 0;
                p.mtiles = (int)((rb + kBM - 1) / kBM);
                p.ktiles = (int)(K / kBN);
                p.batch = Z;
                p.z_dy = rb * Np;
                p.z_w = Np * K / 4;
                p.z_scale = nkb * Np;
                p.z_out = rb * K;
                // each weight as the exact sum of two bf16 values: one launch runs the product over
                // the high halves and, in slices of its own, over the low halves into partials of
                // their own (f32 products of bf16 values are exact); the reduction adds each
                // range's two
                p.both = 1;
                p.dX_lo = part_lo;
                launch_dx<R97Q_CODES8>(p, s);
                if (int e = launch_status("qlinear_dx_both_kernel (vocab head)")) return e;
                hipLaunchKernelGGL(vocab_reduce_kernel, dim3(blocks(rb * K, 256)), dim3(256), 0, s, d_x + m0 * K, part,
                                   part_lo, rb * K, Z);
                if (int e = launch_status("vocab_reduce_kernel")) return e;
            }
        }
    }
    if (plan->transform == 128) {
        hipLaunchKernelGGL(vocab_unrotate_kernel, dim3((unsigned)rows, (unsigned)nkb), dim3(128), 0, s, d_x, K);
        if (int e = launch_status("vocab_unrotate_kernel")) return e;
    }
    return R97Q_OK;
}

int r97q_vocab_head_cast(uint16_t* dst, const float* src, int64_t values, R97IqrStream stream) {
    clear_error();
    if (!dst || !src || values <= 0) {
        set_error("r97q_vocab_head_cast: null buffer or no values");
        return R97Q_EINVAL;
    }
    hipLaunchKernelGGL(vocab_cast_kernel, dim3(blocks(values, 256)), dim3(256), 0, (hipStream_t)stream, src, dst,
                       values);
    return launch_status("vocab_cast_kernel");
}

}  // extern "C"
