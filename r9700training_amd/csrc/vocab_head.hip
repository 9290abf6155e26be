// vocab_head.hip -- the vocabulary head's transposed product on gfx950 (the reference's
// src/vocab_head.h:27-99 contract, its kernels src/adjoint/device/vocab_head.hip:82-238):
//
//   d_x[rows, n_embd] += H . sum over classes c of (dy[:, ids_c] . W_c) * scale.col_c
//
// The reference runs it as a gather, a per-token-row GEMV over the decoded int8 grid with f32
// fmas, and the un-rotation. Here it is the register-fed dX kernel's product. A class's rows go in
// ranges of about 4096 (whole trellis runs); every range is decoded once a call into the int8-code
// form in the workspace (the standalone decode's kernel writing tiled, up to kDecodeRanges ranges
// of a class a launch when the form allows). One qlinear_rt_vocab_kernel launch then runs every
// range: the ranges go in slices of a few of one class (enough slices to fill the chip, so a head
// with few token rows or a narrow n_embd still does), a workgroup summing its tile's
// (gathered . W) over each range of its slice -- the weight as the exact sum of two bf16 halves,
// both reduced into one f32 accumulator -- times the class's scale.col (one factor a 128-column
// tile) into the slice's f32 partial; the partials are then added into d_x in slice order
// (deterministic). Ranges are padded to Np (a multiple of 128) rows with zero codes, zero scales and
// zero cotangent columns. The products' operands -- the cotangent's columns of
// every class's rows, each range's [rows, Np] in the fused kernels' tiled layout -- are gathered
// first, for all classes in one launch whose token rows vary slowest, so the workgroups in flight
// cover a few token rows of every class and each cotangent line is fetched from memory about once
// (the classes split the vocabulary at random: a class on its own touches almost every line).
// Token rows go in blocks of at most kRowBlock, each block's operands held at once. The decode runs
// on a side stream of the device beside the first block's gather, joined back into the caller's
// stream before the first product. Once every class is in, the unnormalised 128-wide Hadamard runs
// over each 128 columns of d_x.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "../../include/r97q.h"
#include "act_tiles.h"
#include "iqr_device.h"
#include "qlinear_rt.h"
#include "status.h"

namespace r97q {
namespace {

constexpr int64_t kRangeRows = 4096;  // rows of a range (whole trellis runs)
constexpr int kDecodeRanges = 8;      // ranges a decode launch
constexpr int kFillWorkgroups = 1024;  // slices enough for this many product workgroups (4 x 256 CUs)
constexpr int64_t kRowBlock = 4096;   // token rows a pass (every class's gathered operands held for them)
constexpr int kGatherRows = 16;  // token rows a gather workgroup
constexpr int kGatherLd = 256 + 8;  // LDS row length: a row's 16-byte units start 16 bytes later each row

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

// every range's rows padded to this: the product's shared reduction length (a multiple of 128)
int64_t padded_rows(const R97qVocabPlan& plan) {
    int64_t Np = 0;
    for (int c = 0; c < plan.classes; ++c) {
        const int64_t s = round_up(range_rows(plan.cls[c]), 128);
        Np = s > Np ? s : Np;
    }
    return Np;
}

int64_t ranges_all(const R97qVocabPlan& plan) {
    int64_t n = 0;
    for (int c = 0; c < plan.classes; ++c) n += ranges_of(plan.cls[c]);
    return n;
}

// The product's slices (the ranges counted class by class): enough for kFillWorkgroups workgroups
// of `rows` token rows, at most kVocabSlices; a class's ranges split evenly over slices of at most
// L ranges, L the ranges over the slices wanted. A slice's ranges share a class (its scale.col
// factor), so a class takes at least one. Returns the slices; slice s holds ranges first[s] ..
// first[s+1]-1 of class cls[s].
int vocab_slices(const R97qVocabPlan& plan, int64_t rows, int* first, int* cls) {
    const int64_t wgs = (rows + rt::kBM - 1) / rt::kBM * (plan.n_embd / rt::kBN);
    const int64_t nr = ranges_all(plan);
    int64_t want = (kFillWorkgroups + wgs - 1) / wgs;
    const int64_t most = rt::kVocabSlices - plan.classes + 1;  // the classes' rounding up adds at most one each
    want = want < 1 ? 1 : want > most ? most : want;
    const int64_t L = (nr + want - 1) / want;  // ranges a slice at most
    int n = 0, y = 0;
    for (int c = 0; c < plan.classes; ++c) {
        const int64_t r = ranges_of(plan.cls[c]), k = (r + L - 1) / L;
        for (int64_t j = 0; j < k; ++j) {
            first[n] = y + (int)(j * r / k);
            cls[n++] = c;
        }
        y += (int)r;
    }
    first[n] = y;
    return n;
}

struct VocabWs {
    int64_t codes, scale, gather, part, cf, total;
};

VocabWs vocab_ws(const R97qVocabPlan& plan, int64_t rows) {
    const int64_t Np = padded_rows(plan), K = plan.n_embd, nkb = K / 128, rb = row_block(rows);
    const int64_t nranges = ranges_all(plan);
    int first[rt::kVocabSlices + 1], cls[rt::kVocabSlices];
    const int64_t S = vocab_slices(plan, rb, first, cls);
    VocabWs w{};
    int64_t off = 0;
    auto take = [&](int64_t bytes) {
        const int64_t at = off;
        off += round_up(bytes, 256);
        return at;
    };
    w.codes = take(nranges * Np * K);
    w.scale = take(nranges * nkb * Np * 2);
    w.gather = take(nranges * act_tile_bytes(rb, Np));
    w.part = take(S * rb * K * 4);
    w.cf = take(plan.classes * nkb * 4);
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

// The gathered operands of one block of token rows, each range's [rb, Np] in the fused kernels'
// tiled layout (act_tiles.h): class c's range z holds a[m][n] = dy[m, ids[z*R + n] - vocab_offset]
// for a class row z*R + n < rows and an id inside this vocabulary, else 0 (the range's padding
// columns up to Np and its padding rows up to a multiple of 32 included).
struct GatherClass {
    const int32_t* ids;
    int64_t rows, R;  // the class's rows; rows a range
    uint16_t* out;    // [ranges][the tiled copy of rb x Np]
    int y0;           // the class's first range (ranges of every class counted in class order)
};
struct GatherAll {
    GatherClass cls[4];
    int classes;
    uint32_t nx, per;  // column blocks a range (Np / 256); workgroups a token-row group (nx x ranges)
    int64_t rb, vocab, vocab_offset, Np, ngroups;  // ngroups: token-row groups to 32-row padding
};
// A workgroup: 256 columns of one range x a group of kGatherRows (16) token rows, written as the
// fused kernel's tiled copy (act_tiles.h). The loads go a column a thread, one token row an
// instruction (a wave's 64 columns of a row: their ids ascend within a class, so a few lines of dy),
// into LDS; the stores then go one 16-byte unit of the tiled layout (8 columns of a row) a thread,
// rows fastest, so 16 consecutive threads write 256 contiguous bytes. The workgroups are dealt so
// that XCD x takes the token-row groups x, x + 8, .. whole, one after another, each for every class
// and range: a cotangent line is then fetched into one L2 while its few token rows are gathered, not
// into all eight (the hardware deals workgroup ids round-robin over the XCDs, in id order on each).
// Within a group the blocks go class by class, range by range. The workgroups' own costs (the ids,
// the dependent loads' latency) weigh more than the lines fetched again for each class (a group's
// rows overflow the L2, the 256 MB cache behind it holds them): measured, 16 rows a group 1.43 ms,
// 8 rows 1.48 (a third of the bytes fetched fewer), 32 rows 1.45, 4 rows 1.82, 2 rows 2.64. Also
// slower: a lane's 8 columns x 8 rows loaded at once (~64 lines an instruction, 2x); 2-byte stores
// straight into the tiled layout (8 pieces of 16 bytes an instruction, 1.3x); the classes' blocks
// interleaved in proportion so that a line's readers of every class run close together in time
// (1.2x); 512 or 1024 columns a workgroup (1.06x, 1.15x).
__global__ __launch_bounds__(256) void vocab_gather_kernel(const uint16_t* __restrict__ dy, const GatherAll g) {
    __shared__ __align__(16) uint16_t tile[kGatherRows * kGatherLd];
    const uint32_t xcd = blockIdx.x & 7, l = blockIdx.x >> 3;
    const uint32_t gi = l / g.per, q = l - gi * g.per;  // 32-bit: the 64-bit divisions cost 5% here
    const int64_t grp = (int64_t)gi * 8 + xcd;
    if (grp >= g.ngroups) return;  // the whole workgroup: the barrier below is reached by all or none
    const uint32_t y = q / g.nx, xb = q - y * g.nx;
    int c = 0;
    while (c + 1 < g.classes && (int)y >= g.cls[c + 1].y0) ++c;
    const GatherClass& k = g.cls[c];
    const int64_t z = (int)y - k.y0;
    const int64_t nb = (int64_t)xb * 256;  // the workgroup's first column
    const int64_t mb = grp * kGatherRows;
    const int t = threadIdx.x;
    {
        const int64_t n = nb + t, r = z * k.R + n;
        int64_t col = -1;
        if (n < k.R && r < k.rows) {
            const int64_t id = k.ids[r];
            if (id >= g.vocab_offset && id < g.vocab_offset + g.vocab) col = id - g.vocab_offset;
        }
#pragma unroll
        for (int i = 0; i < kGatherRows; ++i) {
            const int64_t m = mb + i;
            tile[i * kGatherLd + t] = col >= 0 && m < g.rb ? dy[m * g.vocab + col] : (uint16_t)0;
        }
    }
    __syncthreads();
    // the store: the tile's kGatherRows x 32 units of 16 bytes, a unit a thread at a time, row
    // fastest
    uint16_t* a = k.out + z * act_tile_blocks(g.rb) * 32 * g.Np;
#pragma unroll
    for (int u = t; u < kGatherRows * 32; u += 256) {
        const int i = u % kGatherRows;
        const int nl = 8 * (u / kGatherRows);  // the unit's first column in the workgroup
        if (nb + nl < g.Np)
            *reinterpret_cast<uint4*>(a + act_tile_index(mb + i, nb + nl, g.rb)) =
                *reinterpret_cast<const uint4*>(tile + i * kGatherLd + nl);
    }
}

// d_x[i] += part[0][i] + part[1][i] + ... (the slices in order), four values a thread (n a multiple
// of 4)
__global__ __launch_bounds__(256) void vocab_reduce_kernel(float* __restrict__ d_x, const float* __restrict__ part,
                                                           int64_t n, int S) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    float4 v = *reinterpret_cast<const float4*>(d_x + i);
    for (int z = 0; z < S; ++z) {
        const float4 p = *reinterpret_cast<const float4*>(part + z * n + i);
        v.x += p.x;
        v.y += p.y;
        v.z += p.z;
        v.w += p.w;
    }
    *reinterpret_cast<float4*>(d_x + i) = v;
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

// The side stream of a device (and its fork and join events), made on the first call that finds
// none with that device current and its stream not capturing a graph. A call that cannot make one,
// or whose stream belongs to another device than the current one, runs the decode on its own
// stream. Held until the process ends; used under g_side_mu, so calls from several threads fork
// and join one at a time.
struct SideStream {
    hipStream_t s;
    hipEvent_t fork, join;
};
constexpr int kSideDevices = 64;
SideStream g_side[kSideDevices];
bool g_side_ok[kSideDevices] = {};
std::mutex g_side_mu;

const SideStream* side_stream(hipStream_t caller) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kSideDevices) return nullptr;
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(caller, &sdev) != hipSuccess || sdev != dev) {
        (void)hipGetLastError();
        return nullptr;
    }
    if (g_side_ok[dev]) return &g_side[dev];
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(caller, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
    SideStream& sd = g_side[dev];
    bool ok = hipStreamCreateWithFlags(&sd.s, hipStreamNonBlocking) == hipSuccess;
    bool fork = ok && hipEventCreateWithFlags(&sd.fork, hipEventDisableTiming) == hipSuccess;
    ok = fork && hipEventCreateWithFlags(&sd.join, hipEventDisableTiming) == hipSuccess;
    if (!ok) {  // what was made is given back; a later call tries again
        (void)hipGetLastError();
        if (fork) (void)hipEventDestroy(sd.fork);
        if (sd.s) (void)hipStreamDestroy(sd.s);
        sd = SideStream{};
        return nullptr;
    }
    g_side_ok[dev] = true;
    return &sd;
}

// The caller's stream made to wait for the side stream's work so far, once: by the call when the
// decode is needed, else when the call returns (an error return included).
struct SideJoin {
    const SideStream* side = nullptr;
    hipStream_t caller{};
    bool done = true;
    int wait(const char* who) {
        if (done) return R97Q_OK;
        done = true;
        if (hipEventRecord(side->join, side->s) != hipSuccess || hipStreamWaitEvent(caller, side->join, 0) != hipSuccess) {
            set_error("%s: the decode stream's join failed", who);
            return R97Q_ELAUNCH;
        }
        return R97Q_OK;
    }
    ~SideJoin() { (void)wait("r97q_vocab_head_transpose"); }
};

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
    float* cf = reinterpret_cast<float*>(wsb + ws.cf);
    const hipStream_t s = (hipStream_t)stream;
    const int64_t K = plan->n_embd, nkb = K / 128;

    const int64_t Np = padded_rows(*plan);
    const uint32_t nranges = (uint32_t)ranges_all(*plan);
    const uint32_t nx = blocks(Np, 256), per = nx * nranges;  // a token-row group's gather workgroups

    // range z of class c (range y of all): its decode into the int8-code form, at codes + y * Np * K,
    // its scales at scale_t + y * nkb * Np; every one checked before anything is launched
    auto range_desc = [&](int c, int64_t z, int64_t y) {
        const R97qVocabClass& cls = plan->cls[c];
        const int64_t R = range_rows(cls), r0 = z * R;
        R97IqrDecodeDesc d = cls.decode;
        d.row0 = r0;
        d.rows = R < cls.rows - r0 ? R : cls.rows - r0;
        d.codes = d.codes + r0 * d.codes_row_bytes;
        d.scale = d.scale + r0 * d.scale_row_bytes;
        d.zero = d.zero ? d.zero + r0 * d.zero_row_bytes : nullptr;
        d.out_codes = codes + y * Np * K;
        d.out_scale = scale_t + y * nkb * Np;
        return d;
    };
    for (int c = 0, y = 0; c < plan->classes; ++c)
        for (int64_t z = 0; z < ranges_of(plan->cls[c]); ++z, ++y)
            if (validate(range_desc(c, z, y))) {
                set_error("%s: the plan's class %d decode is outside the kernel's rules", who, c);
                return R97Q_EINVAL;
            }

    // The decode (every class's scale.col factors and every range, once a call) runs on the
    // device's side stream, beside the first token-row block's gather on the caller's stream; the
    // caller's stream waits for it before the first product (and on any early return).
    std::unique_lock<std::mutex> lock(g_side_mu);
    const SideStream* side = side_stream(s);
    const hipStream_t ds = side ? side->s : s;
    SideJoin join;
    if (side) {
        if (hipEventRecord(side->fork, s) != hipSuccess || hipStreamWaitEvent(ds, side->fork, 0) != hipSuccess) {
            set_error("%s: the decode stream's fork failed", who);
            return R97Q_ELAUNCH;
        }
        join.side = side;
        join.caller = s;
        join.done = false;
    }
    for (int c = 0, y = 0; c < plan->classes; ++c) {
        const R97qVocabClass& cls = plan->cls[c];
        hipLaunchKernelGGL(vocab_cf_kernel, dim3(blocks(nkb, 64)), dim3(64), 0, ds,
                           static_cast<const uint8_t*>(cls.scale_col), cls.scale_col_dtype, nkb, cf + c * nkb);
        if (int e = launch_status("vocab_cf_kernel")) return e;
        const int64_t nr = ranges_of(cls);
        for (int64_t z0 = 0; z0 < nr; z0 += kDecodeRanges) {
            const int nz = (int)(nr - z0 < kDecodeRanges ? nr - z0 : kDecodeRanges);
            R97IqrDecodeDesc dz[kDecodeRanges];
            for (int i = 0; i < nz; ++i, ++y) {
                const R97IqrDecodeDesc d = range_desc(c, z0 + i, y);
                const int64_t ns = d.rows;
                if (Np != ns) {
                    const int64_t n = Np * K / 4 - (ns / 8) * (K / 4) * 8;
                    const int64_t m = (Np - ns) * nkb;
                    hipLaunchKernelGGL(vocab_pad_kernel, dim3(blocks(n > m ? n : m, 256)), dim3(256), 0, ds,
                                       d.out_codes, d.out_scale, ns, Np, K);
                    if (int e = launch_status("vocab_pad_kernel")) return e;
                }
                dz[i] = d;
            }
            if (int e = decode_tiled_batch(dz, nz, Np, ds)) return e;
        }
    }

    const int64_t rbmax = row_block(rows);
    rt::VocabRtParams v{};
    v.slices = vocab_slices(*plan, rbmax, v.first, v.cls);  // the partials' workspace holds these
    for (int64_t m0 = 0; m0 < rows; m0 += rbmax) {
        const int64_t rb = rows - m0 < rbmax ? rows - m0 : rbmax;
        // every class's gathered operands for token rows [m0, m0 + rb)
        GatherAll g{};
        g.classes = plan->classes;
        g.nx = nx;
        g.per = per;
        g.rb = rb;
        g.vocab = plan->vocab;
        g.vocab_offset = plan->vocab_offset;
        g.Np = Np;
        int64_t goff = 0;
        int y0 = 0;
        for (int c = 0; c < plan->classes; ++c) {
            const R97qVocabClass& cls = plan->cls[c];
            g.cls[c] = GatherClass{static_cast<const int32_t*>(cls.ids), cls.rows, range_rows(cls), gathered + goff, y0};
            goff += ranges_of(cls) * act_tile_blocks(rb) * 32 * Np;
            y0 += (int)ranges_of(cls);
        }
        g.ngroups = act_tile_blocks(rb) * 32 / kGatherRows;
        const int64_t nwg = (g.ngroups + 7) / 8 * 8 * (int64_t)per;  // every XCD's share whole
        if (nwg > INT32_MAX) {
            set_error("%s: %u ranges of %lld rows are more than a launch's grid takes", who, nranges,
                      (long long)kRangeRows);
            return R97Q_EUNSUPPORTED;
        }
        hipLaunchKernelGGL(vocab_gather_kernel, dim3((unsigned)nwg), dim3(256), 0, s, dy + m0 * plan->vocab, g);
        if (int e = launch_status("vocab_gather_kernel")) return e;
        if (m0 == 0) {  // the decode joins the caller's stream before the first product
            if (int e = join.wait(who)) return e;
            lock.unlock();
        }

        // every range's product on the register-fed kernel (qlinear_rt_vocab_kernel), one launch:
        // each weight as the exact sum of two bf16 values, a workgroup reducing its tile over the
        // high halves and then the low halves of each range of its slice into one f32 accumulator
        // (f32 products of bf16 values are exact), a slice's partial of its own; the partials are
        // then added into d_x in slice order
        rt::Params& p = v.p;
        p.act = gathered;
        p.T = rb;
        p.N = Np;
        p.K = K;
        p.stream = reinterpret_cast<const uint32_t*>(codes);
        p.scale_t = scale_t;
        p.run_rows = 1;
        p.rank = 0;
        p.out = part;
        p.out_f32 = 1;
        p.accumulate = 0;
        p.mtiles = (int)((rb + rt::kBM - 1) / rt::kBM);
        p.otiles = (int)(K / rt::kBN);
        p.ksplit = 1;
        p.nfull = p.mtiles * p.otiles;
        v.z_act = act_tile_blocks(rb) * 32 * Np;
        v.z_w = Np * K / 4;
        v.z_scale = nkb * Np;
        v.cf = cf;
        v.cf_ld = nkb;
        rt::launch_vocab(v, s);
        if (int e = launch_status("qlinear_rt_vocab_kernel")) return e;
        hipLaunchKernelGGL(vocab_reduce_kernel, dim3(blocks(rb * K / 4, 256)), dim3(256), 0, s, d_x + m0 * K, part,
                           rb * K, v.slices);
        if (int e = launch_status("vocab_reduce_kernel")) return e;
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
