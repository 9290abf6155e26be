// rows.cpp -- the MI355X device rows of the quantized linear and its LoRA adapter, registered
// through r97/adjoint.h so the reference's backward walk finds them where it finds its own
// device rows (src/adjoint/device/linear.hip:744-762, src/adjoint/device/lora.hip:439-579):
//
//   gemm_nt      device, dtype bf16, frozen {1}     dc[a] += dy . W
//                  W a stored IQR weight (AdValue raw + enc): the fused decode + MFMA dX kernel;
//                  W dense bf16 values: one rocBLAS bf16 GEMM (a plain library product)
//   lora_shrink  device, float activations, frozen {1, 2, 3}
//                  dc[a] += t_cot . A_s,   leaf lora_A += t_cot^T . x        (per slot s)
//   lora_expand  device, frozen {1, 2, 3}
//                  dc[t] += (y_cot * scale_s) . B_s, leaf lora_B += (y_cot * scale_s)^T . t
//                  and, for an in-place write, the write's own slot passes y_cot through
//   gemm_nt_q    device, dtype i8a8h with group 128, frozen {1, 2, 3} (the coded trunk)
//                  dc[a][m, k] += a_scale[m, k/128] . (dy . W)[m, k]   (the code basis)
//   lora_shrink  device, a coded (int8) activation, frozen {2, 3}
//                  with g = t_cot . A_s: dc[a] += g * a_scale, dc[a_scale] += the group sums of
//                  g * a, leaf lora_A += t_cot^T . (a * a_scale)
//
// Every row follows the contract's ownership rules: it adds into `dc` and the leaves, never
// overwrites, never writes a frozen slot, and returns with its results host-visible (one
// process-wide stream, synchronised before return). The factor gradients (lora_A, lora_B) are
// added into the step's f32 accumulators on the card (r97/grad_stage.h), named and shaped as the
// leaves, as the reference's device rows do; the walk's grad_stage_flush puts them in `grads`. A
// record whose layout is malformed is left untouched, as the reference's rows do. Any rank, and
// any K or N of an activation, a factor or a cotangent, is served through zero padding (the served
// shapes below). A well-formed record this build cannot serve throws std::runtime_error naming the
// op and the shape, instead of dropping a gradient: a stored weight whose N or K is not a multiple
// of 128 (its planes are laid out for those dims), or whose encoding is not a form the decode
// reads.
//
// Numerics: activations and weights arrive as f64 copies of bf16 values and are uploaded exactly;
// a cotangent (an arbitrary f64) is split into a bf16 [hi | lo] pair and both halves are
// multiplied (linearity), so the products carry ~16 significant bits of it; sums accumulate in f32
// on the card and are added into the f64 slots on the host.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "r97/adjoint.h"
#include "r97/adjoint_family.h"
#include "r97/grad_stage.h"
#include "r97/scratch.h"
#include "r97/stored_weight.h"
#include "r97q.h"

namespace r97 {
namespace {

// ---------------------------------------------------------------- record helpers
int operand_pos(const OpRecord& rec, const char* name) {
    for (size_t i = 0; i < rec.operands.size(); ++i)
        if (rec.operands[i].buffer == name) return (int)i;
    return -1;
}

const OpParam* find_param(const std::vector<OpParam>& params, const char* name) {
    for (const OpParam& p : params)
        if (p.first == name) return &p;
    return nullptr;
}

int64_t param_int(const OpRecord& rec, const char* name, int64_t fallback) {
    const OpParam* p = find_param(rec.params, name);
    if (!p) return fallback;
    const int64_t* v = std::get_if<int64_t>(&p->second);
    return v ? *v : fallback;
}

bool param_is(const std::vector<OpParam>& params, const char* name, const char* value) {
    const OpParam* p = find_param(params, name);
    if (!p) return false;
    const std::string* s = std::get_if<std::string>(&p->second);
    return s && *s == value;
}

bool serves_bf16(const std::vector<OpParam>& params) { return param_is(params, "dtype", "bf16"); }

// the activation the shrink reads is a float tensor (not int8 / fp8 codes with a group scale)
bool float_act(const std::vector<OpParam>& params) {
    return !(param_is(params, "dtype", "i8") || param_is(params, "dtype", "fp8_e4m3") ||
             param_is(params, "dtype", "fp8_e5m2"));
}

// the coded trunk's gemm_nt_q: the i8a8h dtype with 128-wide groups (the stored weight's own)
bool serves_i8a8h(const std::vector<OpParam>& params) {
    const OpParam* g = find_param(params, "group");
    const int64_t* gv = g ? std::get_if<int64_t>(&g->second) : nullptr;
    return param_is(params, "dtype", "i8a8h") && gv && *gv == 128;
}

// the shrink's activation is a code stream with a group scale: int8 codes or the fp8 code dtypes
// (the reference's coded_act, src/adjoint/host/lora.cpp:92-101)
bool coded_act(const std::vector<OpParam>& params) { return !float_act(params); }

// a scale operand's value for (row, group), the reference's layout rule for a grouped scale
// (src/adjoint/host/linear.cpp:99-112): [rows, groups], one value, [groups] or [rows]
double scale_at(const AdValue& sc, int64_t row, int64_t group, int64_t rows, int64_t groups) {
    const int64_t n = (int64_t)sc.value.size();
    if (n == 0) return 1.0;
    if (n == 1) return sc.value[0];
    if (n == rows * groups) return sc.value[(size_t)(row * groups + group)];
    if (n == groups) return sc.value[(size_t)group];
    if (n == rows) return sc.value[(size_t)row];
    const int64_t at = std::min<int64_t>(row * groups + group, n - 1);
    return sc.value[(size_t)at];
}

// src/adjoint/host/lora.cpp:70-77: the width of one scale group over k from `groups` columns
int64_t group_width(int64_t k, int64_t groups) {
    if (k <= 0) return 1;
    if (groups <= 1) return k;
    const int64_t lo = (k + groups - 1) / groups;
    int64_t b = 1;
    while (b < lo) b <<= 1;
    return (k + b - 1) / b == groups ? b : lo;
}

// ---------------------------------------------------------------- host threads
// The host side of a row (conversions, staging copies, the adds into the f64 slots) runs on the
// worker count the reference's host loops use (src/parallel.h:39-90): R97_THREADS when it holds an
// integer of at least 1, else min(8, hardware threads). [0, n) is cut into one contiguous range a
// worker; below `serial` items the caller's thread does it all.
int host_threads() {
    if (const char* e = std::getenv("R97_THREADS")) {
        char* end = nullptr;
        const long v = std::strtol(e, &end, 10);
        if (*e && end != e && *end == '\0' && v >= 1) return (int)v;
    }
    const unsigned hw = std::thread::hardware_concurrency();
    return hw == 0 ? 1 : (int)std::min(hw, 8u);
}

template <class F>
void par_ranges(int64_t n, F&& fn, int64_t serial = 1 << 16) {
    const int nt = host_threads();
    if (n <= 0) return;
    if (nt < 2 || n < serial) {
        fn((int64_t)0, n);
        return;
    }
    std::vector<std::thread> workers;
    const int64_t per = (n + nt - 1) / nt;
    for (int t = 1; t < nt; ++t) {
        const int64_t lo = t * per, hi = std::min(n, lo + per);
        if (lo < hi) workers.emplace_back([&fn, lo, hi] { fn(lo, hi); });
    }
    fn((int64_t)0, std::min(n, per));
    for (auto& w : workers) w.join();
}

// dst[i] += src[i] (f32 results into an f64 slot)
void add_into(double* dst, const float* src, int64_t n) {
    par_ranges(n, [&](int64_t lo, int64_t hi) {
        for (int64_t i = lo; i < hi; ++i) dst[i] += (double)src[i];
    });
}

// ---------------------------------------------------------------- served shapes
// The kernels serve ranks 8, 16, 32 and 64 and widths (K of a shrink, N of an expand) that are
// multiples of 128. Every other shape a record carries is served exactly through zero padding: the
// rank in chunks of at most 64 columns, each padded to the next served rank, and a width padded to
// the next multiple of 128. A zero row of A, column of B, column of a cotangent or column of an
// activation adds nothing to any sum, and the padded parts of the outputs are never read back.
struct RankChunk {
    int64_t j0, rc, rp;  // the chunk's first rank column, its column count, the served rank it runs at
};

std::vector<RankChunk> rank_chunks(int64_t R) {
    std::vector<RankChunk> out;
    for (int64_t j0 = 0; j0 < R; j0 += 64) {
        const int64_t rc = std::min<int64_t>(64, R - j0);
        out.push_back({j0, rc, rc <= 8 ? 8 : rc <= 16 ? 16 : rc <= 32 ? 32 : 64});
    }
    return out;
}

int64_t pad128(int64_t n) { return (n + 127) / 128 * 128; }

// rows x cols of `src` (row stride ld) as a zero-padded [rows_p, cols_p] block, converted by `cvt`
template <class T, class F>
std::vector<T> padded(const double* src, int64_t ld, int64_t rows, int64_t cols, int64_t rows_p, int64_t cols_p,
                      F cvt) {
    std::vector<T> out((size_t)(rows_p * cols_p), T{});
    par_ranges(rows, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; ++r)
            for (int64_t c = 0; c < cols; ++c) out[(size_t)(r * cols_p + c)] = cvt(src[r * ld + c]);
    }, cols > 0 ? std::max<int64_t>(1, (int64_t(1) << 16) / cols) : 1);
    return out;
}

[[noreturn]] void refuse(const std::string& op, const std::string& why) {
    throw std::runtime_error(op + " (MI355X device row): " + why);
}

std::string dims(std::initializer_list<int64_t> d) {
    std::string s = "[";
    for (int64_t v : d) s += (s.size() > 1 ? ", " : "") + std::to_string(v);
    return s + "]";
}

// ---------------------------------------------------------------- leaves
std::string grad_name(const char* prefix, const char* leaf) {
    if (!prefix || !*prefix) return leaf;
    return std::string(prefix) + "." + leaf;
}

// a slot's factor leaf: the record's fused name, the slot's module, or the record's prefix
std::string factor_grad_name(const AdjointCall& call, const char* leaf, int64_t slot) {
    if (call.fused_slots) return grad_name(call.prefix, leaf);
    if (call.slot_prefix) return grad_name(call.slot_prefix(slot).c_str(), leaf);
    return grad_name(call.prefix, leaf);
}

// The step's accumulator each pool row's factor gradient lands in (the reference's grad_dest,
// src/adjoint/device/lora.hip:125-152): the row's block of the fused factor (`stride` elements
// apart), the row's own leaf (slot_prefix), or the one leaf every row sums into. Pool rows the
// record never names get none; a leaf the stage refuses comes out nullptr.
std::vector<float*> stage_dest(const AdjointCall& call, const char* leaf, int64_t S, const std::vector<char>& used,
                               const std::vector<int64_t>& shape, int64_t stride) {
    std::vector<float*> dest((size_t)S, nullptr);
    if (!call.grads) return dest;
    if (call.fused_slots) {
        float* base = device::grad_stage_slot(factor_grad_name(call, leaf, 0), shape);
        for (int64_t s = 0; base && s < S; ++s)
            if (used[(size_t)s]) dest[(size_t)s] = base + s * stride;
        return dest;
    }
    if (call.slot_prefix) {
        for (int64_t s = 0; s < S; ++s)
            if (used[(size_t)s]) dest[(size_t)s] = device::grad_stage_slot(factor_grad_name(call, leaf, s), shape);
        return dest;
    }
    float* base = device::grad_stage_slot(factor_grad_name(call, leaf, 0), shape);
    for (int64_t s = 0; base && s < S; ++s)
        if (used[(size_t)s]) dest[(size_t)s] = base;
    return dest;
}

bool stage_refused(const std::vector<float*>& dest, const std::vector<char>& used, bool want) {
    if (!want) return false;
    for (size_t s = 0; s < used.size(); ++s)
        if (used[s] && !dest[s]) return true;
    return false;
}

// dst[r * ld_dst + c] += src[r * ld_src + c] for r < rows, c < cols: a served chunk's f32 sum into its
// block of a staged leaf (a slot's rank columns of a fused [N, S*R] factor, or the unpadded part)
__global__ void add_block_kernel(float* dst, int64_t ld_dst, const float* src, int64_t ld_src, int64_t rows,
                                 int64_t cols) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * cols) return;
    const int64_t r = i / cols, c = i % cols;
    dst[r * ld_dst + c] += src[r * ld_src + c];
}

// row m's adapter slot, or -1 for a base row (negative, NaN or past the pool)
int64_t row_slot(const AdValue& slot, int64_t m, int64_t S) {
    const double v = slot.value[(size_t)m];
    if (!(v >= 0.0)) return -1;
    const int64_t s = (int64_t)v;
    return s < S ? s : -1;
}

// ---------------------------------------------------------------- bf16 on the host
uint16_t to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x0040u);  // quiet NaN
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float from_bf16(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

void to_bf16(const double* v, size_t n, std::vector<uint16_t>& out) {
    out.resize(n);
    par_ranges((int64_t)n, [&](int64_t lo, int64_t hi) {
        for (int64_t i = lo; i < hi; ++i) out[(size_t)i] = to_bf16((float)v[i]);
    });
}

// v ~ hi + lo, both bf16 (~16 significant bits)
void split_bf16(const std::vector<double>& v, std::vector<uint16_t>& hi, std::vector<uint16_t>& lo) {
    hi.resize(v.size());
    lo.resize(v.size());
    par_ranges((int64_t)v.size(), [&](int64_t a, int64_t b) {
        for (int64_t i = a; i < b; ++i) {
            hi[(size_t)i] = to_bf16((float)v[(size_t)i]);
            lo[(size_t)i] = to_bf16((float)(v[(size_t)i] - (double)from_bf16(hi[(size_t)i])));
        }
    });
}

// ---------------------------------------------------------------- the card
// One stream, buffers by role (device scratch, and pinned host memory for the staging copies), one
// rocBLAS handle; created on first use. A row's device buffers are scratch of that call
// (r97/scratch.h, as the reference's rows take theirs): taken from the ledger as the call needs them
// and all returned when the row ends, so the ledger holds nothing between calls. The pinned buffers
// stay for the next call unless more than kHeldBytes is held. A mutex serialises rows called from
// more than one thread.
constexpr size_t kHeldBytes = size_t(1) << 30;
struct Card {
    std::mutex mu;
    hipStream_t stream = nullptr;
    rocblas_handle blas = nullptr;
    std::map<std::string, std::pair<void*, size_t>> bufs;
    std::map<std::string, std::pair<void*, size_t>> pinned;
};

Card& card() {
    static Card* c = new Card;
    return *c;
}

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void r97q_ok(int rc, const char* what) {
    if (rc != R97Q_OK) throw std::runtime_error(std::string(what) + ": " + r97q_last_error());
}

hipStream_t stream_of(Card& c) {
    if (!c.stream) hip_ok(hipStreamCreate(&c.stream), "hipStreamCreate");
    return c.stream;
}

void* buffer(Card& c, const std::string& role, size_t bytes) {
    auto& b = c.bufs[role];
    if (b.second < bytes || !b.first) {
        device::scratch_free(b.first);
        b = {nullptr, 0};
        b.first = device::scratch_alloc(bytes ? (int64_t)bytes : 1);
        if (!b.first)
            throw std::runtime_error("device scratch: " + std::to_string(bytes) + " bytes refused (" + role + ")");
        b.second = bytes;
    }
    return b.first;
}

// the pinned host buffer of a role (grow-only within a call)
void* pinned(Card& c, const std::string& role, size_t bytes) {
    auto& b = c.pinned[role];
    if (b.second < bytes || !b.first) {
        if (b.first) hip_ok(hipHostFree(b.first), "hipHostFree");
        b = {nullptr, 0};
        hip_ok(hipHostMalloc(&b.first, bytes ? bytes : 1, hipHostMallocDefault), "hipHostMalloc");
        b.second = bytes;
    }
    return b.first;
}

// a row's end: every device buffer returned to the scratch ledger, the pinned buffers freed when
// they hold more than kHeldBytes (the card's work is done: the row synchronised its stream before it
// read its results back, and a row that throws midway returns its scratch through hipFree, which
// waits for the card)
void trim(Card& c) {
    for (auto& kv : c.bufs) device::scratch_free(kv.second.first);
    c.bufs.clear();
    size_t host = 0;
    for (const auto& kv : c.pinned) host += kv.second.second;
    if (host > kHeldBytes) {
        for (auto& kv : c.pinned)
            if (kv.second.first) (void)hipHostFree(kv.second.first);
        c.pinned.clear();
    }
}

// held for the length of one row call, after its lock: trims the card's buffers on the way out
struct RowScope {
    Card& c;
    ~RowScope() { trim(c); }
};

// uploads complete before return: the host vectors are temporaries of the row. The values go
// through the role's pinned buffer (copied in by the host threads), then one DMA copy.
template <class T>
T* upload(Card& c, const std::string& role, const std::vector<T>& h) {
    const size_t bytes = h.size() * sizeof(T);
    void* d = buffer(c, role, bytes);
    uint8_t* p = static_cast<uint8_t*>(pinned(c, role, bytes));
    const uint8_t* src = reinterpret_cast<const uint8_t*>(h.data());
    par_ranges((int64_t)bytes, [&](int64_t lo, int64_t hi) { std::memcpy(p + lo, src + lo, (size_t)(hi - lo)); },
               int64_t(1) << 20);
    hip_ok(hipMemcpyAsync(d, p, bytes, hipMemcpyHostToDevice, stream_of(c)), "upload");
    hip_ok(hipStreamSynchronize(stream_of(c)), "hipStreamSynchronize");
    return static_cast<T*>(d);
}

float* zeros(Card& c, const std::string& role, size_t n) {
    void* d = buffer(c, role, n * sizeof(float));
    hip_ok(hipMemsetAsync(d, 0, n * sizeof(float), stream_of(c)), "hipMemsetAsync");
    return static_cast<float*>(d);
}

// `count` values of T written into the role's pinned buffer by fill(p, lo, hi) over parts [lo, hi)
// of [0, parts) on the host threads (a part: a row, say), then one DMA copy to the role's device
// buffer (no intermediate host vector)
template <class T, class F>
T* upload_fill(Card& c, const std::string& role, int64_t count, int64_t parts, int64_t serial, F&& fill) {
    const size_t bytes = (size_t)count * sizeof(T);
    void* d = buffer(c, role, bytes);
    T* p = static_cast<T*>(pinned(c, role, bytes));
    par_ranges(parts, [&](int64_t lo, int64_t hi) { fill(p, lo, hi); }, serial);
    hip_ok(hipMemcpyAsync(d, p, bytes, hipMemcpyHostToDevice, stream_of(c)), "upload");
    hip_ok(hipStreamSynchronize(stream_of(c)), "hipStreamSynchronize");
    return static_cast<T*>(d);
}

// the n f32 results at `d`, in the download's pinned buffer: valid until the next download
const float* download(Card& c, const float* d, size_t n) {
    float* h = static_cast<float*>(pinned(c, "download", n * sizeof(float)));
    hip_ok(hipMemcpyAsync(h, d, n * sizeof(float), hipMemcpyDeviceToHost, stream_of(c)), "download");
    hip_ok(hipStreamSynchronize(stream_of(c)), "hipStreamSynchronize");
    return h;
}

void add_block(hipStream_t s, float* dst, int64_t ld_dst, const float* src, int64_t ld_src, int64_t rows, int64_t cols) {
    hipLaunchKernelGGL(add_block_kernel, dim3((unsigned)((rows * cols + 255) / 256)), dim3(256), 0, s, dst, ld_dst, src,
                       ld_src, rows, cols);
    hip_ok(hipGetLastError(), "add_block_kernel");
}

// a [rows, cols] block of host f64 values, added into the f64 slot `dst` (row stride ld_dst) from a
// downloaded f32 block of row stride ld_src
void add_host(double* dst, int64_t ld_dst, const float* src, int64_t ld_src, int64_t rows, int64_t cols) {
    par_ranges(rows, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; ++r)
            for (int64_t c = 0; c < cols; ++c) dst[r * ld_dst + c] += (double)src[r * ld_src + c];
    }, cols > 0 ? std::max<int64_t>(1, (int64_t(1) << 16) / cols) : 1);
}

// The prepared weight of a stored operand: its encoding (AdValue::enc, an R97Encoding) over its
// joined device planes (AdValue::raw).
const R97qWeight* stored_weight_of(const AdValue& b, int64_t rows, int64_t cols, hipStream_t s) {
    return device_weight_get(static_cast<const R97Encoding*>(b.enc), b.raw, rows, cols, s);
}

// ---------------------------------------------------------------- gemm_nt
// The reference's gemm_nt adjoint (src/adjoint/host/linear.cpp:221-243, device row
// src/adjoint/device/linear.hip:745): dx[m, k] += sum_n dy[m, n] W(n, k).
void gemm_nt_device(const AdjointCall& call) {
    const OpRecord& rec = call.rec;
    const int ia = operand_pos(rec, "a"), ib = operand_pos(rec, "b");
    if (ia < 0 || ib < 0 || call.cot.empty() || !call.dc || (size_t)std::max(ia, ib) >= call.fwd.size()) return;
    const AdValue& a = call.fwd[(size_t)ia];
    const AdValue& b = call.fwd[(size_t)ib];
    const AdValue& dy = call.cot[0];
    const int64_t K = param_int(rec, "K", a.shape.size() >= 2 ? a.shape[1] : 0);
    const int64_t N = param_int(rec, "N", b.shape.size() >= 2 ? b.shape[0] : 0);
    const int64_t M = param_int(rec, "M", a.shape.empty() ? 0 : a.shape[0]);
    AdValue& dx = (*call.dc)[(size_t)ia];
    if (M <= 0 || N <= 0 || K <= 0 || (int64_t)dy.value.size() != M * N || (int64_t)dx.value.size() != M * K) return;
    const bool stored = b.raw != nullptr || b.enc != nullptr;
    if (!stored && (int64_t)b.value.size() != N * K) return;

    Card& c = card();
    std::lock_guard<std::mutex> lock(c.mu);
    RowScope scope{c};
    const hipStream_t s = stream_of(c);
    std::vector<uint16_t> hi, lo;
    split_bf16(dy.value, hi, lo);
    const uint16_t* d_hi = upload(c, "dy_hi", hi);
    const uint16_t* d_lo = upload(c, "dy_lo", lo);
    float* d_dx = static_cast<float*>(buffer(c, "dx", (size_t)(M * K) * 4));
    if (stored) {
        if (!b.enc) refuse(rec.op, "a stored weight operand carries no encoding");
        if (K % 128 || N % 128) refuse(rec.op, "stored weight " + dims({N, K}) + ": N and K must be multiples of 128");
        if (!b.raw) refuse(rec.op, "a stored weight operand carries no planes");
        const R97qWeight* w = stored_weight_of(b, N, K, s);
        // rank 0: the prep stage only lays the cotangent half out for the fused kernel
        const int64_t wsb = r97q_bwd_workspace_bytes(M, N, K, 0);
        void* ws = buffer(c, "gemm_nt_ws", (size_t)wsb);
        for (int half = 0; half < 2; ++half) {
            r97q_ok(r97q_lora_bwd_prep(M, N, K, half ? d_lo : d_hi, nullptr, nullptr, nullptr, 0, 0.0f, ws, wsb, s),
                    "gemm_nt dX");
            r97q_ok(r97q_qlinear_dx_base(w, half ? d_lo : d_hi, M, 0, d_dx, R97Q_F32, half, ws, wsb, s), "gemm_nt dX");
        }
    } else {
        std::vector<uint16_t> wb;
        to_bf16(b.value.data(), b.value.size(), wb);
        const uint16_t* d_w = upload(c, "w", wb);
        if (!c.blas) {
            if (rocblas_create_handle(&c.blas) != rocblas_status_success) refuse(rec.op, "rocblas_create_handle failed");
        }
        rocblas_set_stream(c.blas, s);
        // row-major dx[M, K] = dy[M, N] . W[N, K] is column-major dx^T[K, M] = W^T[K, N] . dy^T[N, M]
        const float one = 1.0f, zero = 0.0f;
        for (int half = 0; half < 2; ++half) {
            const rocblas_status st = rocblas_gemm_ex(
                c.blas, rocblas_operation_none, rocblas_operation_none, (rocblas_int)K, (rocblas_int)M, (rocblas_int)N,
                &one, d_w, rocblas_datatype_bf16_r, (rocblas_int)K, half ? d_lo : d_hi, rocblas_datatype_bf16_r,
                (rocblas_int)N, half ? &one : &zero, d_dx, rocblas_datatype_f32_r, (rocblas_int)K, d_dx,
                rocblas_datatype_f32_r, (rocblas_int)K, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
            if (st != rocblas_status_success) refuse(rec.op, std::string("rocblas_gemm_ex: ") + rocblas_status_to_string(st));
        }
    }
    add_into(dx.value.data(), download(c, d_dx, (size_t)(M * K)), M * K);
}

// ---------------------------------------------------------------- lora_shrink
// The float shrink's adjoint (src/adjoint/host/lora.cpp:260-328): schema a, a_scale (absent, dtype
// "invalid"), slot, lora_a [S, R, K], t. Per slot s, over that slot's rows:
//   dc[a][m, k] += sum_j t_cot[m, j] A[s, j, k];   lora_A(s)[j, k] += sum_m t_cot[m, j] x[m, k]
// Any rank and K: rank chunks of at most 64 and K padded to 128 (see "served shapes").
void lora_shrink_device(const AdjointCall& call) {
    const std::vector<AdValue>& v = call.fwd;
    if ((v.size() != 4 && v.size() != 5) || call.cot.empty() || !call.dc) return;
    const AdValue &a = v[0], &held = v[1], &slot = v[2], &la = v[3];
    if (held.dtype != "invalid") return;  // a coded activation: the coded row's record
    if (a.shape.size() != 2 || slot.shape.size() != 1 || la.shape.size() != 3) return;
    const int64_t M = a.shape[0], K = a.shape[1], S = la.shape[0], R = la.shape[1];
    if (M <= 0 || K <= 0 || R <= 0 || S <= 0 || la.shape[2] != K || slot.shape[0] != M) return;
    if ((int64_t)a.value.size() != M * K || (int64_t)slot.value.size() != M || (int64_t)la.value.size() != S * R * K)
        return;
    const AdValue& t_cot = call.cot[0];
    AdValue& a_cot = call.dc->at(0);
    if ((int64_t)t_cot.value.size() != M * R || (int64_t)a_cot.value.size() != M * K) return;
    std::vector<char> used((size_t)S, 0);
    for (int64_t m = 0; m < M; ++m) {
        const int64_t sl = row_slot(slot, m, S);
        if (sl >= 0) used[(size_t)sl] = 1;
    }
    if (std::find(used.begin(), used.end(), 1) == used.end()) return;  // every row a base row
    // dA waits in the step's staging on the card (r97/grad_stage.h)
    const std::vector<int64_t> a_shape = call.fused_slots ? std::vector<int64_t>{S * R, K} : std::vector<int64_t>{R, K};
    const std::vector<float*> d_dA = stage_dest(call, "lora_A", S, used, a_shape, R * K);
    if (stage_refused(d_dA, used, call.grads != nullptr)) return;

    Card& c = card();
    std::lock_guard<std::mutex> lock(c.mu);
    RowScope scope{c};
    const hipStream_t s = stream_of(c);
    const int64_t Kp = pad128(K);
    const std::vector<RankChunk> chunks = rank_chunks(R);
    const uint16_t* d_x = upload(c, "x", padded<uint16_t>(a.value.data(), K, M, K, M, Kp, [](double d) { return to_bf16((float)d); }));
    float* d_dx = zeros(c, "dx", (size_t)(M * Kp));
    const int64_t wsb = r97q_lora_shrink_bwd_workspace_bytes(M, Kp, (int32_t)chunks[0].rp);
    void* d_ws = buffer(c, "ws", (size_t)wsb);
    const bool direct = Kp == K;  // a chunk's dA lands in the leaf as it is (unpadded K, rank rc == rp)
    for (int64_t sl = 0; sl < S; ++sl) {
        if (!used[(size_t)sl]) continue;
        for (const RankChunk& ch : chunks) {
            const double* arow = la.value.data() + (sl * R + ch.j0) * K;
            const uint16_t* d_a =
                upload(c, "a_s", padded<uint16_t>(arow, K, ch.rc, K, ch.rp, Kp, [](double d) { return to_bf16((float)d); }));
            std::vector<float> tc((size_t)(M * ch.rp), 0.0f);
            for (int64_t m = 0; m < M; ++m)
                if (row_slot(slot, m, S) == sl)
                    for (int64_t j = 0; j < ch.rc; ++j)
                        tc[(size_t)(m * ch.rp + j)] = (float)t_cot.value[(size_t)(m * R + ch.j0 + j)];
            const float* d_tc = upload(c, "t_cot", tc);
            float* leaf = call.grads ? d_dA[(size_t)sl] + ch.j0 * K : nullptr;
            const bool via = leaf && !(direct && ch.rc == ch.rp);
            float* dA = via ? zeros(c, "dA_chunk", (size_t)(ch.rp * Kp)) : leaf;
            r97q_ok(r97q_lora_shrink_bwd(M, Kp, d_x, d_a, (int32_t)ch.rp, d_tc, d_dx, 1, dA, d_ws, wsb, s),
                    "lora_shrink adjoint");
            if (via) add_block(s, leaf, K, dA, Kp, ch.rc, K);
        }
    }
    add_host(a_cot.value.data(), K, download(c, d_dx, (size_t)(M * Kp)), Kp, M, K);
}

// ---------------------------------------------------------------- lora_expand
// The expand's adjoint (src/adjoint/host/lora.cpp:451-521): schema t, slot, lora_b [S, N, R],
// scale [S, N] (absent in a float trunk's 4-operand record: 1), y. Per slot s, over its rows:
//   dc[t][m, j] += sum_n y_cot[m, n] scale[s, n] B[s, n, j]
//   lora_B(s)[n, j] += sum_m y_cot[m, n] scale[s, n] t[m, j]
// and an in-place write's slot takes y_cot back unchanged. Any rank and N: rank chunks of at most
// 64 and N padded to 128.
void lora_expand_device(const AdjointCall& call) {
    const OpRecord& rec = call.rec;
    const std::vector<AdValue>& v = call.fwd;
    const size_t n = v.size();
    if ((n != 4 && n != 5) || call.cot.empty() || !call.dc || rec.operands.size() < 4) return;
    const AdValue &t = v[0], &slot = v[1], &lb = v[2];
    const bool has_scale = n == 5 || !rec.operands[3].written;
    const AdValue* sc = has_scale ? &v[3] : nullptr;
    if (t.shape.size() != 2 || slot.shape.size() != 1 || lb.shape.size() != 3) return;
    const int64_t M = t.shape[0], R = t.shape[1], S = lb.shape[0], N = lb.shape[1];
    if (M <= 0 || N <= 0 || R <= 0 || S <= 0 || lb.shape[2] != R || slot.shape[0] != M) return;
    if ((int64_t)t.value.size() != M * R || (int64_t)slot.value.size() != M || (int64_t)lb.value.size() != S * N * R)
        return;
    if (sc && (sc->shape.size() != 2 || sc->shape[0] != S || sc->shape[1] != N || (int64_t)sc->value.size() != S * N))
        return;
    const AdValue& y_cot = call.cot[0];
    AdValue& t_cot = call.dc->at(0);
    if ((int64_t)y_cot.value.size() != M * N || (int64_t)t_cot.value.size() != M * R) return;
    // the in-place write's direct path
    for (size_t i = 0; i < rec.operands.size() && i < call.dc->size(); ++i)
        if (rec.operands[i].written && rec.operands[i].in_place) {
            AdValue& d = call.dc->at(i);
            if (d.value.size() == y_cot.value.size())
                par_ranges((int64_t)d.value.size(), [&](int64_t lo, int64_t hi) {
                    for (int64_t e = lo; e < hi; ++e) d.value[(size_t)e] += y_cot.value[(size_t)e];
                });
        }
    std::vector<char> used((size_t)S, 0);
    for (int64_t m = 0; m < M; ++m) {
        const int64_t sl = row_slot(slot, m, S);
        if (sl >= 0) used[(size_t)sl] = 1;
    }
    if (std::find(used.begin(), used.end(), 1) == used.end()) return;
    // dB waits in the step's staging on the card: a slot's [N, R] leaf, or its R columns of the
    // fused [N, S*R] one
    const std::vector<int64_t> b_shape = call.fused_slots ? std::vector<int64_t>{N, S * R} : std::vector<int64_t>{N, R};
    const std::vector<float*> d_dB = stage_dest(call, "lora_B", S, used, b_shape, R);
    if (stage_refused(d_dB, used, call.grads != nullptr)) return;
    const int64_t ld_leaf = call.fused_slots ? S * R : R;

    Card& c = card();
    std::lock_guard<std::mutex> lock(c.mu);
    RowScope scope{c};
    const hipStream_t s = stream_of(c);
    const int64_t Np = pad128(N);
    const std::vector<RankChunk> chunks = rank_chunks(R);
    const int64_t wsb = r97q_lora_expand_bwd_workspace_bytes(M, Np, (int32_t)chunks[0].rp);
    void* d_ws = buffer(c, "ws", (size_t)wsb);
    for (int64_t sl = 0; sl < S; ++sl) {
        if (!used[(size_t)sl]) continue;
        // the slot's rows of y_cot times the slot's scale, as [hi | lo] bf16 halves [M, Np] (other
        // slots' rows and the padded columns zero), written straight into the staging buffers
        const auto half = [&](bool low) {
            return [&, low](uint16_t* p, int64_t lo_m, int64_t hi_m) {
                for (int64_t m = lo_m; m < hi_m; ++m) {
                    uint16_t* row = p + m * Np;
                    if (row_slot(slot, m, S) != sl) {
                        std::memset(row, 0, (size_t)Np * 2);
                        continue;
                    }
                    for (int64_t k = 0; k < N; ++k) {
                        const double v = y_cot.value[(size_t)(m * N + k)] * (sc ? sc->value[(size_t)(sl * N + k)] : 1.0);
                        const uint16_t h = to_bf16((float)v);
                        row[k] = low ? to_bf16((float)(v - (double)from_bf16(h))) : h;
                    }
                    for (int64_t k = N; k < Np; ++k) row[k] = 0;
                }
            };
        };
        const int64_t rows_serial = std::max<int64_t>(1, (int64_t(1) << 16) / Np);
        const uint16_t* d_hi = upload_fill<uint16_t>(c, "dy_hi", M * Np, M, rows_serial, half(false));
        const uint16_t* d_lo = upload_fill<uint16_t>(c, "dy_lo", M * Np, M, rows_serial, half(true));
        for (const RankChunk& ch : chunks) {
            const uint16_t* d_b = upload(c, "b_s", padded<uint16_t>(lb.value.data() + sl * N * R + ch.j0, R, N, ch.rc, Np,
                                                                    ch.rp, [](double d) { return to_bf16((float)d); }));
            const float* d_t = upload(c, "t", padded<float>(t.value.data() + ch.j0, R, M, ch.rc, M, ch.rp,
                                                            [](double d) { return (float)d; }));
            float* d_tc = zeros(c, "t_cot", (size_t)(M * ch.rp));
            float* leaf = call.grads ? d_dB[(size_t)sl] + ch.j0 : nullptr;
            float* d_db = leaf ? zeros(c, "db", (size_t)(Np * ch.rp)) : nullptr;
            r97q_ok(r97q_lora_expand_bwd(M, Np, d_hi, d_b, (int32_t)ch.rp, 1.0f, d_t, d_tc, d_db, d_ws, wsb, s),
                    "lora_expand adjoint");
            r97q_ok(r97q_lora_expand_bwd(M, Np, d_lo, d_b, (int32_t)ch.rp, 1.0f, d_t, d_tc, d_db, d_ws, wsb, s),
                    "lora_expand adjoint");
            if (leaf) add_block(s, leaf, ld_leaf, d_db, ch.rp, N, ch.rc);
            add_host(t_cot.value.data() + ch.j0, R, download(c, d_tc, (size_t)(M * ch.rp)), ch.rp, M, ch.rc);
        }
    }
}

// ---------------------------------------------------------------- gemm_nt_q
// gemm_nt_q's adjoint (src/adjoint/host/linear.cpp:284-317, device row
// src/adjoint/device/linear.hip:744-760): schema a [M, K] codes, a_scale, b [N, K], b_scale, y;
//   dc[a][m, k] += a_scale[m, k/128] . sum_n dy[m, n] code[n, k] b_scale[n, k/128]
// the cotangent of the int8 codes (not a code itself: f64, added in unrounded). A stored weight is
// the prepared weight of its encoding; a weight carried as codes and their scale becomes the same
// int8-code form on the card for the call (N and K zero-padded to 128), read by the same fused
// kernel with the activation's scale in its epilogue.
void gemm_nt_q_device(const AdjointCall& call) {
    const OpRecord& rec = call.rec;
    const int ia = operand_pos(rec, "a"), ias = operand_pos(rec, "a_scale"), ib = operand_pos(rec, "b"),
              ibs = operand_pos(rec, "b_scale");
    if (ia < 0 || ib < 0 || ias < 0 || call.cot.empty() || !call.dc ||
        (size_t)std::max(std::max(ia, ib), std::max(ias, ibs)) >= call.fwd.size())
        return;
    const AdValue& a = call.fwd[(size_t)ia];
    const AdValue& as = call.fwd[(size_t)ias];
    const AdValue& b = call.fwd[(size_t)ib];
    const AdValue& dy = call.cot[0];
    const int64_t K = param_int(rec, "K", a.shape.size() >= 2 ? a.shape[1] : 0);
    const int64_t N = param_int(rec, "N", b.shape.size() >= 2 ? b.shape[0] : 0);
    const int64_t M = param_int(rec, "M", a.shape.empty() ? 0 : a.shape[0]);
    AdValue& da = (*call.dc)[(size_t)ia];
    if (M <= 0 || N <= 0 || K <= 0 || (int64_t)dy.value.size() != M * N || (int64_t)da.value.size() != M * K) return;
    const bool stored = b.raw != nullptr || b.enc != nullptr;
    if (!stored && ((int64_t)b.value.size() != N * K || ibs < 0)) return;
    if (stored && (K % 128 || N % 128)) refuse(rec.op, "stored weight " + dims({N, K}) + ": N and K must be multiples of 128");
    const int64_t Kp = pad128(K), Np = pad128(N);
    const int64_t groups = Kp / 128;  // the record's 128-wide groups, the last one short when K is
    std::vector<float> sa((size_t)(M * groups));
    for (int64_t m = 0; m < M; ++m)
        for (int64_t g = 0; g < groups; ++g) sa[(size_t)(m * groups + g)] = (float)scale_at(as, m, g, M, groups);

    Card& c = card();
    std::lock_guard<std::mutex> lock(c.mu);
    RowScope scope{c};
    const hipStream_t s = stream_of(c);
    std::vector<uint16_t> hi, lo;
    split_bf16(dy.value, hi, lo);
    const auto widen = [&](const std::vector<uint16_t>& h) {
        std::vector<uint16_t> out((size_t)(M * Np), 0);
        for (int64_t m = 0; m < M; ++m) std::memcpy(&out[(size_t)(m * Np)], &h[(size_t)(m * N)], (size_t)N * 2);
        return out;
    };
    const uint16_t* d_hi = upload(c, "dy_hi", widen(hi));
    const uint16_t* d_lo = upload(c, "dy_lo", widen(lo));
    float* d_da = static_cast<float*>(buffer(c, "dx", (size_t)(M * Kp) * 4));
    const float* d_sa = upload(c, "a_scale", sa);
    const R97qWeight* w = nullptr;
    R97qWeight dense{};
    if (stored) {
        if (!b.enc) refuse(rec.op, "a stored weight operand carries no encoding");
        if (!b.raw) refuse(rec.op, "a stored weight operand carries no planes");
        w = stored_weight_of(b, N, K, s);
    } else {
        const AdValue& bs = call.fwd[(size_t)ibs];
        std::vector<int8_t> codes((size_t)(Np * Kp), 0);
        std::vector<uint16_t> scale((size_t)(Np * groups), 0);
        for (int64_t n = 0; n < N; ++n) {
            for (int64_t k = 0; k < K; ++k) codes[(size_t)(n * Kp + k)] = (int8_t)std::lrint(b.value[(size_t)(n * K + k)]);
            for (int64_t g = 0; g < groups; ++g) scale[(size_t)(n * groups + g)] = to_bf16((float)scale_at(bs, n, g, N, groups));
        }
        const int8_t* d_codes = upload(c, "w_codes", codes);
        const uint16_t* d_scale = upload(c, "w_scale", scale);
        int8_t* d_form = static_cast<int8_t*>(buffer(c, "w_form", (size_t)(Np * Kp)));
        uint16_t* d_st = static_cast<uint16_t*>(buffer(c, "w_scale_t", (size_t)(Np * groups) * 2));
        r97q_ok(r97q_weight_from_decoded(d_codes, d_scale, Np, Kp, d_form, d_st, &dense, s), "gemm_nt_q weight");
        w = &dense;
    }
    r97q_ok(r97q_gemm_nt_q_dx(w, d_hi, M, d_sa, d_da, R97Q_F32, 0, s), "gemm_nt_q dA");
    r97q_ok(r97q_gemm_nt_q_dx(w, d_lo, M, d_sa, d_da, R97Q_F32, 1, s), "gemm_nt_q dA");
    add_host(da.value.data(), K, download(c, d_da, (size_t)(M * Kp)), Kp, M, K);
}

// ---------------------------------------------------------------- the coded lora_shrink
// The coded shrink's adjoint (src/adjoint/host/lora.cpp:246-328, device row
// src/adjoint/device/lora.hip:437-577): schema a [M, K] codes (int8, or an fp8 code dtype), a_scale
// [M, groups] f32, slot, lora_a [S, R, K], t. With x = a * a_scale[m, k / group_width(K, groups)]
// and, per slot s over its rows, g = t_cot . A_s:
//   dc[a] += g * a_scale;  dc[a_scale][m, q] += sum_{k in q} g[m, k] a[m, k];
//   lora_A(s) += t_cot^T . x
// Any rank and K: rank chunks of at most 64, K padded to 128 with the unpadded K's group width.
void lora_shrink_q_device(const AdjointCall& call) {
    const std::vector<AdValue>& v = call.fwd;
    if ((v.size() != 4 && v.size() != 5) || call.cot.empty() || !call.dc || call.dc->size() < 2) return;
    const AdValue &a = v[0], &held = v[1], &slot = v[2], &la = v[3];
    if (held.dtype == "invalid") return;  // a float activation: the float row's record
    if (a.shape.size() != 2 || slot.shape.size() != 1 || la.shape.size() != 3 || held.shape.size() != 2) return;
    const int64_t M = a.shape[0], K = a.shape[1], S = la.shape[0], R = la.shape[1];
    if (M <= 0 || K <= 0 || R <= 0 || S <= 0 || la.shape[2] != K || slot.shape[0] != M) return;
    const int64_t groups = held.shape[1];
    if (held.shape[0] != M || groups <= 0 || groups > K || (int64_t)held.value.size() != M * groups) return;
    if ((int64_t)a.value.size() != M * K || (int64_t)slot.value.size() != M || (int64_t)la.value.size() != S * R * K)
        return;
    // the record's `group` states the same grid the scale's columns give (lora.cpp:183-191)
    const int64_t gw = group_width(K, groups);
    const int64_t stated = param_int(call.rec, "group", 0);
    if (stated > 0 && (K + stated - 1) / stated != (K + gw - 1) / gw) return;
    const AdValue& t_cot = call.cot[0];
    AdValue& a_cot = call.dc->at(0);
    AdValue& s_cot = call.dc->at(1);
    if ((int64_t)t_cot.value.size() != M * R || (int64_t)a_cot.value.size() != M * K ||
        (int64_t)s_cot.value.size() != M * groups)
        return;
    std::vector<char> used((size_t)S, 0);
    for (int64_t m = 0; m < M; ++m) {
        const int64_t sl = row_slot(slot, m, S);
        if (sl >= 0) used[(size_t)sl] = 1;
    }
    if (std::find(used.begin(), used.end(), 1) == used.end()) return;  // every row a base row
    const std::vector<int64_t> a_shape = call.fused_slots ? std::vector<int64_t>{S * R, K} : std::vector<int64_t>{R, K};
    const std::vector<float*> d_dA = stage_dest(call, "lora_A", S, used, a_shape, R * K);
    if (stage_refused(d_dA, used, call.grads != nullptr)) return;

    Card& c = card();
    std::lock_guard<std::mutex> lock(c.mu);
    RowScope scope{c};
    const hipStream_t s = stream_of(c);
    const int64_t Kp = pad128(K);
    const std::vector<RankChunk> chunks = rank_chunks(R);
    // int8 codes travel as int8; an fp8 code's value is exact in f32
    const bool i8 = param_is(call.rec.params, "dtype", "i8");
    const void* d_a = i8 ? (const void*)upload(c, "codes", padded<int8_t>(a.value.data(), K, M, K, M, Kp,
                                                                         [](double d) { return (int8_t)std::lrint(d); }))
                         : (const void*)upload(c, "codes", padded<float>(a.value.data(), K, M, K, M, Kp,
                                                                        [](double d) { return (float)d; }));
    std::vector<float> sc(held.value.begin(), held.value.end());
    const float* d_s = upload(c, "a_scale", sc);
    float* d_da = zeros(c, "dx", (size_t)(M * Kp));
    float* d_ds = zeros(c, "ds", (size_t)(M * groups));
    const int64_t wsb = r97q_lora_shrink_q_bwd_workspace_bytes(M, Kp, (int32_t)chunks[0].rp);
    void* d_ws = buffer(c, "ws", (size_t)wsb);
    const bool direct = Kp == K;
    for (int64_t sl = 0; sl < S; ++sl) {
        if (!used[(size_t)sl]) continue;
        for (const RankChunk& ch : chunks) {
            const double* arow = la.value.data() + (sl * R + ch.j0) * K;
            const uint16_t* d_A =
                upload(c, "a_s", padded<uint16_t>(arow, K, ch.rc, K, ch.rp, Kp, [](double d) { return to_bf16((float)d); }));
            std::vector<float> tc((size_t)(M * ch.rp), 0.0f);
            for (int64_t m = 0; m < M; ++m)
                if (row_slot(slot, m, S) == sl)
                    for (int64_t j = 0; j < ch.rc; ++j)
                        tc[(size_t)(m * ch.rp + j)] = (float)t_cot.value[(size_t)(m * R + ch.j0 + j)];
            const float* d_tc = upload(c, "t_cot", tc);
            float* leaf = call.grads ? d_dA[(size_t)sl] + ch.j0 * K : nullptr;
            const bool via = leaf && !(direct && ch.rc == ch.rp);
            float* dA = via ? zeros(c, "dA_chunk", (size_t)(ch.rp * Kp)) : leaf;
            r97q_ok(r97q_lora_shrink_q_bwd(M, Kp, d_a, i8 ? R97Q_I8 : R97Q_F32, d_s, groups, gw, d_A, (int32_t)ch.rp,
                                           d_tc, d_da, d_ds, dA, d_ws, wsb, s),
                    "lora_shrink (coded) adjoint");
            if (via) add_block(s, leaf, K, dA, Kp, ch.rc, K);
        }
    }
    add_host(a_cot.value.data(), K, download(c, d_da, (size_t)(M * Kp)), Kp, M, K);
    add_host(s_cot.value.data(), groups, download(c, d_ds, (size_t)(M * groups)), groups, M, groups);
}

// ---------------------------------------------------------------- the activation quantiser
// A numeric parameter as the reference's rows read one (src/adjoint/device/quant.hip:95-118): an
// int, or a string that is a whole decimal number; false otherwise.
bool num_param(const std::vector<OpParam>& params, const char* name, double* out) {
    const OpParam* p = find_param(params, name);
    if (!p) return false;
    if (const int64_t* i = std::get_if<int64_t>(&p->second)) {
        *out = (double)*i;
        return true;
    }
    const std::string* s = std::get_if<std::string>(&p->second);
    if (!s || s->empty()) return false;
    char* end = nullptr;
    const double v = std::strtod(s->c_str(), &end);
    if (!end || *end != '\0') return false;
    *out = v;
    return true;
}

double param_num(const OpRecord& rec, const char* name, double fallback) {
    double v = 0.0;
    return num_param(rec.params, name, &v) ? v : fallback;
}

// had_quant_act_i8g's straight-through adjoint on the card (the reference's device row
// src/adjoint/device/quant.hip:951-958 with its predicate :129-137; the rule
// src/adjoint/host/quant.cpp:318-372): schema x (read); codes, scale (written). dc[x] += W^T (live
// * cot[codes] / scale); the scale's cotangent is dropped.
bool serves_rotated(const std::vector<OpParam>& params) {
    double n = 0.0, group = 0.0;
    if (!num_param(params, "n", &n) || !num_param(params, "group", &group)) return false;
    if (n <= 0.0 || n != std::floor(n) || group <= 0.0 || group != std::floor(group) || group > 1024.0) return false;
    const int64_t g = (int64_t)group;
    return (g & (g - 1)) == 0 && (int64_t)n % g == 0;
}

void had_quant_device(const AdjointCall& call) {
    const OpRecord& rec = call.rec;
    size_t reads = 0;
    for (const Operand& o : rec.operands)
        if (!o.written) ++reads;
    if (reads == 0 || call.fwd.size() < reads + 2)
        refuse(rec.op, "the record must read the activation and write the codes and the scale");
    if (call.cot.empty()) refuse(rec.op, "the walk handed no cotangent for the codes");
    if (!call.dc || call.dc->empty()) refuse(rec.op, "the walk handed no room for the activation's cotangent");
    const int64_t n = param_int(rec, "n", 0), group = param_int(rec, "group", 0);
    const AdValue& x = call.fwd[0];
    const AdValue& scale = call.fwd[reads + 1];
    const AdValue& g = call.cot[0];
    if (n <= 0 || x.value.size() % (size_t)n != 0) refuse(rec.op, "the activation is not a whole number of rows of 'n'");
    const int64_t rows = (int64_t)x.value.size() / n;
    if (g.value.size() != x.value.size()) refuse(rec.op, "the codes' cotangent has the activation's shape");
    if ((int64_t)scale.value.size() != rows * (n / group)) refuse(rec.op, "the scale does not have one value per (row, group)");
    for (double sv : scale.value)
        if (!(sv > 0.0)) refuse(rec.op, "the scale of a group must be positive");
    AdValue& dx = call.dc->at(0);
    if (dx.value.size() != x.value.size()) refuse(rec.op, "the activation's cotangent has the activation's shape");
    std::vector<float> xf(x.value.begin(), x.value.end()), sf(scale.value.begin(), scale.value.end()),
        gf(g.value.begin(), g.value.end());
    Card& c = card();
    std::lock_guard<std::mutex> lock(c.mu);
    RowScope scope{c};
    const hipStream_t s = stream_of(c);
    const float* d_x = upload(c, "q_x", xf);
    const float* d_s = upload(c, "q_scale", sf);
    const float* d_g = upload(c, "q_g", gf);
    float* d_dx = zeros(c, "q_dx", xf.size());
    r97q_ok(r97q_quant_act_i8g_bwd(d_x, R97Q_F32, rows, n, group, 1, d_s, d_g, d_dx, s), "had_quant_act_i8g adjoint");
    add_into(dx.value.data(), download(c, d_dx, xf.size()), (int64_t)xf.size());
}


// ---------------------------------------------------------------- the fused quantiser producers
// rmsnorm_had_quant_i8g, gated_had_quant_i8g and gate_had_quant_i8g on the card: the reference's
// device rows src/adjoint/device/quant.hip:959-961 (predicates :129-159, the record's roles
// :540-700, the output write's cotangent :817-880) over the composition of its host rows
// src/adjoint/host/quant.cpp:1008-1405. The roles come from the operands, never from positions or
// the `n` / `group` parameters: the codes are the written int8 [rows, n] operand, the scale the
// written float [rows, k] operand with k < n dividing n (group = n / k), a written operand with
// no dtype or shape is a phantom; the layouts served are the schema's two writes, the live tape's
// three (the part's output beside the codes) and, with at most one phantom, four. A write of the
// part's width adds its cotangent to the quantiser's before the part's adjoint; a write over a
// buffer the record also reads, of that read's size, is the direct path and adds its cotangent
// into that read's slot. The norm's gain is frozen (no cotangent), and a norm row no consumer reads
// (the two-way rule, AdjointCall::read_rows) is left out of the result. The intermediate is formed
// on the card from the inputs uploaded at f64, so the clamp decisions are the host twin's.
bool serves_gated(const std::vector<OpParam>& params) {
    if (!serves_rotated(params)) return false;
    const OpParam* a = find_param(params, "act");
    return !a || param_is(params, "act", "silu");
}

bool serves_gate(const std::vector<OpParam>& params) {
    return serves_rotated(params) && param_is(params, "act", "sigmoid");
}

int64_t write_slot(const OpRecord& rec, int64_t operand) {
    int64_t at = 0;
    for (int64_t j = 0; j < (int64_t)rec.operands.size(); ++j) {
        if (!rec.operands[(size_t)j].written) continue;
        if (j == operand) return at;
        ++at;
    }
    return -1;
}

void fused_quant_device(const AdjointCall& call, int32_t part) {
    const OpRecord& rec = call.rec;
    const int64_t operands = (int64_t)rec.operands.size();
    if (!call.dc) refuse(rec.op, "the walk handed no gradient slots");
    if (call.cot.size() < 2) refuse(rec.op, "a record that writes the codes and the scale has two cotangents at least");
    if ((int64_t)call.fwd.size() != operands || (int64_t)call.dc->size() < operands)
        refuse(rec.op, std::to_string(call.fwd.size()) + " forward values and " + std::to_string(call.dc->size()) +
                           " gradient slots for a record of " + std::to_string(operands) + " operands");
    int64_t codes_at = -1, scale_at = -1, reads = 0, writes = 0, phantom = 0;
    std::string listed;
    for (int64_t j = 0; j < operands; ++j) {
        const Operand& o = rec.operands[(size_t)j];
        if (!o.written) {
            ++reads;
            continue;
        }
        ++writes;
        listed += " [" + o.buffer + " " + o.dtype;
        for (int64_t d : o.shape) listed += " " + std::to_string(d);
        listed += "]";
        if (o.dtype.empty() || o.dtype == "invalid" || o.shape.empty()) {
            ++phantom;
            continue;
        }
        if (codes_at < 0 && o.shape.size() == 2 && (o.dtype == "i8" || o.dtype == "fp8_e4m3" || o.dtype == "fp8_e5m2"))
            codes_at = j;
    }
    if (codes_at < 0) refuse(rec.op, "its writes carry no codes operand:" + listed);
    if (rec.operands[(size_t)codes_at].dtype != "i8")
        refuse(rec.op, "fp8 codes are not served by this row (int8 only)");
    const int64_t rows = rec.operands[(size_t)codes_at].shape[0], n = rec.operands[(size_t)codes_at].shape[1];
    for (int64_t j = 0; j < operands && scale_at < 0; ++j) {
        const Operand& o = rec.operands[(size_t)j];
        if (!o.written || j == codes_at || o.shape.size() != 2 || o.shape[0] != rows) continue;
        if (o.dtype != "f32" && o.dtype != "f16" && o.dtype != "bf16") continue;
        if (o.shape[1] > 0 && o.shape[1] < n && n % o.shape[1] == 0) scale_at = j;
    }
    if (rows <= 0 || n <= 0 || scale_at < 0) refuse(rec.op, "its writes carry no group scale over the codes:" + listed);
    const int64_t ngrp = rec.operands[(size_t)scale_at].shape[1], group = n / ngrp;
    if (group > 1024 || (group & (group - 1)) != 0)
        refuse(rec.op, "codes " + std::to_string(n) + " wide over " + std::to_string(ngrp) + " groups is not a group size");
    const int64_t part_reads = part == R97Q_PART_SILU_MUL ? 1 : 2;
    if (reads != part_reads || !(writes == 2 || writes == 3 || (writes == 4 && phantom <= 1)))
        refuse(rec.op, "a record of " + std::to_string(reads) + " reads and " + std::to_string(writes) + " writes (" +
                           std::to_string(phantom) + " phantom) is not a layout this row serves; its writes:" + listed);
    int64_t second_at = -1;
    for (int64_t k = 1; k < operands && second_at < 0; ++k)
        if (!rec.operands[(size_t)k].written) second_at = k;
    if (rec.operands[0].written) refuse(rec.op, "its first operand is a write, not the part's input");
    const int64_t total = rows * n;
    const int64_t in0 = part == R97Q_PART_SILU_MUL ? 2 * total : total;
    const AdValue& x0 = call.fwd[0];
    if ((int64_t)x0.value.size() != in0)
        refuse(rec.op, "its input holds " + std::to_string(x0.value.size()) + " values, the codes need " + std::to_string(in0));
    const AdValue* x1 = second_at >= 0 ? &call.fwd[(size_t)second_at] : nullptr;
    if (part == R97Q_PART_RMSNORM && (int64_t)x1->value.size() < n)
        refuse(rec.op, "the gain holds " + std::to_string(x1->value.size()) + " values for " + std::to_string(n) + " columns");
    if (part == R97Q_PART_SIGMOID_MUL && (int64_t)x1->value.size() != total)
        refuse(rec.op, "the gate's second input holds " + std::to_string(x1->value.size()) + " values, not " +
                           std::to_string(total));
    const AdValue& scale = call.fwd[(size_t)scale_at];
    if ((int64_t)scale.value.size() < rows * ngrp) refuse(rec.op, "the scale holds fewer values than its shape");
    for (int64_t i = 0; i < rows * ngrp; ++i)
        if (!(scale.value[(size_t)i] > 0.0)) refuse(rec.op, "the scale of a group must be positive");
    const int64_t codes_cot = write_slot(rec, codes_at);
    if (codes_cot < 0 || (size_t)codes_cot >= call.cot.size() || (int64_t)call.cot[(size_t)codes_cot].value.size() < total)
        refuse(rec.op, "the codes' cotangent is missing or short");
    AdValue& dc0 = call.dc->at(0);
    if ((int64_t)dc0.value.size() < in0) refuse(rec.op, "the input's gradient slot is short");
    if (part == R97Q_PART_SIGMOID_MUL && (int64_t)call.dc->at((size_t)second_at).value.size() < total)
        refuse(rec.op, "the second input's gradient slot is short");
    const double eps = param_num(rec, "eps", 1e-6), wadd = param_num(rec, "wadd", 0.0),
                 mult = param_num(rec, "mult", 1.0);
    // the norm's live rows: a non-finite activation in a read row refuses (elementwise.cpp:587-603)
    std::vector<char> live_row((size_t)rows, 1);
    if (part == R97Q_PART_RMSNORM) {
        int64_t zeroed = 0, admitted = 0, refused = 0;
        for (int64_t r = 0; r < rows; ++r) {
            if (!row_readable(call, r)) {
                live_row[(size_t)r] = 0;
                ++zeroed;
                continue;
            }
            ++admitted;
            double ss = 0.0;
            for (int64_t i = 0; i < n && std::isfinite(ss); ++i) ss += x0.value[(size_t)(r * n + i)] * x0.value[(size_t)(r * n + i)];
            if (!std::isfinite(ss)) ++refused;
        }
        count_read_rows(call.row_count, call.read_rows, zeroed, admitted, refused);
        if (refused > 0)
            refuse(rec.op, std::to_string(refused) + " of " + std::to_string(admitted) +
                               " rows a consumer reads have a non-finite activation");
    }
    // the output writes' cotangents: the part's width joins the quantiser's, a read's size over the
    // read's buffer is the direct path (quant.cpp:1340-1380)
    std::vector<const AdValue*> outs;
    for (int64_t j = 0; j < operands; ++j) {
        const Operand& o = rec.operands[(size_t)j];
        if (!o.written || j == codes_at || j == scale_at) continue;
        const int64_t at = write_slot(rec, j);
        if (at < 0 || (size_t)at >= call.cot.size()) refuse(rec.op, "the write '" + o.buffer + "' has no cotangent slot");
        const AdValue& oc = call.cot[(size_t)at];
        const int64_t count = (int64_t)oc.value.size();
        if (count == 0 || count == 1) continue;
        if (count == total) {
            outs.push_back(&oc);
            continue;
        }
        int64_t read_at = -1;
        for (int64_t k = 0; k < operands && read_at < 0; ++k)
            if (!rec.operands[(size_t)k].written && rec.operands[(size_t)k].buffer == o.buffer) read_at = k;
        if (read_at < 0 || count != in0)
            refuse(rec.op, "the write '" + o.buffer + "' carries " + std::to_string(count) + " values, not the part's " +
                               std::to_string(total) + " or the direct path's " + std::to_string(in0));
        AdValue& into = call.dc->at((size_t)read_at);
        if ((int64_t)into.value.size() != count) refuse(rec.op, "the direct path's slot is not its cotangent's size");
        for (int64_t i = 0; i < count; ++i) into.value[(size_t)i] += oc.value[(size_t)i];
    }

    Card& c = card();
    std::lock_guard<std::mutex> lock(c.mu);
    RowScope scope{c};
    const hipStream_t s = stream_of(c);
    const double* d_x0 = upload_fill<double>(c, "fq_x0", in0, rows, 64, [&](double* p, int64_t lo, int64_t hi) {
        const int64_t w = in0 / rows;
        std::memcpy(p + lo * w, x0.value.data() + lo * w, sizeof(double) * (size_t)((hi - lo) * w));
    });
    const double* d_x1 = nullptr;
    if (part == R97Q_PART_RMSNORM)
        d_x1 = upload(c, "fq_x1", std::vector<double>(x1->value.begin(), x1->value.begin() + n));
    else if (part == R97Q_PART_SIGMOID_MUL)
        d_x1 = upload_fill<double>(c, "fq_x1", total, rows, 64, [&](double* p, int64_t lo, int64_t hi) {
            std::memcpy(p + lo * n, x1->value.data() + lo * n, sizeof(double) * (size_t)((hi - lo) * n));
        });
    const float* d_s = upload_fill<float>(c, "fq_scale", rows * ngrp, rows, 256, [&](float* p, int64_t lo, int64_t hi) {
        for (int64_t i = lo * ngrp; i < hi * ngrp; ++i) p[i] = (float)scale.value[(size_t)i];
    });
    const AdValue& gc = call.cot[(size_t)codes_cot];
    const float* d_g = upload_fill<float>(c, "fq_g", total, rows, 64, [&](float* p, int64_t lo, int64_t hi) {
        for (int64_t i = lo * n; i < hi * n; ++i) p[i] = (float)gc.value[(size_t)i];
    });
    const float* d_go = nullptr;
    if (!outs.empty())
        d_go = upload_fill<float>(c, "fq_gout", total, rows, 64, [&](float* p, int64_t lo, int64_t hi) {
            for (int64_t i = lo * n; i < hi * n; ++i) {
                double v = 0.0;
                for (const AdValue* o : outs) v += o->value[(size_t)i];
                p[i] = (float)v;
            }
        });
    float* d_dx0 = zeros(c, "fq_dx0", (size_t)in0);
    float* d_dx1 = part == R97Q_PART_SIGMOID_MUL ? zeros(c, "fq_dx1", (size_t)total) : nullptr;
    r97q_ok(r97q_fused_had_quant_i8g_bwd(part, d_x0, d_x1, R97Q_F64, rows, n, group, eps, wadd, mult, d_s, d_g, d_go,
                                         d_dx0, d_dx1, s),
            rec.op.c_str());
    const float* h0 = download(c, d_dx0, (size_t)in0);
    const int64_t w0 = in0 / rows;
    par_ranges(rows, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; ++r)
            if (live_row[(size_t)r])
                for (int64_t i = r * w0; i < (r + 1) * w0; ++i) dc0.value[(size_t)i] += (double)h0[i];
    }, 64);
    if (d_dx1) add_into(call.dc->at((size_t)second_at).value.data(), download(c, d_dx1, (size_t)total), total);
}

void rmsnorm_quant_device(const AdjointCall& call) { fused_quant_device(call, R97Q_PART_RMSNORM); }
void gated_quant_device(const AdjointCall& call) { fused_quant_device(call, R97Q_PART_SILU_MUL); }
void gate_quant_device(const AdjointCall& call) { fused_quant_device(call, R97Q_PART_SIGMOID_MUL); }

}  // namespace

// The frozen positions are the reference's (the weight for gemm_nt; slot, factor and scale for
// the adapter's ops); the float shrink's device row is new here (the reference serves the float
// shrink on the host only).
R97_REGISTER_ADJOINT_IF_F("gemm_nt", device, gemm_nt_device, serves_bf16, 1)
R97_REGISTER_ADJOINT_IF("had_quant_act_i8g", device, had_quant_device, serves_rotated)
R97_REGISTER_ADJOINT_IF_F("rmsnorm_had_quant_i8g", device, rmsnorm_quant_device, serves_rotated, 1)
R97_REGISTER_ADJOINT_IF("gated_had_quant_i8g", device, gated_quant_device, serves_gated)
R97_REGISTER_ADJOINT_IF("gate_had_quant_i8g", device, gate_quant_device, serves_gate)
R97_REGISTER_ADJOINT_IF_F("lora_shrink", device, lora_shrink_device, float_act, 1, 2, 3)
R97_REGISTER_ADJOINT_F("lora_expand", device, lora_expand_device, 1, 2, 3)
// lora_expand_mm is lora_expand with t rounded to bf16 in its twin only (src/adjoint/host/lora.cpp:
// 33-35, 420): the rounding has no derivative, so its adjoint is the expand's row
R97_REGISTER_ADJOINT_F("lora_expand_mm", device, lora_expand_device, 1, 2, 3)
R97_REGISTER_ADJOINT_IF_F("gemm_nt_q", device, gemm_nt_q_device, serves_i8a8h, 1, 2, 3)
R97_REGISTER_ADJOINT_IF_F("lora_shrink", device, lora_shrink_q_device, coded_act, 2, 3)

R97_REGISTER_ADJOINT_FAMILY(Linear, "gemm_nt", "gemm_nt_q");
R97_REGISTER_ADJOINT_FAMILY(Lora, "lora_shrink", "lora_expand", "lora_expand_mm");
R97_REGISTER_ADJOINT_FAMILY(Quant, "had_quant_act_i8g", "rmsnorm_had_quant_i8g", "gated_had_quant_i8g",
                            "gate_had_quant_i8g");

}  // namespace r97
