// rows_hook.cpp -- TEST INFRASTRUCTURE ONLY: a C entry for each device row of libr97rows.so, so the
// Python tests can hand it numpy arrays. Each entry builds the record and the call the way the
// reference's backward walk builds them (schema-ordered operands, f64 forward values, the stored
// weight as raw + enc, dc pre-sized), looks the row up through the registry (adjoint_find on the
// device side) and runs it. Also a self-test of the registry's lookup rules.
#include <chrono>
#include <cstdint>
#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "r97/adjoint.h"
#include "r97/adjoint_family.h"
#include "r97/grad_stage.h"
#include "r97/scratch.h"
#include "r97/stored_weight.h"

using namespace r97;

namespace {

thread_local std::string g_err;
// the wall time of the last row invocation alone (the row's own staging, kernels and adds; not the
// hook's building of the record's f64 values around it), in ms
thread_local double g_row_ms = 0.0;

template <class F>
void timed_row(F&& f) {
    const auto t0 = std::chrono::steady_clock::now();
    f();
    g_row_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

Operand opd(const char* name, const char* dtype, std::vector<int64_t> shape, bool written = false,
            bool in_place = false) {
    Operand o;
    o.buffer = name;
    o.dtype = dtype;
    o.shape = std::move(shape);
    o.written = written;
    o.in_place = in_place;
    return o;
}

AdValue val(const char* dtype, std::vector<int64_t> shape, const double* v) {
    AdValue a;
    a.dtype = dtype;
    a.shape = std::move(shape);
    int64_t n = 1;
    for (int64_t d : a.shape) n *= d;
    if (v) a.value.assign(v, v + n);
    else a.value.assign((size_t)n, 0.0);
    return a;
}

AdjointFn row(const char* op, const std::vector<OpParam>& params) {
    std::string err;
    AdjointFn fn = adjoint_find(op, Side::device, params, &err);
    if (!fn) throw std::runtime_error(err);
    return fn;
}

// a staged leaf's f32 accumulator copied out (the step's staging on the card), n floats
void staged(const std::string& name, const std::vector<int64_t>& shape, float* out, size_t n) {
    float* d = device::grad_stage_slot(name, shape);
    if (!d) throw std::runtime_error("no staged leaf " + name);
    if (hipMemcpy(out, d, n * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess)
        throw std::runtime_error("staged leaf copy failed");
}

// registry self-test rows
void fa(const AdjointCall&) {}
void fb(const AdjointCall&) {}
void fc(const AdjointCall&) {}
void twin_a(const OpRecord&, const std::vector<AdValue>&, std::vector<AdValue>*) {}
void twin_b(const OpRecord&, const std::vector<AdValue>&, std::vector<AdValue>*) {}
bool is_x(const std::vector<OpParam>& p) {
    for (const auto& kv : p)
        if (kv.first == "dtype") {
            const std::string* s = std::get_if<std::string>(&kv.second);
            return s && *s == "x";
        }
    return false;
}

}  // namespace

extern "C" {

const char* rh_last_error() { return g_err.c_str(); }
double rh_last_row_ms() { return g_row_ms; }

// 0, or the line of the first failed check
int rh_registry_selftest() {
#define CHECK(c) \
    do {         \
        if (!(c)) return __LINE__; \
    } while (0)
    const std::vector<OpParam> px = {{"dtype", std::string("x")}}, py = {{"dtype", std::string("y")}};
    // a catch-all registered before a predicated row still loses to it when the predicate accepts
    adjoint_register("rh_op", Side::host, fa, {}, nullptr);
    adjoint_register("rh_op", Side::host, fb, {1}, is_x);
    adjoint_register("rh_op", Side::device, fc, {2}, nullptr);
    CHECK(adjoint_find("rh_op", Side::host, px, nullptr) == fb);
    CHECK(adjoint_find("rh_op", Side::host, py, nullptr) == fa);
    CHECK(adjoint_frozen("rh_op", Side::host, px) == std::vector<int>{1});
    CHECK(adjoint_frozen("rh_op", Side::host, py).empty());
    CHECK(adjoint_find("rh_op", Side::device, py, nullptr) == fc);
    CHECK(adjoint_frozen("rh_op", Side::device, px) == std::vector<int>{2});
    std::string err;
    CHECK(adjoint_find("rh_missing", Side::device, px, &err) == nullptr);
    CHECK(err.find("rh_missing") != std::string::npos && err.find("dtype=x") != std::string::npos);
    const OpRows rows = op_rows("rh_op");
    CHECK(rows.host_adjoint && rows.device_adjoint && rows.device_frozen == std::vector<int>{2});
    CHECK(!rows.twin);
    twin_register("rh_op", twin_a, nullptr);
    twin_register("rh_op", twin_b, is_x);
    CHECK(twin_find("rh_op", px, nullptr) == twin_b && twin_find("rh_op", py, nullptr) == twin_a);
    CHECK(op_rows("rh_op").twin);
    bool seen = false;
    for (const std::string& op : ops_registered()) seen = seen || op == "rh_op";
    CHECK(seen);
    // families: the same family twice is fine, a second family is a hard error
    family_register(AdjointFamily::Lora, {"rh_fam"});
    family_register(AdjointFamily::Lora, {"rh_fam"});
    CHECK(family_find("rh_fam") == AdjointFamily::Lora);
    bool threw = false;
    try {
        family_register(AdjointFamily::Linear, {"rh_fam"});
    } catch (const std::logic_error&) {
        threw = true;
    }
    CHECK(threw);
    CHECK(family_find("rh_unclaimed") == AdjointFamily::None);
    CHECK(std::strcmp(adjoint_family_name(AdjointFamily::Lora), "lora") == 0);
    // this build's device rows
    const std::vector<OpParam> bf16 = {{"dtype", std::string("bf16")}}, f32 = {{"dtype", std::string("f32")}},
                               i8 = {{"dtype", std::string("i8")}};
    CHECK(adjoint_find("gemm_nt", Side::device, bf16, nullptr) != nullptr);
    CHECK(adjoint_frozen("gemm_nt", Side::device, bf16) == std::vector<int>{1});
    CHECK(adjoint_find("gemm_nt", Side::device, f32, nullptr) == nullptr);
    CHECK(adjoint_find("lora_shrink", Side::device, bf16, nullptr) != nullptr);
    CHECK(adjoint_frozen("lora_shrink", Side::device, bf16) == (std::vector<int>{1, 2, 3}));
    // the coded trunk: the coded shrink (i8 and both fp8 code dtypes, the reference's coded_act) and
    // gemm_nt_q (i8a8h, group 128) have device rows; another group width does not
    CHECK(adjoint_find("lora_shrink", Side::device, i8, nullptr) != nullptr);
    CHECK(adjoint_find("lora_shrink", Side::device, i8, nullptr) != adjoint_find("lora_shrink", Side::device, bf16, nullptr));
    CHECK(adjoint_frozen("lora_shrink", Side::device, i8) == (std::vector<int>{2, 3}));
    for (const char* fp8 : {"fp8_e4m3", "fp8_e5m2"})
        CHECK(adjoint_find("lora_shrink", Side::device, {{"dtype", std::string(fp8)}}, nullptr) ==
              adjoint_find("lora_shrink", Side::device, i8, nullptr));
    const std::vector<OpParam> q128 = {{"dtype", std::string("i8a8h")}, {"group", int64_t(128)}},
                               q64 = {{"dtype", std::string("i8a8h")}, {"group", int64_t(64)}};
    CHECK(adjoint_find("gemm_nt_q", Side::device, q128, nullptr) != nullptr);
    CHECK(adjoint_frozen("gemm_nt_q", Side::device, q128) == (std::vector<int>{1, 2, 3}));
    CHECK(adjoint_find("gemm_nt_q", Side::device, q64, nullptr) == nullptr);
    CHECK(family_find("gemm_nt_q") == AdjointFamily::Linear);
    CHECK(adjoint_find("lora_expand", Side::device, bf16, nullptr) != nullptr);
    CHECK(adjoint_frozen("lora_expand", Side::device, f32) == (std::vector<int>{1, 2, 3}));
    CHECK(family_find("gemm_nt") == AdjointFamily::Linear);
    CHECK(family_find("lora_shrink") == AdjointFamily::Lora && family_find("lora_expand") == AdjointFamily::Lora);
    CHECK(adjoint_find("lora_expand_mm", Side::device, bf16, nullptr) ==
          adjoint_find("lora_expand", Side::device, bf16, nullptr));
    CHECK(adjoint_frozen("lora_expand_mm", Side::device, f32) == (std::vector<int>{1, 2, 3}));
    CHECK(family_find("lora_expand_mm") == AdjointFamily::Lora);
#undef CHECK
    return 0;
}

// dx[M, K] += dy[M, N] . W: W the stored IQR weight (its encoding `enc` over the joined device
// planes `raw`, the operand the tape hands) when w_dense is null, else the dense bf16-valued W[N, K].
int rh_gemm_nt(int64_t M, int64_t N, int64_t K, const double* dy, const R97Encoding* enc, const void* raw,
               const double* w_dense, double* dx) {
    try {
        OpRecord rec;
        rec.op = "gemm_nt";
        rec.params = {{"dtype", std::string("bf16")}, {"M", M}, {"N", N}, {"K", K}};
        rec.operands = {opd("a", "bf16", {M, K}), opd("b", w_dense ? "bf16" : "iqr", {N, K}),
                        opd("y", "bf16", {M, N}, true)};
        std::vector<AdValue> fwd = {val("bf16", {M, K}, nullptr), AdValue{}, AdValue{}};
        fwd[1].dtype = rec.operands[1].dtype;
        fwd[1].shape = {N, K};
        if (w_dense) {
            fwd[1].value.assign(w_dense, w_dense + N * K);
        } else {
            fwd[1].raw = raw;
            fwd[1].enc = enc;
            rec.operands[1].enc = enc;
        }
        fwd[2].dtype = "bf16";
        fwd[2].shape = {M, N};
        const std::vector<AdValue> cot = {val("bf16", {M, N}, dy)};
        std::vector<AdValue> dc = {val("bf16", {M, K}, dx), AdValue{}, AdValue{}};
        const AdjointCall call{rec, fwd, cot, &dc, nullptr, "", {}, false, nullptr, nullptr};
        timed_row([&] { row("gemm_nt", rec.params)(call); });
        std::memcpy(dx, dc[0].value.data(), sizeof(double) * (size_t)(M * K));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// the float shrink's row: dx[M, K] += ..., dA: the lora_A leaves, written as [S, R, K] (one slot's
// leaf after another; with `fused` the one [S*R, K] leaf)
int rh_lora_shrink(int64_t M, int64_t K, int64_t R, int64_t S, const double* x, const double* slot, const double* la,
                   const double* t_cot, double* dx, float* dA, int fused) {
    try {
        OpRecord rec;
        rec.op = "lora_shrink";
        rec.params = {{"dtype", std::string("bf16")}};
        rec.operands = {opd("a", "bf16", {M, K}), opd("none:1", "invalid", {}), opd("slot", "i32", {M}),
                        opd("lora_a", "bf16", {S, R, K}), opd("t", "f32", {M, R}, true)};
        AdValue held;
        held.dtype = "invalid";
        const std::vector<AdValue> fwd = {val("bf16", {M, K}, x), held, val("i32", {M}, slot),
                                          val("bf16", {S, R, K}, la), val("f32", {M, R}, nullptr)};
        const std::vector<AdValue> cot = {val("f32", {M, R}, t_cot)};
        std::vector<AdValue> dc = {val("bf16", {M, K}, dx), AdValue{}, AdValue{}, AdValue{}, AdValue{}};
        ParamSet grads;
        AdjointCall call{rec, fwd, cot, &dc, dA ? &grads : nullptr, "layers.0.q", {}, fused != 0, nullptr, nullptr};
        if (!fused) call.slot_prefix = [](int64_t s) { return "adapter" + std::to_string(s); };
        timed_row([&] { row("lora_shrink", rec.params)(call); });
        std::memcpy(dx, dc[0].value.data(), sizeof(double) * (size_t)(M * K));
        if (dA) {
            // the leaves wait in the step's staging; nothing reached `grads`
            if (!grads.empty()) throw std::runtime_error("a leaf reached grads before the flush");
            std::memset(dA, 0, sizeof(float) * (size_t)(S * R * K));
            if (fused) {
                staged("layers.0.q.lora_A", {S * R, K}, dA, (size_t)(S * R * K));
            } else {
                for (int64_t s = 0; s < S; ++s) {
                    bool used = false;
                    for (int64_t m = 0; m < M; ++m) used = used || (slot[m] >= 0 && (int64_t)slot[m] == s);
                    if (used) staged("adapter" + std::to_string(s) + ".lora_A", {R, K}, dA + s * R * K, (size_t)(R * K));
                }
            }
            device::grad_stage_discard();
        }
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// the expand's row: t_cot[M, R] += ..., dB: the lora_B leaves written as [S, N, R] (fused: the one
// [N, S*R] leaf, copied as is), scale [S, N] or null (a 4-operand record), in_place: y is an
// in-place write whose own slot gets y_cot (returned in d_base[M, N])
// the expand's record under `op`: lora_expand, or lora_expand_mm (the same adjoint: the mm form's
// bf16 rounding of t is in its twin only)
int rh_lora_expand_op(const char* op, int64_t M, int64_t N, int64_t R, int64_t S, const double* t, const double* slot,
                      const double* lb, const double* scale, const double* y_cot, double* t_cot, float* dB, int fused,
                      int in_place, double* d_base) {
    try {
        OpRecord rec;
        rec.op = op;
        rec.params = {{"dtype", std::string("bf16")}};
        rec.operands = {opd("t", "f32", {M, R}), opd("slot", "i32", {M}), opd("lora_b", "bf16", {S, N, R})};
        std::vector<AdValue> fwd = {val("f32", {M, R}, t), val("i32", {M}, slot), val("bf16", {S, N, R}, lb)};
        if (scale) {
            rec.operands.push_back(opd("scale", "f32", {S, N}));
            fwd.push_back(val("f32", {S, N}, scale));
        }
        rec.operands.push_back(opd("y", "bf16", {M, N}, true, in_place != 0));
        fwd.push_back(val("bf16", {M, N}, nullptr));  // y's value (an in-place write: the old one it reads)
        const std::vector<AdValue> cot = {val("bf16", {M, N}, y_cot)};
        std::vector<AdValue> dc(rec.operands.size());
        dc[0] = val("f32", {M, R}, t_cot);
        if (in_place) dc.back() = val("bf16", {M, N}, nullptr);
        ParamSet grads;
        AdjointCall call{rec, fwd, cot, &dc, dB ? &grads : nullptr, "layers.0.q", {}, fused != 0, nullptr, nullptr};
        if (!fused) call.slot_prefix = [](int64_t s) { return "adapter" + std::to_string(s); };
        timed_row([&] { row(op, rec.params)(call); });
        std::memcpy(t_cot, dc[0].value.data(), sizeof(double) * (size_t)(M * R));
        if (in_place && d_base) std::memcpy(d_base, dc.back().value.data(), sizeof(double) * (size_t)(M * N));
        if (dB) {
            if (!grads.empty()) throw std::runtime_error("a leaf reached grads before the flush");
            std::memset(dB, 0, sizeof(float) * (size_t)(S * N * R));
            if (fused) {
                staged("layers.0.q.lora_B", {N, S * R}, dB, (size_t)(S * N * R));
            } else {
                for (int64_t s = 0; s < S; ++s) {
                    bool used = false;
                    for (int64_t m = 0; m < M; ++m) used = used || (slot[m] >= 0 && (int64_t)slot[m] == s);
                    if (used) staged("adapter" + std::to_string(s) + ".lora_B", {N, R}, dB + s * N * R, (size_t)(N * R));
                }
            }
            device::grad_stage_discard();
        }
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

int rh_lora_expand(int64_t M, int64_t N, int64_t R, int64_t S, const double* t, const double* slot, const double* lb,
                   const double* scale, const double* y_cot, double* t_cot, float* dB, int fused, int in_place,
                   double* d_base) {
    return rh_lora_expand_op("lora_expand", M, N, R, S, t, slot, lb, scale, y_cot, t_cot, dB, fused, in_place, d_base);
}

// gemm_nt_q's row (the coded trunk): da[M, K] += ..., a codes (values unused by the adjoint),
// a_scale [M, ceil(K/128)], the weight stored (enc over raw) or, when w_codes is given, carried as
// codes [N, K] with b_scale [N, ceil(K/128)]
int rh_gemm_nt_q(int64_t M, int64_t N, int64_t K, const double* dy, const double* a_scale, const R97Encoding* enc,
                 const void* raw, const double* w_codes, const double* b_scale, double* da) {
    try {
        const int64_t G = (K + 127) / 128;
        OpRecord rec;
        rec.op = "gemm_nt_q";
        rec.params = {{"M", M}, {"N", N}, {"K", K}, {"group", int64_t(128)}, {"dtype", std::string("i8a8h")}};
        rec.operands = {opd("a", "i8", {M, K}), opd("a_scale", "f32", {M, G}), opd("b", w_codes ? "i8" : "iqr", {N, K}),
                        opd("b_scale", "bf16", {N, G}), opd("y", "f32", {M, N}, true)};
        std::vector<AdValue> fwd = {val("i8", {M, K}, nullptr), val("f32", {M, G}, a_scale), AdValue{},
                                    val("bf16", {N, G}, b_scale), val("f32", {M, N}, nullptr)};
        fwd[2].dtype = rec.operands[2].dtype;
        fwd[2].shape = {N, K};
        if (w_codes) {
            fwd[2].value.assign(w_codes, w_codes + N * K);
        } else {
            fwd[2].raw = raw;
            fwd[2].enc = enc;
            rec.operands[2].enc = enc;
        }
        const std::vector<AdValue> cot = {val("f32", {M, N}, dy)};
        std::vector<AdValue> dc = {val("i8", {M, K}, da), AdValue{}, AdValue{}, AdValue{}, AdValue{}};
        const AdjointCall call{rec, fwd, cot, &dc, nullptr, "", {}, false, nullptr, nullptr};
        row("gemm_nt_q", rec.params)(call);
        std::memcpy(da, dc[0].value.data(), sizeof(double) * (size_t)(M * K));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// the coded shrink's row: da[M, K] and ds[M, groups] += ..., dA: the lora_A leaves as [S, R, K]
// (fused: the one [S*R, K] leaf)
int rh_lora_shrink_q(int64_t M, int64_t K, int64_t R, int64_t S, int64_t groups, int64_t group, const char* dtype,
                     const double* a, const double* a_scale, const double* slot, const double* la, const double* t_cot,
                     double* da, double* ds, float* dA, int fused) {
    try {
        OpRecord rec;
        rec.op = "lora_shrink";
        rec.params = {{"M", M}, {"K", K}, {"R", R}, {"S", S}, {"group", group}, {"dtype", std::string(dtype)}};
        rec.operands = {opd("a", dtype, {M, K}), opd("a_scale", "f32", {M, groups}), opd("slot", "i32", {M}),
                        opd("lora_a", "bf16", {S, R, K}), opd("t", "f32", {M, R}, true)};
        const std::vector<AdValue> fwd = {val(dtype, {M, K}, a), val("f32", {M, groups}, a_scale), val("i32", {M}, slot),
                                          val("bf16", {S, R, K}, la), val("f32", {M, R}, nullptr)};
        const std::vector<AdValue> cot = {val("f32", {M, R}, t_cot)};
        std::vector<AdValue> dc = {val(dtype, {M, K}, da), val("f32", {M, groups}, ds), AdValue{}, AdValue{}, AdValue{}};
        ParamSet grads;
        AdjointCall call{rec, fwd, cot, &dc, dA ? &grads : nullptr, "layers.1.q", {}, fused != 0, nullptr, nullptr};
        if (!fused) call.slot_prefix = [](int64_t s) { return "adapter" + std::to_string(s); };
        timed_row([&] { row("lora_shrink", rec.params)(call); });
        std::memcpy(da, dc[0].value.data(), sizeof(double) * (size_t)(M * K));
        std::memcpy(ds, dc[1].value.data(), sizeof(double) * (size_t)(M * groups));
        if (dA) {
            if (!grads.empty()) throw std::runtime_error("a leaf reached grads before the flush");
            std::memset(dA, 0, sizeof(float) * (size_t)(S * R * K));
            if (fused) {
                staged("layers.1.q.lora_A", {S * R, K}, dA, (size_t)(S * R * K));
            } else {
                for (int64_t s = 0; s < S; ++s) {
                    bool used = false;
                    for (int64_t m = 0; m < M; ++m) used = used || (slot[m] >= 0 && (int64_t)slot[m] == s);
                    if (used) staged("adapter" + std::to_string(s) + ".lora_A", {R, K}, dA + s * R * K, (size_t)(R * K));
                }
            }
            device::grad_stage_discard();
        }
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// The staging's own rules: `n` floats staged under "stage.x" (twice, adding, the same block both
// times), a second name asked with another shape refused; then flushed into a ParamSet holding
// "stage.x" = base (n) -- out = base + bf16(total) -- and a fresh leaf "stage.y" (zeros + bf16 of its
// total) returned in out_y; the staging is empty after. Returns 0, or the failing check's line.
int rh_stage_flush(const float* a, const float* b, const float* base, int64_t n, float* out, float* out_y) {
    const std::vector<int64_t> shape = {n};
    float* d = device::grad_stage_slot("stage.x", shape);
    if (!d || device::grad_stage_slot("stage.x", shape) != d) return __LINE__;
    if (device::grad_stage_slot("stage.x", {n + 1}) != nullptr) return __LINE__;
    if (device::grad_stage_bytes() != n * (int64_t)sizeof(float)) return __LINE__;
    std::vector<float> zero((size_t)n);
    if (hipMemcpy(zero.data(), d, n * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess) return __LINE__;
    for (float z : zero)
        if (z != 0.0f) return __LINE__;  // a fresh block is zeroed
    if (hipMemcpy(d, a, n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) return __LINE__;
    float* e = device::grad_stage_slot("stage.y", shape);
    if (!e || hipMemcpy(e, b, n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) return __LINE__;
    ParamSet grads(1);
    grads[0].name = "stage.x";
    grads[0].shape = shape;
    grads[0].value.assign(base, base + n);
    if (!device::grad_stage_flush(&grads)) return __LINE__;
    if (grads.size() != 2 || grads[1].name != "stage.y" || grads[1].shape != shape) return __LINE__;
    std::memcpy(out, grads[0].value.data(), n * sizeof(float));
    std::memcpy(out_y, grads[1].value.data(), n * sizeof(float));
    if (device::grad_stage_bytes() != 0) return __LINE__;
    return 0;
}

// had_quant_act_i8g's device row: x [rows, n] f64, scale [rows, n/group] (the forward's), g the codes'
// cotangent; dx [rows, n] added to. Returns -2 when no device row serves the parameters.
int rh_had_quant(int64_t rows, int64_t n, int64_t group, const double* x, const double* scale, const double* g,
                 double* dx) {
    try {
        OpRecord rec;
        rec.op = "had_quant_act_i8g";
        rec.params = {{"M", rows}, {"n", n}, {"group", group}, {"dtype", std::string("bf16")}};
        rec.operands = {opd("x", "bf16", {rows, n}), opd("q", "i8", {rows, n}, true),
                        opd("scale", "f32", {rows, n / group}, true)};
        const std::vector<AdValue> fwd = {val("bf16", {rows, n}, x), val("i8", {rows, n}, nullptr),
                                          val("f32", {rows, n / group}, scale)};
        const std::vector<AdValue> cot = {val("f32", {rows, n}, g), val("f32", {rows, n / group}, nullptr)};
        std::vector<AdValue> dc = {val("bf16", {rows, n}, dx), AdValue{}, AdValue{}};
        AdjointFn fn = adjoint_find(rec.op, Side::device, rec.params, nullptr);
        if (!fn) return -2;
        AdjointCall call{rec, fwd, cot, &dc, nullptr, "", {}, false, nullptr, nullptr};
        fn(call);
        std::memcpy(dx, dc[0].value.data(), sizeof(double) * (size_t)(rows * n));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// The fused quantiser producers' device rows (rmsnorm_had_quant_i8g, gated_had_quant_i8g,
// gate_had_quant_i8g). part 0 rmsnorm (x0 [rows, n], x1 w [n]), 1 silu_mul (x0 gate_up [rows, 2n]),
// 2 sigmoid_mul (x0 gate, x1 x [rows, n]). layout 0: the schema's record (reads, codes, scale);
// 1: the live tape's (the part's output written beside the codes, its cotangent gout, and for the
// norm a phantom write ahead of them, tests/gpu/adjoint_quant.cpp:128-175 of the reference);
// 2: the output write and a write over the first input's buffer (the direct path, cotangent gdir
// of x0's size), no phantom: four writes; 3: layout 2 with the norm's phantom, five writes, which
// no row serves. read_rows (count >= 0) is the two-way rule's read set. dx0 / dx1 are added to. Returns
// -2 when no device row serves the parameters.
int rh_fused_quant(int32_t part, int64_t rows, int64_t n, int64_t group, int32_t layout, const double* x0,
                   const double* x1, const double* scale, const double* g, const double* gout, const double* gdir,
                   double eps, double wadd, double mult, const int64_t* read_rows, int64_t read_count, double* dx0,
                   double* dx1) {
    try {
        static const char* ops[] = {"rmsnorm_had_quant_i8g", "gated_had_quant_i8g", "gate_had_quant_i8g"};
        OpRecord rec;
        rec.op = ops[part];
        rec.params = {{"M", rows}, {"n", n}, {"group", group}, {"dtype", std::string("bf16")}};
        char b[3][64];
        std::snprintf(b[0], sizeof b[0], "%.17g", eps);
        std::snprintf(b[1], sizeof b[1], "%.17g", wadd);
        std::snprintf(b[2], sizeof b[2], "%.17g", mult);
        if (part == 0) rec.params.insert(rec.params.end(), {{"eps", std::string(b[0])}, {"wadd", std::string(b[1])},
                                                           {"mult", std::string(b[2])}});
        if (part == 2) rec.params.push_back({"act", std::string("sigmoid")});
        const int64_t w0 = part == 1 ? 2 * n : n, ngrp = n / group;
        std::vector<AdValue> fwd, cot;
        const char* in0 = part == 0 ? "x" : part == 1 ? "gate_up" : "gate";
        rec.operands.push_back(opd(in0, "bf16", {rows, w0}));
        fwd.push_back(val("bf16", {rows, w0}, x0));
        const bool phantom = part == 0 && (layout == 1 || layout == 3);
        if (phantom) {
            rec.operands.push_back(opd("none:1", "invalid", {}, true));
            fwd.emplace_back();
            cot.emplace_back();
        }
        if (part == 0) {
            rec.operands.push_back(opd("w", "bf16", {n}));
            fwd.push_back(val("bf16", {n}, x1));
        } else if (part == 2) {
            rec.operands.push_back(opd("x", "bf16", {rows, n}));
            fwd.push_back(val("bf16", {rows, n}, x1));
        }
        rec.operands.push_back(opd("q", "i8", {rows, n}, true));
        fwd.push_back(val("i8", {rows, n}, nullptr));
        cot.push_back(val("f32", {rows, n}, g));
        rec.operands.push_back(opd("scale", "f32", {rows, ngrp}, true));
        fwd.push_back(val("f32", {rows, ngrp}, scale));
        cot.push_back(val("f32", {rows, ngrp}, nullptr));
        if (layout >= 1) {
            rec.operands.push_back(opd("out_bf16", "bf16", {rows, n}, true));
            fwd.push_back(val("bf16", {rows, n}, nullptr));
            cot.push_back(val("f32", {rows, n}, gout));
        }
        if (layout >= 2) {
            rec.operands.push_back(opd(in0, "bf16", {rows, w0}, true));
            fwd.push_back(val("bf16", {rows, w0}, nullptr));
            cot.push_back(val("f32", {rows, w0}, gdir));
        }
        std::vector<AdValue> dc;
        for (size_t j = 0; j < rec.operands.size(); ++j) dc.push_back(val("f32", fwd[j].shape, nullptr));
        dc[0].value.assign(dx0, dx0 + rows * w0);
        const size_t second = phantom ? 2 : 1;
        if (part == 2) dc[second].value.assign(dx1, dx1 + rows * n);
        AdjointFn fn = adjoint_find(rec.op, Side::device, rec.params, nullptr);
        if (!fn) return -2;
        std::vector<int64_t> rr;
        if (read_count >= 0) rr.assign(read_rows, read_rows + read_count);
        AdjointCall call{rec, fwd, cot, &dc, nullptr, "", {}, false, read_count >= 0 ? &rr : nullptr, nullptr};
        timed_row([&] { fn(call); });
        std::memcpy(dx0, dc[0].value.data(), sizeof(double) * (size_t)(rows * w0));
        if (part == 2) std::memcpy(dx1, dc[second].value.data(), sizeof(double) * (size_t)(rows * n));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

int64_t rh_weights_prepared() { return device_weight_count(); }
void rh_weights_clear() { device_weight_clear(); }

// the scratch ledger (r97/scratch.h): its counters, a reset (0, or -1 with the error when scratch is
// still held), and a block taken and returned outside any row (a test's stand-in for a leak)
void rh_scratch_stats(int64_t* live, int64_t* peak, int64_t* allocations) {
    const device::ScratchStats s = device::scratch_stats();
    *live = s.live_bytes;
    *peak = s.peak_bytes;
    *allocations = s.allocations;
}
int rh_scratch_reset() {
    try {
        device::scratch_reset();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}
void* rh_scratch_alloc(int64_t bytes) { return device::scratch_alloc(bytes); }
void rh_scratch_free(void* p) { device::scratch_free(p); }

}  // extern "C"
