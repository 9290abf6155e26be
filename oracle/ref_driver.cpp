// oracle/ref_driver.cpp -- a C ABI over the reference's own host rows, for golden vectors.
//
// TEST INFRASTRUCTURE ONLY. Built by oracle/Makefile together with the reference's sources where
// they lie under /root/reference (nothing is copied) into oracle/_ref/libr97ref.so, which only
// tests/golden/make_golden.py, the oracle's tests and bench.py's cpu_baseline leg load.
//
// Each entry builds the OpRecord the reference's own tests build (tests/host/adjoint_linear.cpp:
// 96-106, tests/host/adjoint_lora.cpp:90-121), looks the row up through the reference registry
// (twin_find / adjoint_find, src/adjoint_registry.cpp:99-113) and calls it. A stored IQR weight
// reaches the rows the way the join hands it: a StoredWeight put under an encoding pointer
// (src/stored_weight.h:35-47) and an operand with `raw`/`enc` set and no values.
#include "r97/adjoint.h"

#include "iqr_decode.h"
#include "r97/optim.h"
#include "stored_weight.h"

#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

using namespace r97;

namespace {

const int kEncToken = 0;  // the encoding pointer the stored weight is keyed by

AdValue values(const char* dtype, std::vector<int64_t> shape, const double* v) {
    AdValue a;
    a.dtype = dtype;
    a.shape = std::move(shape);
    int64_t n = 1;
    for (int64_t d : a.shape) n *= d;
    if (v) a.value.assign(v, v + n);
    else a.value.assign((size_t)n, 0.0);
    return a;
}

OpRecord gemm_nt_rec(int64_t M, int64_t N, int64_t K) {
    OpRecord rec;
    rec.op = "gemm_nt";
    rec.params = {{"M", M}, {"N", N}, {"K", K}, {"dtype", "bf16"}};
    rec.operands = {
        {"a", "bf16", {M, K}, 0, M, false},
        {"b", "bf16", {N, K}, 0, N, false},
        {"y", "f32", {M, N}, 0, M, true},
    };
    return rec;
}

void put_weight(int64_t N, int64_t K, const int8_t* codes, const uint16_t* scale) {
    StoredWeight w;
    w.rows = N;
    w.cols = K;
    w.groups = K / 128;
    w.codes.assign(codes, codes + N * K);
    w.scale.assign(scale, scale + N * (K / 128));
    stored_weight_put(&kEncToken, std::move(w));
}

AdValue stored_operand(int64_t N, int64_t K) {
    AdValue b;
    b.dtype = "bf16";
    b.shape = {N, K};
    b.raw = &kEncToken;
    b.enc = &kEncToken;
    return b;
}

OpRecord shrink_rec(int64_t M, int64_t K, int64_t R, int64_t S) {
    OpRecord rec;
    rec.op = "lora_shrink";
    rec.params = {{"M", M}, {"K", K}, {"R", R}, {"S", S}, {"group", 0}, {"dtype", "bf16"}};
    rec.operands = {{"a", "bf16", {M, K}, 0, M, false},
                    {"a_scale", "invalid", {}, 0, 0, false},
                    {"slot", "i32", {M}, 0, M, false},
                    {"lora_a", "bf16", {S, R, K}, 0, S, false},
                    {"t", "f32", {M, R}, 0, M, true}};
    return rec;
}

OpRecord expand_rec(int64_t M, int64_t N, int64_t R, int64_t S, bool mm) {
    OpRecord rec;
    rec.op = mm ? "lora_expand_mm" : "lora_expand";
    rec.params = {{"M", M}, {"N", N}, {"R", R}, {"S", S}, {"dtype", "bf16"}};
    rec.operands = {{"t", "f32", {M, R}, 0, M, false},
                    {"slot", "i32", {M}, 0, M, false},
                    {"lora_b", "bf16", {S, N, R}, 0, S, false},
                    {"scale", "f32", {S, N}, 0, S, false},
                    {"y", "bf16", {M, N}, 0, M, true}};
    return rec;
}

// tests/host/adjoint_linear.cpp:108-120, the weight stored
OpRecord gemm_nt_q_rec(int64_t M, int64_t N, int64_t K) {
    OpRecord rec;
    rec.op = "gemm_nt_q";
    rec.params = {{"M", M}, {"N", N}, {"K", K}, {"group", 128}, {"dtype", "i8a8h"}};
    rec.operands = {
        {"a", "i8", {M, K}, 0, M, false},
        {"a_scale", "f32", {M, K / 128}, 0, M, false},
        {"b", "i8", {N, K}, 0, N, false},
        {"b_scale", "bf16", {N, K / 128}, 0, N, false},
        {"y", "f32", {M, N}, 0, M, true},
    };
    return rec;
}

// tests/host/adjoint_lora.cpp:89-106, the coded form
OpRecord shrink_q_rec(int64_t M, int64_t K, int64_t R, int64_t S, int64_t group) {
    OpRecord rec;
    rec.op = "lora_shrink";
    rec.params = {{"M", M}, {"K", K}, {"R", R}, {"S", S}, {"group", group}, {"dtype", "i8"}};
    rec.operands = {{"a", "i8", {M, K}, 0, M, false},
                    {"a_scale", "f32", {M, (K + group - 1) / group}, 0, M, false},
                    {"slot", "i32", {M}, 0, M, false},
                    {"lora_a", "bf16", {S, R, K}, 0, S, false},
                    {"t", "f32", {M, R}, 0, M, true}};
    return rec;
}

thread_local std::string g_err;

// The elementwise parts of the fused quantiser producers (src/adjoint/host/elementwise.cpp's rows,
// found through the registry): part 0 rmsnorm (x [rows, n], w [n]; params n, eps, wadd, mult),
// 1 silu_mul (gate_up [rows, 2n]; param n), 2 act_mul with act = sigmoid (a, b [rows, n]).
OpRecord part_rec(int32_t part, int64_t rows, int64_t n, double eps, double wadd, double mult) {
    OpRecord rec;
    auto spell = [](double v) {
        char b[64];
        std::snprintf(b, sizeof b, "%.17g", v);
        return std::string(b);
    };
    if (part == 0) {
        rec.op = "rmsnorm";
        rec.params = {{"n", n}, {"eps", spell(eps)}, {"wadd", spell(wadd)}, {"mult", spell(mult)}};
        rec.operands = {{"x", "bf16", {rows, n}, 0, rows, false},
                        {"w", "bf16", {n}, 0, 1, false},
                        {"y", "bf16", {rows, n}, 0, rows, true}};
    } else if (part == 1) {
        rec.op = "silu_mul";
        rec.params = {{"n", n}};
        rec.operands = {{"gate_up", "bf16", {rows, 2 * n}, 0, rows, false},
                        {"y", "bf16", {rows, n}, 0, rows, true}};
    } else {
        rec.op = "act_mul";
        rec.params = {{"act", std::string("sigmoid")}};
        rec.operands = {{"a", "bf16", {rows, n}, 0, rows, false},
                        {"b", "bf16", {rows, n}, 0, rows, false},
                        {"y", "bf16", {rows, n}, 0, rows, true}};
    }
    return rec;
}

std::vector<OpParam> spec_params(const char* spec) {
    std::vector<OpParam> params;
    std::string s(spec ? spec : "");
    size_t at = 0;
    while (at < s.size()) {
        size_t end = s.find(';', at);
        if (end == std::string::npos) end = s.size();
        const std::string kv = s.substr(at, end - at);
        const size_t eq = kv.find('=');
        if (eq != std::string::npos) {
            const std::string k = kv.substr(0, eq), v = kv.substr(eq + 1);
            const bool digits = !v.empty() && v.find_first_not_of("0123456789") == std::string::npos;
            if (digits) params.push_back({k, (int64_t)std::stoll(v)});
            else params.push_back({k, v});
        }
        at = end + 1;
    }
    return params;
}

std::vector<AdValue> part_inputs(int32_t part, int64_t rows, int64_t n, const double* x0, const double* x1) {
    if (part == 0) return {values("bf16", {rows, n}, x0), values("bf16", {n}, x1)};
    if (part == 1) return {values("bf16", {rows, 2 * n}, x0)};
    return {values("bf16", {rows, n}, x0), values("bf16", {rows, n}, x1)};
}

}  // namespace

extern "C" {

const char* ref_last_error() { return g_err.c_str(); }

int ref_iqr_validate(const R97IqrDecodeDesc* d) { return r97_iqr_validate(*d); }
int ref_iqr_decode(const R97IqrDecodeDesc* d) { return r97_iqr_decode_host(*d); }

int ref_gemm_nt_twin(int64_t M, int64_t N, int64_t K, const double* x, const int8_t* codes,
                     const uint16_t* scale, double* y) {
    try {
        put_weight(N, K, codes, scale);
        OpRecord rec = gemm_nt_rec(M, N, K);
        std::vector<AdValue> reads = {values("bf16", {M, K}, x), stored_operand(N, K)};
        std::vector<AdValue> out;
        TwinFn fn = twin_find(rec.op, rec.params, &g_err);
        if (!fn) return 1;
        fn(rec, reads, &out);
        stored_weight_clear();
        if (out.size() != 1 || (int64_t)out[0].value.size() != M * N) return 2;
        std::memcpy(y, out[0].value.data(), sizeof(double) * (size_t)(M * N));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 3;
    }
}

int ref_gemm_nt_adjoint(int64_t M, int64_t N, int64_t K, const double* dy, const int8_t* codes,
                        const uint16_t* scale, double* dx) {
    try {
        put_weight(N, K, codes, scale);
        OpRecord rec = gemm_nt_rec(M, N, K);
        std::vector<AdValue> fwd = {values("bf16", {M, K}, nullptr), stored_operand(N, K),
                                    values("f32", {M, N}, nullptr)};
        std::vector<AdValue> cot = {values("f32", {M, N}, dy)};
        std::vector<AdValue> dc = {values("bf16", {M, K}, dx), AdValue{}, AdValue{}};
        AdjointFn fn = adjoint_find(rec.op, Side::host, rec.params, &g_err);
        if (!fn) return 1;
        AdjointCall call{rec, fwd, cot, &dc, nullptr, ""};
        fn(call);
        stored_weight_clear();
        std::memcpy(dx, dc[0].value.data(), sizeof(double) * (size_t)(M * K));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 3;
    }
}

int ref_lora_shrink_twin(int64_t M, int64_t K, int64_t R, int64_t S, const double* x,
                         const double* slot, const double* la, double* t) {
    try {
        OpRecord rec = shrink_rec(M, K, R, S);
        AdValue absent;
        absent.dtype = "invalid";
        std::vector<AdValue> reads = {values("bf16", {M, K}, x), absent, values("i32", {M}, slot),
                                      values("bf16", {S, R, K}, la)};
        std::vector<AdValue> out;
        TwinFn fn = twin_find(rec.op, rec.params, &g_err);
        if (!fn) return 1;
        fn(rec, reads, &out);
        if (out.size() != 1) return 2;
        std::memcpy(t, out[0].value.data(), sizeof(double) * (size_t)(M * R));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 3;
    }
}

int ref_lora_shrink_adjoint(int64_t M, int64_t K, int64_t R, int64_t S, const double* x,
                            const double* slot, const double* la, const double* ct, double* dx,
                            float* da, int fused) {
    try {
        OpRecord rec = shrink_rec(M, K, R, S);
        AdValue absent;
        absent.dtype = "invalid";
        std::vector<AdValue> fwd = {values("bf16", {M, K}, x), absent, values("i32", {M}, slot),
                                    values("bf16", {S, R, K}, la), values("f32", {M, R}, nullptr)};
        std::vector<AdValue> cot = {values("f32", {M, R}, ct)};
        std::vector<AdValue> dc = {values("bf16", {M, K}, dx), AdValue{}, AdValue{}, AdValue{},
                                   AdValue{}};
        ParamSet grads;
        Param p;
        p.name = "site.lora_A";
        p.shape = fused ? std::vector<int64_t>{S * R, K} : std::vector<int64_t>{R, K};
        const int64_t na = (fused ? S * R : R) * K;
        p.value.assign(da, da + na);
        grads.push_back(std::move(p));
        AdjointFn fn = adjoint_find(rec.op, Side::host, rec.params, &g_err);
        if (!fn) return 1;
        AdjointCall call{rec, fwd, cot, &dc, &grads, "site"};
        call.fused_slots = fused != 0;
        fn(call);
        std::memcpy(dx, dc[0].value.data(), sizeof(double) * (size_t)(M * K));
        std::memcpy(da, grads[0].value.data(), sizeof(float) * (size_t)na);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 3;
    }
}

int ref_lora_expand_twin(int64_t M, int64_t N, int64_t R, int64_t S, const double* t,
                         const double* slot, const double* lb, const double* scale, int mm,
                         double* y) {
    try {
        OpRecord rec = expand_rec(M, N, R, S, mm != 0);
        std::vector<AdValue> reads = {values("f32", {M, R}, t), values("i32", {M}, slot),
                                      values("bf16", {S, N, R}, lb), values("f32", {S, N}, scale)};
        std::vector<AdValue> out;
        TwinFn fn = twin_find(rec.op, rec.params, &g_err);
        if (!fn) return 1;
        fn(rec, reads, &out);
        if (out.size() != 1) return 2;
        std::memcpy(y, out[0].value.data(), sizeof(double) * (size_t)(M * N));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 3;
    }
}

int ref_lora_expand_adjoint(int64_t M, int64_t N, int64_t R, int64_t S, const double* t,
                            const double* slot, const double* lb, const double* scale,
                            const double* cy, double* dt, float* db, int fused) {
    try {
        OpRecord rec = expand_rec(M, N, R, S, false);
        std::vector<AdValue> fwd = {values("f32", {M, R}, t), values("i32", {M}, slot),
                                    values("bf16", {S, N, R}, lb), values("f32", {S, N}, scale),
                                    values("bf16", {M, N}, nullptr)};
        std::vector<AdValue> cot = {values("bf16", {M, N}, cy)};
        std::vector<AdValue> dc = {values("f32", {M, R}, dt), AdValue{}, AdValue{}, AdValue{},
                                   AdValue{}};
        ParamSet grads;
        Param p;
        p.name = "site.lora_B";
        p.shape = fused ? std::vector<int64_t>{N, S * R} : std::vector<int64_t>{N, R};
        const int64_t nb = N * (fused ? S * R : R);
        p.value.assign(db, db + nb);
        grads.push_back(std::move(p));
        AdjointFn fn = adjoint_find(rec.op, Side::host, rec.params, &g_err);
        if (!fn) return 1;
        AdjointCall call{rec, fwd, cot, &dc, &grads, "site"};
        call.fused_slots = fused != 0;
        fn(call);
        std::memcpy(dt, dc[0].value.data(), sizeof(double) * (size_t)(M * R));
        std::memcpy(db, grads[0].value.data(), sizeof(float) * (size_t)nb);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 3;
    }
}

int ref_gemm_nt_q_twin(int64_t M, int64_t N, int64_t K, const double* a, const double* a_scale,
                       const int8_t* codes, const uint16_t* scale, double* y) {
    try {
        put_weight(N, K, codes, scale);
        OpRecord rec = gemm_nt_q_rec(M, N, K);
        AdValue b = stored_operand(N, K);
        b.dtype = "i8";
        std::vector<AdValue> reads = {values("i8", {M, K}, a), values("f32", {M, K / 128}, a_scale), b,
                                      values("bf16", {N, K / 128}, nullptr)};
        std::vector<AdValue> out;
        TwinFn fn = twin_find(rec.op, rec.params, &g_err);
        if (!fn) return 1;
        fn(rec, reads, &out);
        stored_weight_clear();
        if (out.size() != 1 || (int64_t)out[0].value.size() != M * N) return 2;
        std::memcpy(y, out[0].value.data(), sizeof(double) * (size_t)(M * N));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 3;
    }
}

int ref_gemm_nt_q_adjoint(int64_t M, int64_t N, int64_t K, const double* dy, const int8_t* codes,
                          const uint16_t* scale, const double* a_scale, double* da) {
    try {
        put_weight(N, K, codes, scale);
        OpRecord rec = gemm_nt_q_rec(M, N, K);
        AdValue b = stored_operand(N, K);
        b.dtype = "i8";
        std::vector<AdValue> fwd = {values("i8", {M, K}, nullptr), values("f32", {M, K / 128}, a_scale), b,
                                    values("bf16", {N, K / 128}, nullptr), values("f32", {M, N}, nullptr)};
        std::vector<AdValue> cot = {values("f32", {M, N}, dy)};
        std::vector<AdValue> dc = {values("i8", {M, K}, da), AdValue{}, AdValue{}, AdValue{}, AdValue{}};
        AdjointFn fn = adjoint_find(rec.op, Side::host, rec.params, &g_err);
        if (!fn) return 1;
        AdjointCall call{rec, fwd, cot, &dc, nullptr, ""};
        fn(call);
        stored_weight_clear();
        std::memcpy(da, dc[0].value.data(), sizeof(double) * (size_t)(M * K));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 3;
    }
}

int ref_lora_shrink_q_twin(int64_t M, int64_t K, int64_t R, int64_t S, int64_t group, const double* a,
                           const double* a_scale, const double* slot, const double* la, double* t) {
    try {
        OpRecord rec = shrink_q_rec(M, K, R, S, group);
        const int64_t groups = (K + group - 1) / group;
        std::vector<AdValue> reads = {values("i8", {M, K}, a), values("f32", {M, groups}, a_scale),
                                      values("i32", {M}, slot), values("bf16", {S, R, K}, la)};
        std::vector<AdValue> out;
        TwinFn fn = twin_find(rec.op, rec.params, &g_err);
        if (!fn) return 1;
        fn(rec, reads, &out);
        if (out.size() != 1) return 2;
        std::memcpy(t, out[0].value.data(), sizeof(double) * (size_t)(M * R));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 3;
    }
}

int ref_lora_shrink_q_adjoint(int64_t M, int64_t K, int64_t R, int64_t S, int64_t group, const double* a,
                              const double* a_scale, const double* slot, const double* la, const double* ct,
                              double* da, double* ds, float* dA, int fused) {
    try {
        OpRecord rec = shrink_q_rec(M, K, R, S, group);
        const int64_t groups = (K + group - 1) / group;
        std::vector<AdValue> fwd = {values("i8", {M, K}, a), values("f32", {M, groups}, a_scale),
                                    values("i32", {M}, slot), values("bf16", {S, R, K}, la),
                                    values("f32", {M, R}, nullptr)};
        std::vector<AdValue> cot = {values("f32", {M, R}, ct)};
        std::vector<AdValue> dc = {values("i8", {M, K}, da), values("f32", {M, groups}, ds), AdValue{},
                                   AdValue{}, AdValue{}};
        ParamSet grads;
        Param p;
        p.name = "site.lora_A";
        p.shape = fused ? std::vector<int64_t>{S * R, K} : std::vector<int64_t>{R, K};
        const int64_t na = (fused ? S * R : R) * K;
        p.value.assign(dA, dA + na);
        grads.push_back(std::move(p));
        AdjointFn fn = adjoint_find(rec.op, Side::host, rec.params, &g_err);
        if (!fn) return 1;
        AdjointCall call{rec, fwd, cot, &dc, &grads, "site"};
        call.fused_slots = fused != 0;
        fn(call);
        std::memcpy(da, dc[0].value.data(), sizeof(double) * (size_t)(M * K));
        std::memcpy(ds, dc[1].value.data(), sizeof(double) * (size_t)(M * groups));
        std::memcpy(dA, grads[0].value.data(), sizeof(float) * (size_t)na);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 3;
    }
}

// ---- AdamW: the reference's Optimiser (src/optim.cpp) ----
struct RefAdamWConfig {
    float lr, beta1, beta2, eps, weight_decay, clip_norm, lr_floor_frac;
    int32_t warmup_steps, total_steps, accum_steps;
};

static AdamWConfig adamw_cfg(const RefAdamWConfig* c) {
    AdamWConfig a;
    a.lr = c->lr;
    a.beta1 = c->beta1;
    a.beta2 = c->beta2;
    a.eps = c->eps;
    a.weight_decay = c->weight_decay;
    a.clip_norm = c->clip_norm;
    a.lr_floor_frac = c->lr_floor_frac;
    a.warmup_steps = c->warmup_steps;
    a.total_steps = c->total_steps;
    a.accum_steps = c->accum_steps;
    a.threads = 1;
    return a;
}

float ref_scheduled_lr(const RefAdamWConfig* c, int32_t step) { return scheduled_lr(adamw_cfg(c), step); }

float ref_clip_global_norm(float* x, int64_t n, float max_norm) {
    ParamSet g(1);
    g[0].name = "g";
    g[0].shape = {n};
    g[0].value.assign(x, x + n);
    const float norm = clip_global_norm(g, max_norm, 1);
    std::memcpy(x, g[0].value.data(), sizeof(float) * (size_t)n);
    return norm;
}

// `count` parameters named p0, p1, ... (decay[i] == 0: the name carries the no_decay marker), initial
// values w (concatenated), `nsteps` gradient sets g (nsteps x the concatenation); returns the final
// w, m, v and accumulation buffer (each the concatenation), the updates done and the pending count,
// read back through the optimiser's own serialise().
int ref_adamw_run(const RefAdamWConfig* c, const int64_t* n, const int32_t* decay, int32_t count, float* w,
                  const float* g, int32_t nsteps, float* m_out, float* v_out, float* acc_out, int32_t* updates,
                  int32_t* pending) {
    try {
        ParamSet params((size_t)count);
        int64_t total = 0;
        for (int32_t i = 0; i < count; ++i) {
            params[i].name = std::string("p") + std::to_string(i) + (decay[i] ? "" : ".nodecay");
            params[i].shape = {n[i]};
            params[i].value.assign(w + total, w + total + n[i]);
            total += n[i];
        }
        AdamWConfig cfg = adamw_cfg(c);
        cfg.no_decay = {".nodecay"};
        Optimiser opt(params, cfg);
        for (int32_t s = 0; s < nsteps; ++s) {
            ParamSet grads = params;
            int64_t off = 0;
            for (int32_t i = 0; i < count; ++i) {
                grads[i].value.assign(g + s * total + off, g + s * total + off + n[i]);
                off += n[i];
            }
            opt.step(grads);
        }
        const std::vector<uint8_t> b = opt.serialise();
        // "R97OPT" u16 version, u16 0, i64 step, i32 pending, i32 count, then per parameter u64 n and
        // n floats each of w, m, v, acc
        size_t at = 6 + 2 + 2;
        int64_t step = 0;
        std::memcpy(&step, b.data() + at, 8);
        at += 8;
        std::memcpy(pending, b.data() + at, 4);
        at += 4 + 4;
        int64_t off = 0;
        for (int32_t i = 0; i < count; ++i) {
            at += 8;
            float* dst[4] = {w + off, m_out + off, v_out + off, acc_out + off};
            for (int a = 0; a < 4; ++a) {
                std::memcpy(dst[a], b.data() + at, sizeof(float) * (size_t)n[i]);
                at += sizeof(float) * (size_t)n[i];
            }
            off += n[i];
        }
        *updates = (int32_t)step;
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 3;
    }
}

// The reference registry's answer for (op, side, dtype): the row's function pointer, or null. With
// this build's libr97rows.so loaded after this library into the same global symbol scope, its
// device rows register here (its registry definitions are weak, this one's are the reference's).
const void* ref_adjoint_find(const char* op, int32_t device, const char* dtype, int64_t group) {
    std::vector<OpParam> params = {{"dtype", std::string(dtype)}};
    if (group > 0) params.push_back({"group", group});
    std::string err;
    AdjointFn fn = adjoint_find(op, device ? Side::device : Side::host, params, &err);
    return reinterpret_cast<const void*>(fn);
}

// The frozen positions the reference registry holds for that row, as a count and the first four.
int32_t ref_adjoint_frozen(const char* op, int32_t device, const char* dtype, int64_t group, int32_t* first4) {
    std::vector<OpParam> params = {{"dtype", std::string(dtype)}};
    if (group > 0) params.push_back({"group", group});
    const std::vector<int> f = adjoint_frozen(op, device ? Side::device : Side::host, params);
    for (size_t i = 0; i < f.size() && i < 4; ++i) first4[i] = f[i];
    return (int32_t)f.size();
}

// The same for a record with parameters spelled "key=value;key=value" (a value of digits only is an
// int, anything else a string), for rows whose predicates read more than the dtype and the group.
const void* ref_adjoint_find_spec(const char* op, int32_t device, const char* spec) {
    std::string err;
    AdjointFn fn = adjoint_find(op, device ? Side::device : Side::host, spec_params(spec), &err);
    return reinterpret_cast<const void*>(fn);
}

int32_t ref_adjoint_frozen_spec(const char* op, int32_t device, const char* spec, int32_t* first4) {
    const std::vector<int> f = adjoint_frozen(op, device ? Side::device : Side::host, spec_params(spec));
    for (size_t i = 0; i < f.size() && i < 4; ++i) first4[i] = f[i];
    return (int32_t)f.size();
}

// y [rows, n] = the part's twin over its inputs
int ref_part_twin(int32_t part, int64_t rows, int64_t n, const double* x0, const double* x1, double eps, double wadd,
                  double mult, double* y) {
    try {
        const OpRecord rec = part_rec(part, rows, n, eps, wadd, mult);
        TwinFn tw = twin_find(rec.op, rec.params, nullptr);
        if (!tw) throw std::runtime_error("no twin for " + rec.op);
        std::vector<AdValue> out;
        tw(rec, part_inputs(part, rows, n, x0, x1), &out);
        if (out.empty() || (int64_t)out[0].value.size() != rows * n) throw std::runtime_error(rec.op + ": no output");
        std::memcpy(y, out[0].value.data(), sizeof(double) * (size_t)(rows * n));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// dx0 (+)= and dx1 (+)= the part's host adjoint of dy [rows, n]: dx0 has x0's shape; dx1 b's for
// act_mul (the rmsnorm gain is frozen: dx1 untouched)
int ref_part_adjoint(int32_t part, int64_t rows, int64_t n, const double* x0, const double* x1, const double* dy,
                     double eps, double wadd, double mult, double* dx0, double* dx1) {
    try {
        const OpRecord rec = part_rec(part, rows, n, eps, wadd, mult);
        AdjointFn fn = adjoint_find(rec.op, Side::host, rec.params, nullptr);
        if (!fn) throw std::runtime_error("no host adjoint for " + rec.op);
        std::vector<AdValue> fwd = part_inputs(part, rows, n, x0, x1);
        std::vector<AdValue> y;
        TwinFn tw = twin_find(rec.op, rec.params, nullptr);
        tw(rec, fwd, &y);
        fwd.push_back(y[0]);
        const std::vector<AdValue> cot = {values("f32", {rows, n}, dy)};
        const int64_t n0 = part == 1 ? rows * 2 * n : rows * n;
        std::vector<AdValue> dc;
        dc.push_back(values("f32", part == 1 ? std::vector<int64_t>{rows, 2 * n} : std::vector<int64_t>{rows, n}, dx0));
        if (part == 0) dc.push_back(values("f32", {n}, nullptr));
        if (part == 2) dc.push_back(values("f32", {rows, n}, dx1));
        dc.push_back(values("f32", {rows, n}, nullptr));
        AdjointCall call{rec, fwd, cot, &dc, nullptr, ""};
        fn(call);
        std::memcpy(dx0, dc[0].value.data(), sizeof(double) * (size_t)n0);
        if (part == 2) std::memcpy(dx1, dc[1].value.data(), sizeof(double) * (size_t)(rows * n));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

}  // extern "C"
