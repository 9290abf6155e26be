// r97/adjoint.h -- the adjoint-row contract of the reference (include/r97/adjoint.h:54-235 of
// Code000-211/R9700Training), restated so that this build's device rows register and are looked
// up exactly as the reference's are:
//
//   * a row is `void(const AdjointCall&)`; it ADDS its results into `dc` (operand cotangents, f64,
//     schema order) and `grads` (the trainable leaves, f32), never overwrites, and never writes a
//     frozen operand's slot;
//   * rows register from static objects (R97_REGISTER_ADJOINT_* below); for one (op, side) the
//     first row whose predicate accepts the record's parameters serves it, a row with a predicate
//     beats a catch-all whatever the registration order, and rows of equal specificity keep
//     registration order;
//   * a device row is handed the same f64 values a host row is (`AdValue::value`), except for a
//     stored weight, which arrives as `raw` + `enc` with `value` empty.
//
// The registry functions are defined weak in this build's library (rows/registry.cpp): linked into
// the reference's executable, the executable's own registry wins and these rows land in it.
#pragma once

#include <algorithm>
#include <cstdint>
#include <functional>
#include <string>
#include <utility>
#include <variant>
#include <vector>

#include "r97/op.h"
#include "r97/params.h"

namespace r97 {

using OpParam = std::pair<std::string, std::variant<int64_t, std::string>>;

enum class Side { host, device };

// One operand's forward value, or one cotangent.
struct AdValue {
    std::string dtype;           // the forward dtype the record carries
    std::vector<int64_t> shape;  // full logical shape, row-major
    std::vector<double> value;   // numel(shape) values; empty for a stored operand
    const void* raw = nullptr;   // a stored operand's bytes (device memory under the device join)
    const void* enc = nullptr;   // a stored operand's encoding (this build: an R97Encoding, include/r97q.h)
};

struct AdjointCall {
    const OpRecord& rec;              // name, parameters, operands
    const std::vector<AdValue>& fwd;  // every operand's forward value, schema order
    const std::vector<AdValue>& cot;  // the cotangent of each written operand, writes' order
    std::vector<AdValue>* dc;         // every operand's cotangent, schema order: added into
    ParamSet* grads;                  // the trainable leaves, or null
    const char* prefix;               // the leaves' name prefix
    std::function<std::string(int64_t slot)> slot_prefix;  // per-slot prefix, when set
    bool fused_slots = false;         // slots share one [S*R, K] / [N, S*R] factor leaf
    const std::vector<int64_t>* read_rows = nullptr;  // proven read rows, or null (all)
    struct RowCount {
        int64_t zeroed_unreadable = 0;
        int64_t readable = 0;
        int64_t refused_non_finite = 0;
    };
    RowCount* row_count = nullptr;
};

// Whether `row` is read by a consumer: an unproven (null) or empty set reads every row.
inline bool row_readable(const std::vector<int64_t>* rows, int64_t row) {
    if (rows == nullptr || rows->empty()) return true;
    return std::binary_search(rows->begin(), rows->end(), row);
}
inline bool row_readable(const AdjointCall& call, int64_t row) { return row_readable(call.read_rows, row); }

inline void count_read_rows(AdjointCall::RowCount* c, const std::vector<int64_t>* rows, int64_t zeroed,
                            int64_t admitted, int64_t refused) {
    if (c == nullptr || rows == nullptr) return;
    c->zeroed_unreadable += zeroed;
    c->readable += admitted;
    c->refused_non_finite += refused;
}

using TwinFn = void (*)(const OpRecord& rec, const std::vector<AdValue>& operands, std::vector<AdValue>* out);
using AdjointFn = void (*)(const AdjointCall& call);
using ParamPred = bool (*)(const std::vector<OpParam>& params);

// -- registry ----------------------------------------------------------------

void twin_register(const char* op, TwinFn fn, ParamPred pred);
void adjoint_register(const char* op, Side side, AdjointFn fn, const std::vector<int>& frozen, ParamPred pred);

TwinFn twin_find(const std::string& op, const std::vector<OpParam>& params, std::string* error);
AdjointFn adjoint_find(const std::string& op, Side side, const std::vector<OpParam>& params, std::string* error);
std::vector<int> adjoint_frozen(const std::string& op, Side side, const std::vector<OpParam>& params);
std::vector<std::string> ops_registered();

struct OpRows {
    bool twin = false;
    bool host_adjoint = false;
    bool device_adjoint = false;
    std::vector<int> host_frozen;
    std::vector<int> device_frozen;
};
OpRows op_rows(const std::string& op);

// -- registration ------------------------------------------------------------

struct TwinRow {
    const char* op;
    TwinFn fn;
    ParamPred pred;
};
struct AdjointRow {
    const char* op;
    Side side;
    AdjointFn fn;
    std::vector<int> frozen;
    ParamPred pred;
};
struct Registrar {
    explicit Registrar(const TwinRow& r) { twin_register(r.op, r.fn, r.pred); }
    explicit Registrar(const AdjointRow& r) { adjoint_register(r.op, r.side, r.fn, r.frozen, r.pred); }
};

#define R97_REG_NAME2(a, b) a##b
#define R97_REG_NAME(a, b) R97_REG_NAME2(a, b)

#define R97_REGISTER_TWIN(op, fn) \
    static ::r97::Registrar R97_REG_NAME(r97_reg_twin_, __LINE__){::r97::TwinRow{op, fn, nullptr}};
#define R97_REGISTER_TWIN_IF(op, fn, pred) \
    static ::r97::Registrar R97_REG_NAME(r97_reg_twin_, __LINE__){::r97::TwinRow{op, fn, pred}};
#define R97_REGISTER_ADJOINT(op, side, fn) \
    static ::r97::Registrar R97_REG_NAME(r97_reg_adj_, __LINE__){::r97::AdjointRow{op, ::r97::Side::side, fn, {}, nullptr}};
#define R97_REGISTER_ADJOINT_F(op, side, fn, ...)                  \
    static ::r97::Registrar R97_REG_NAME(r97_reg_adj_, __LINE__){ \
        ::r97::AdjointRow{op, ::r97::Side::side, fn, {__VA_ARGS__}, nullptr}};
#define R97_REGISTER_ADJOINT_IF(op, side, fn, pred) \
    static ::r97::Registrar R97_REG_NAME(r97_reg_adj_, __LINE__){::r97::AdjointRow{op, ::r97::Side::side, fn, {}, pred}};
#define R97_REGISTER_ADJOINT_IF_F(op, side, fn, pred, ...)         \
    static ::r97::Registrar R97_REG_NAME(r97_reg_adj_, __LINE__){ \
        ::r97::AdjointRow{op, ::r97::Side::side, fn, {__VA_ARGS__}, pred}};

}  // namespace r97
