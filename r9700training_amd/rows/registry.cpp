// registry.cpp -- the adjoint-row registry and the family table behind r97/adjoint.h and
// r97/adjoint_family.h (the reference's src/adjoint_registry.cpp:53-152 and
// src/adjoint_family.cpp:14-53 contracts).
//
// Every definition here is weak: linked into the reference's executable (built with its registry
// exported), the executable's own definitions win and the rows of this library register into
// that registry; loaded on its own (tests, a standalone walk), these serve.
//
// Lookup rule: for one (op, side), the first row with a predicate that accepts the parameters;
// failing that, the first catch-all. Tables are function-local statics created on first use (rows
// register from static initialisers in any order) and never destroyed (a lookup may run from an
// atexit handler).
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "r97/adjoint.h"
#include "r97/adjoint_family.h"

#define R97_WEAK __attribute__((weak))

namespace r97 {
namespace {

struct TwinEntry {
    TwinFn fn;
    ParamPred pred;
};
struct AdjointEntry {
    Side side;
    AdjointFn fn;
    std::vector<int> frozen;
    ParamPred pred;
};
struct Tables {
    std::map<std::string, std::vector<TwinEntry>> twins;        // per op, registration order
    std::map<std::string, std::vector<AdjointEntry>> adjoints;  // per op, registration order
};

Tables& tables() {
    static Tables* t = new Tables;
    return *t;
}

std::string describe(const std::vector<OpParam>& params) {
    std::string out;
    for (const OpParam& p : params) {
        if (!out.empty()) out += ", ";
        out += p.first;
        out += '=';
        if (const int64_t* i = std::get_if<int64_t>(&p.second)) out += std::to_string(*i);
        else out += std::get<std::string>(p.second);
    }
    return out;
}

template <class Entry, class Keep>
const Entry* pick(const std::vector<Entry>& rows, const std::vector<OpParam>& params, Keep keep) {
    const Entry* fallback = nullptr;
    for (const Entry& e : rows) {
        if (!keep(e)) continue;
        if (e.pred == nullptr) {
            if (fallback == nullptr) fallback = &e;
        } else if (e.pred(params)) {
            return &e;
        }
    }
    return fallback;
}

const AdjointEntry* adjoint_row(const std::string& op, Side side, const std::vector<OpParam>& params) {
    const auto it = tables().adjoints.find(op);
    if (it == tables().adjoints.end()) return nullptr;
    return pick(it->second, params, [side](const AdjointEntry& e) { return e.side == side; });
}

std::map<std::string, AdjointFamily>& families() {
    static std::map<std::string, AdjointFamily>* f = new std::map<std::string, AdjointFamily>;
    return *f;
}

}  // namespace

R97_WEAK void twin_register(const char* op, TwinFn fn, ParamPred pred) { tables().twins[op].push_back({fn, pred}); }

R97_WEAK void adjoint_register(const char* op, Side side, AdjointFn fn, const std::vector<int>& frozen,
                               ParamPred pred) {
    tables().adjoints[op].push_back({side, fn, frozen, pred});
}

R97_WEAK TwinFn twin_find(const std::string& op, const std::vector<OpParam>& params, std::string* error) {
    const auto it = tables().twins.find(op);
    const TwinEntry* e =
        it == tables().twins.end() ? nullptr : pick(it->second, params, [](const TwinEntry&) { return true; });
    if (e) return e->fn;
    if (error) *error = "no twin registered for op '" + op + "' (params: " + describe(params) + ")";
    return nullptr;
}

R97_WEAK AdjointFn adjoint_find(const std::string& op, Side side, const std::vector<OpParam>& params,
                                std::string* error) {
    if (const AdjointEntry* e = adjoint_row(op, side, params)) return e->fn;
    if (error)
        *error = std::string("no ") + (side == Side::host ? "host" : "device") + " adjoint for op '" + op +
                 "' (params: " + describe(params) + ")";
    return nullptr;
}

R97_WEAK std::vector<int> adjoint_frozen(const std::string& op, Side side, const std::vector<OpParam>& params) {
    const AdjointEntry* e = adjoint_row(op, side, params);
    return e ? e->frozen : std::vector<int>{};
}

R97_WEAK std::vector<std::string> ops_registered() {
    std::map<std::string, int> names;
    for (const auto& kv : tables().twins) names[kv.first] = 1;
    for (const auto& kv : tables().adjoints) names[kv.first] = 1;
    std::vector<std::string> out;
    for (const auto& kv : names) out.push_back(kv.first);
    return out;
}

R97_WEAK OpRows op_rows(const std::string& op) {
    OpRows r;
    const auto t = tables().twins.find(op);
    r.twin = t != tables().twins.end() && !t->second.empty();
    const auto a = tables().adjoints.find(op);
    if (a == tables().adjoints.end()) return r;
    for (const AdjointEntry& e : a->second) {
        if (e.side == Side::host && !r.host_adjoint) {
            r.host_adjoint = true;
            r.host_frozen = e.frozen;
        } else if (e.side == Side::device && !r.device_adjoint) {
            r.device_adjoint = true;
            r.device_frozen = e.frozen;
        }
    }
    return r;
}

R97_WEAK const char* adjoint_family_name(AdjointFamily family) {
    switch (family) {
        case AdjointFamily::None: return "none";
        case AdjointFamily::Elementwise: return "elementwise";
        case AdjointFamily::Linear: return "linear";
        case AdjointFamily::Quant: return "quant";
        case AdjointFamily::Lora: return "lora";
        case AdjointFamily::Qk: return "qk";
        case AdjointFamily::Attention: return "attention";
        case AdjointFamily::GdnPrep: return "gdn_prep";
        case AdjointFamily::GdnKkt: return "gdn_kkt";
        case AdjointFamily::GdnScan: return "gdn_scan";
    }
    return "?";
}

R97_WEAK AdjointFamily family_find(const std::string& op) {
    const auto it = families().find(op);
    return it == families().end() ? AdjointFamily::None : it->second;
}

R97_WEAK void family_register(AdjointFamily family, std::initializer_list<const char*> ops) {
    for (const char* op : ops) {
        const auto ins = families().emplace(op, family);
        if (!ins.second && ins.first->second != family)
            throw std::logic_error(std::string("adjoint family: op '") + op + "' is claimed by two families");
    }
}

}  // namespace r97
