// scratch.cpp -- the device scratch ledger (r97/scratch.h) over hipMalloc / hipFree.
//
// The reference takes its scratch from radiance's device layer (src/adjoint/device/scratch.cpp);
// radiance is absent here, so the blocks come from the HIP runtime (hipMalloc aligns to 256 bytes,
// the alignment the contract promises). A block is recorded with its size when handed out and
// dropped when returned; the counters move under one mutex.
//
// Every definition is weak: linked into the reference's executable, its own ledger serves these
// rows too, and a test there sees their scratch in the same counters.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>

#include "r97/scratch.h"

#define R97_WEAK __attribute__((weak))

namespace r97 {
namespace device {
namespace {

struct Ledger {
    std::mutex mu;
    std::unordered_map<void*, int64_t> held;
    ScratchStats stats;
};

Ledger& ledger() {
    static Ledger* l = new Ledger;  // never destroyed: rows may return blocks during static teardown
    return *l;
}

}  // namespace

R97_WEAK ScratchStats scratch_stats() {
    Ledger& l = ledger();
    std::lock_guard<std::mutex> lock(l.mu);
    return l.stats;
}

R97_WEAK void scratch_reset() {
    Ledger& l = ledger();
    std::lock_guard<std::mutex> lock(l.mu);
    if (l.stats.live_bytes != 0)
        throw std::runtime_error("device scratch: " + std::to_string(l.stats.live_bytes) +
                                 " bytes still held; the row that took them leaked");
    l.stats = ScratchStats{};
}

R97_WEAK void* scratch_alloc(int64_t bytes) {
    if (bytes <= 0) return nullptr;
    void* p = nullptr;
    if (hipMalloc(&p, (size_t)bytes) != hipSuccess) {
        (void)hipGetLastError();  // the failure is the null return, not a sticky error for the next call
        return nullptr;
    }
    Ledger& l = ledger();
    std::lock_guard<std::mutex> lock(l.mu);
    l.held[p] = bytes;
    l.stats.live_bytes += bytes;
    l.stats.peak_bytes = std::max(l.stats.peak_bytes, l.stats.live_bytes);
    ++l.stats.allocations;
    return p;
}

R97_WEAK void scratch_free(void* p) {
    if (!p) return;
    {
        Ledger& l = ledger();
        std::lock_guard<std::mutex> lock(l.mu);
        auto it = l.held.find(p);
        if (it == l.held.end()) return;
        l.stats.live_bytes -= it->second;
        l.held.erase(it);
    }
    (void)hipFree(p);
}

}  // namespace device
}  // namespace r97
