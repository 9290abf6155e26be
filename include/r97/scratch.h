// r97/scratch.h -- device scratch for one adjoint call, with the ledger a test reads: the
// reference's src/adjoint/device/scratch.h:15-48 contract, restated.
//
// Every device buffer a row holds for one call is scratch (uploads, outputs, a reduction's
// staging). The ledger counts what is held now, the high-water mark since the last reset and the
// number of allocations, so a test can say how much a row needed and catch one that leaked. The
// counters are process-wide, across every row and every call since the last reset.
#pragma once

#include <cstdint>

namespace r97 {
namespace device {

struct ScratchStats {
    int64_t live_bytes = 0;   // held now: zero between calls, or a row leaked
    int64_t peak_bytes = 0;   // the high-water mark of live_bytes since the last reset
    int64_t allocations = 0;  // calls to scratch_alloc that returned memory since the last reset
};

ScratchStats scratch_stats();

// Zeroes the counters. Throws std::runtime_error when scratch is still held: folding two runs'
// peaks together would hide the leak, and the live bytes are its only trace.
void scratch_reset();

// Device memory for the length of one call, 256-byte aligned. Null for a request of zero or fewer
// bytes and when the device refuses the allocation.
void* scratch_alloc(int64_t bytes);

// Returns a block from scratch_alloc. Null and pointers the ledger does not hold are ignored.
void scratch_free(void* p);

// One call's buffer, freed on every return path. One block owns one allocation: no copies, no moves.
struct ScratchBlock {
    void* p = nullptr;
    explicit ScratchBlock(int64_t bytes) : p(scratch_alloc(bytes)) {}
    ~ScratchBlock() { scratch_free(p); }
    ScratchBlock(const ScratchBlock&) = delete;
    ScratchBlock& operator=(const ScratchBlock&) = delete;
    ScratchBlock(ScratchBlock&&) = delete;
    ScratchBlock& operator=(ScratchBlock&&) = delete;
    explicit operator bool() const { return p != nullptr; }
};

}  // namespace device
}  // namespace r97
