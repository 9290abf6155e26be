// grad_stage.cpp -- the step's gradient staging on the card (r97/grad_stage.h), restating the
// reference's src/adjoint/device/grad_stage.cpp:80-175: one f32 device block per leaf name, zeroed
// on the step's first ask, copied out at the step's end with one bf16 rounding (round to nearest
// even, NaN quieted) added into the leaf. Every definition is weak: inside the reference's
// executable its own staging serves these rows too.
#include <hip/hip_runtime.h>

#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "r97/grad_stage.h"

#define R97_WEAK __attribute__((weak))

namespace r97 {
namespace device {
namespace {

struct Block {
    std::string name;
    std::vector<int64_t> shape;
    int64_t n = 0;
    float* p = nullptr;
};

struct Stage {
    std::mutex mu;
    std::vector<Block> blocks;
    int64_t bytes = 0;
    hipStream_t stream = nullptr;
};

Stage& stage() {
    static Stage* s = new Stage;
    return *s;
}

hipStream_t stage_stream(Stage& s) {
    if (!s.stream && hipStreamCreate(&s.stream) != hipSuccess) s.stream = nullptr;
    return s.stream;
}

int64_t elements(const std::vector<int64_t>& shape) {
    if (shape.empty()) return 0;
    int64_t n = 1;
    for (int64_t d : shape) {
        if (d <= 0) return 0;
        n *= d;
    }
    return n;
}

float bf16_rounded(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) {
        u = (u | 0x00400000u) & 0xFFFF0000u;  // NaN, quieted
    } else {
        u += 0x7FFFu + ((u >> 16) & 1u);
        u &= 0xFFFF0000u;
    }
    std::memcpy(&f, &u, 4);
    return f;
}

void release(Stage& s) {
    for (Block& b : s.blocks) (void)hipFree(b.p);
    s.blocks.clear();
    s.bytes = 0;
}

}  // namespace

R97_WEAK float* grad_stage_slot(const std::string& name, const std::vector<int64_t>& shape) {
    const int64_t n = elements(shape);
    if (n <= 0) return nullptr;
    Stage& s = stage();
    std::lock_guard<std::mutex> lock(s.mu);
    for (const Block& b : s.blocks)
        if (b.name == name) return b.n == n && b.shape == shape ? b.p : nullptr;
    const hipStream_t st = stage_stream(s);
    if (!st) return nullptr;
    float* p = nullptr;
    if (hipMalloc(&p, (size_t)n * sizeof(float)) != hipSuccess) return nullptr;
    if (hipMemsetAsync(p, 0, (size_t)n * sizeof(float), st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess) {
        (void)hipFree(p);
        return nullptr;
    }
    s.blocks.push_back(Block{name, shape, n, p});
    s.bytes += n * (int64_t)sizeof(float);
    return p;
}

R97_WEAK int64_t grad_stage_bytes() {
    Stage& s = stage();
    std::lock_guard<std::mutex> lock(s.mu);
    return s.bytes;
}

R97_WEAK bool grad_stage_flush(ParamSet* grads) {
    Stage& s = stage();
    std::lock_guard<std::mutex> lock(s.mu);
    if (!grads) {
        release(s);
        return false;
    }
    const hipStream_t st = stage_stream(s);
    bool ok = st != nullptr;
    std::vector<float> f32;
    for (const Block& b : s.blocks) {
        Param* leaf = nullptr;
        for (Param& p : *grads)
            if (p.name == b.name) leaf = &p;
        if (!leaf) {
            Param p;
            p.name = b.name;
            p.shape = b.shape;
            p.value.assign((size_t)b.n, 0.0f);
            grads->push_back(std::move(p));
            leaf = &grads->back();
        }
        if (leaf->shape != b.shape || (int64_t)leaf->value.size() != b.n) {
            ok = false;
            continue;
        }
        if (!st) continue;
        f32.resize((size_t)b.n);
        if (hipMemcpyAsync(f32.data(), b.p, (size_t)b.n * sizeof(float), hipMemcpyDeviceToHost, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess) {
            ok = false;
            continue;
        }
        for (size_t i = 0; i < f32.size(); ++i) leaf->value[i] += bf16_rounded(f32[i]);
    }
    release(s);
    return ok;
}

R97_WEAK void grad_stage_discard() {
    Stage& s = stage();
    std::lock_guard<std::mutex> lock(s.mu);
    release(s);
}

}  // namespace device
}  // namespace r97
