// grad_stage.cpp -- the step's gradient staging on the card (r97/grad_stage.h).
//
// Layout: one arena a step. Leaves are carved out of large zero-filled f32 chunks of device memory
// in the order the rows first ask for them (each leaf 256-byte aligned, so its pointer is stable for
// the step and rows may launch into it); a chunk is added when the current one is full. A name maps
// to its leaf's chunk, offset and shape.
//
// Flush: for each chunk, one kernel rounds the chunk's used range from f32 to bf16 (round to
// nearest even, NaN quieted) into a bf16 mirror of the chunk, and one copy brings the mirror to the
// host; each leaf then adds its rounded values into the ParamSet leaf of its name (made, zeroed,
// when the step has not made it). The arena is freed at the end of every flush or discard.
//
// Every definition is weak: inside the reference's executable its own staging serves these rows too.
#include <hip/hip_runtime.h>

#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "r97/grad_stage.h"

#define R97_WEAK __attribute__((weak))

namespace r97 {
namespace device {
namespace {

constexpr int64_t kChunkFloats = int64_t(4) << 20;  // 16 MiB of f32 a chunk, or one leaf's size when larger
constexpr int64_t kAlignFloats = 64;                // 256-byte leaf alignment

__global__ void fill_zero_kernel(float* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0.0f;
}

// bf16 bits of f: the upper half rounded to nearest even; a NaN keeps its sign and upper payload,
// with the quiet bit set
__device__ uint16_t round_bf16(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

__global__ void round_kernel(const float* src, uint16_t* dst, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = round_bf16(src[i]);
}

float bf16_value(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

unsigned grid_for(int64_t n) {
    const int64_t g = (n + 255) / 256;
    return (unsigned)(g < 4096 ? (g > 0 ? g : 1) : 4096);
}

struct Chunk {
    float* f32 = nullptr;
    int64_t cap = 0;   // floats
    int64_t used = 0;  // floats handed out (with alignment)
};

struct Leaf {
    size_t chunk;
    int64_t offset, n;
    std::vector<int64_t> shape;
};

struct Arena {
    std::mutex mu;
    hipStream_t stream = nullptr;
    std::vector<Chunk> chunks;
    std::vector<std::string> order;  // leaf names in the order first asked: the flush's order
    std::unordered_map<std::string, Leaf> leaves;

    bool ready() {
        if (!stream && hipStreamCreate(&stream) != hipSuccess) stream = nullptr;
        return stream != nullptr;
    }

    // the staged leaves' f32 bytes (the chunks hold at most one chunk's worth more)
    int64_t bytes() const {
        int64_t b = 0;
        for (const auto& kv : leaves) b += kv.second.n * (int64_t)sizeof(float);
        return b;
    }

    void free_all() {
        for (Chunk& c : chunks) (void)hipFree(c.f32);
        chunks.clear();
        order.clear();
        leaves.clear();
    }

    // room for n floats: the current chunk's tail, or a new zero-filled chunk
    bool carve(int64_t n, size_t* chunk, int64_t* offset) {
        if (chunks.empty() || chunks.back().cap - chunks.back().used < n) {
            Chunk c;
            c.cap = n > kChunkFloats ? (n + kAlignFloats - 1) / kAlignFloats * kAlignFloats : kChunkFloats;
            if (hipMalloc(&c.f32, (size_t)c.cap * sizeof(float)) != hipSuccess) return false;
            hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(c.cap)), dim3(256), 0, stream, c.f32, c.cap);
            if (hipGetLastError() != hipSuccess || hipStreamSynchronize(stream) != hipSuccess) {
                (void)hipFree(c.f32);
                return false;
            }
            chunks.push_back(c);
        }
        Chunk& c = chunks.back();
        *chunk = chunks.size() - 1;
        *offset = c.used;
        c.used += (n + kAlignFloats - 1) / kAlignFloats * kAlignFloats;
        if (c.used > c.cap) c.used = c.cap;
        return true;
    }
};

Arena& arena() {
    static Arena* a = new Arena;
    return *a;
}

int64_t count_of(const std::vector<int64_t>& shape) {
    if (shape.empty()) return 0;
    int64_t n = 1;
    for (int64_t d : shape) {
        if (d <= 0) return 0;
        n *= d;
    }
    return n;
}

// the ParamSet leaf named `name`, made (zeroed, of `shape`) when absent
Param& leaf_of(ParamSet* grads, const std::string& name, const std::vector<int64_t>& shape, int64_t n) {
    for (Param& p : *grads)
        if (p.name == name) return p;
    Param p;
    p.name = name;
    p.shape = shape;
    p.value.assign((size_t)n, 0.0f);
    grads->push_back(std::move(p));
    return grads->back();
}

}  // namespace

R97_WEAK float* grad_stage_slot(const std::string& name, const std::vector<int64_t>& shape) {
    const int64_t n = count_of(shape);
    if (n <= 0) return nullptr;
    Arena& a = arena();
    std::lock_guard<std::mutex> lock(a.mu);
    const auto it = a.leaves.find(name);
    if (it != a.leaves.end())
        return it->second.shape == shape ? a.chunks[it->second.chunk].f32 + it->second.offset : nullptr;
    if (!a.ready()) return nullptr;
    size_t chunk = 0;
    int64_t offset = 0;
    if (!a.carve(n, &chunk, &offset)) return nullptr;
    a.leaves.emplace(name, Leaf{chunk, offset, n, shape});
    a.order.push_back(name);
    return a.chunks[chunk].f32 + offset;
}

R97_WEAK int64_t grad_stage_bytes() {
    Arena& a = arena();
    std::lock_guard<std::mutex> lock(a.mu);
    return a.bytes();
}

R97_WEAK bool grad_stage_flush(ParamSet* grads) {
    Arena& a = arena();
    std::lock_guard<std::mutex> lock(a.mu);
    bool ok = grads != nullptr && (a.chunks.empty() || a.ready());
    // every chunk rounded on the card and brought over in one copy
    std::vector<std::vector<uint16_t>> host(a.chunks.size());
    for (size_t c = 0; ok && c < a.chunks.size(); ++c) {
        const Chunk& ch = a.chunks[c];
        uint16_t* mirror = nullptr;
        if (hipMalloc(&mirror, (size_t)ch.used * sizeof(uint16_t)) != hipSuccess) {
            ok = false;
            break;
        }
        hipLaunchKernelGGL(round_kernel, dim3(grid_for(ch.used)), dim3(256), 0, a.stream, ch.f32, mirror, ch.used);
        host[c].resize((size_t)ch.used);
        ok = hipGetLastError() == hipSuccess &&
             hipMemcpyAsync(host[c].data(), mirror, (size_t)ch.used * sizeof(uint16_t), hipMemcpyDeviceToHost,
                            a.stream) == hipSuccess &&
             hipStreamSynchronize(a.stream) == hipSuccess;
        (void)hipFree(mirror);
    }
    if (ok) {
        for (const std::string& name : a.order) {
            const Leaf& l = a.leaves.at(name);
            Param& p = leaf_of(grads, name, l.shape, l.n);
            if (p.shape != l.shape || (int64_t)p.value.size() != l.n) {
                ok = false;  // a leaf of that name with another shape: left as it is
                continue;
            }
            const uint16_t* src = host[l.chunk].data() + l.offset;
            for (int64_t i = 0; i < l.n; ++i) p.value[(size_t)i] += bf16_value(src[i]);
        }
    }
    a.free_all();
    return ok;
}

R97_WEAK void grad_stage_discard() {
    Arena& a = arena();
    std::lock_guard<std::mutex> lock(a.mu);
    a.free_all();
}

}  // namespace device
}  // namespace r97
