// stored_weight.cpp -- the device store of prepared IQR weights (r97/stored_weight.h).
#include "r97/stored_weight.h"

#include <hip/hip_runtime.h>

#include <cstring>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <tuple>

namespace r97 {
namespace {

// The first and last 64 bytes of the codes and scale planes: a new weight written into the same
// buffers under the same encoding (a buffer reused after a free) differs there.
struct Print {
    uint8_t b[4][64];
};

struct Entry {
    R97Encoding enc{};  // the encoding the weight was prepared from, compared on every lookup
    Print print{};      // and its planes' print
    R97qWeight w{};
    void* stream_buf = nullptr;
    void* scale_buf = nullptr;
    int64_t bytes = 0;
};
using Key = std::tuple<const void*, const void*, int64_t, int64_t>;

struct Store {
    std::mutex mu;
    std::map<Key, Entry> weights;
    uint8_t* pinned = nullptr;  // the print's staging buffer (pinned host memory, sizeof(Print))
};

Store& store() {
    static Store* s = new Store;
    return *s;
}

void release(Entry& e) {
    if (e.stream_buf) (void)hipFree(e.stream_buf);
    if (e.scale_buf) (void)hipFree(e.scale_buf);
    e.stream_buf = e.scale_buf = nullptr;
}

[[noreturn]] void fail(const std::string& what, int64_t rows, int64_t cols) {
    throw std::runtime_error("stored IQR weight [" + std::to_string(rows) + ", " + std::to_string(cols) +
                             "]: " + what);
}

// the encodings say the same thing (field by field: the struct's padding is not compared)
bool same(const R97Encoding& a, const R97Encoding& b) {
    if (std::strncmp(a.scheme, b.scheme, R97_ENC_STR) || std::strncmp(a.transform, b.transform, R97_ENC_STR) ||
        a.n_planes != b.n_planes || a.n_planes < 0 || a.n_planes > R97_ENC_MAX_PLANES)
        return false;
    for (int i = 0; i < a.n_planes; ++i) {
        const R97EncPlane &p = a.plane[i], &q = b.plane[i];
        if (std::strncmp(p.role, q.role, R97_ENC_STR) || p.kind != q.kind || p.dtype != q.dtype ||
            p.block[0] != q.block[0] || p.block[1] != q.block[1] || p.extent[0] != q.extent[0] ||
            p.extent[1] != q.extent[1])
            return false;
    }
    return true;
}

// The description of the weight's joined device planes `raw` under `enc`, and its scale.col
// factor (device, or null).
R97IqrDecodeDesc describe(const R97Encoding* enc, const void* raw, int64_t rows, int64_t cols, const float** factor) {
    int64_t off[R97_ENC_MAX_PLANES] = {};
    if (r97_enc_plane_offsets(enc, rows, cols, off) < 0) fail("the encoding has no planes, or too many", rows, cols);
    R97IqrStoredPlane plane[R97_ENC_MAX_PLANES] = {};
    const uint8_t* base = static_cast<const uint8_t*>(raw);
    uint32_t mad_words[2] = {0, 0};
    for (int i = 0; i < enc->n_planes; ++i) {
        plane[i].data = base + off[i];
        plane[i].bytes = r97_enc_plane_bytes(&enc->plane[i], rows, cols);
        // the computed codebook's two words travel in the description by value: read them here
        if (std::strncmp(enc->plane[i].role, "trellis.mad", R97_ENC_STR) == 0 && plane[i].bytes >= 8) {
            if (hipMemcpy(mad_words, plane[i].data, sizeof mad_words, hipMemcpyDeviceToHost) != hipSuccess)
                fail("reading the trellis.mad plane failed", rows, cols);
            plane[i].data = reinterpret_cast<const uint8_t*>(mad_words);
        }
    }
    R97IqrDecodeDesc d;
    if (!r97_iqr_desc_from_encoding(enc, plane, rows, cols, &d))
        fail(std::string("the encoding (scheme '") + std::string(enc->scheme, strnlen(enc->scheme, R97_ENC_STR)) +
                 "') is not a form the decode reads, or a plane it needs is missing",
             rows, cols);
    if (!r97_iqr_scale_col(enc, plane, rows, cols, factor))
        fail("the scale.col factor is not one f32 a 128 columns beside one f32 scale a row", rows, cols);
    return d;
}

// The print of the weight's planes as they are on `stream`: every piece copied on the stream into
// the store's pinned buffer, then one synchronisation (a lookup costs one round trip, not four
// blocking copies).
Print print_of(const R97Encoding* enc, const void* raw, int64_t rows, int64_t cols, hipStream_t stream,
               uint8_t* pinned) {
    Print p{};
    int64_t off[R97_ENC_MAX_PLANES] = {};
    if (r97_enc_plane_offsets(enc, rows, cols, off) < 0) return p;
    std::memset(pinned, 0, sizeof p);
    int at = 0;
    for (int i = 0; i < enc->n_planes && at < 4; ++i) {
        const char* role = enc->plane[i].role;
        if (std::strncmp(role, "codes", R97_ENC_STR) && std::strncmp(role, "scale", R97_ENC_STR)) continue;
        const int64_t bytes = r97_enc_plane_bytes(&enc->plane[i], rows, cols);
        const int64_t n = bytes < 64 ? bytes : 64;
        const uint8_t* base = static_cast<const uint8_t*>(raw) + off[i];
        if (hipMemcpyAsync(pinned + 64 * at++, base, (size_t)n, hipMemcpyDeviceToHost, stream) != hipSuccess ||
            hipMemcpyAsync(pinned + 64 * at++, base + bytes - n, (size_t)n, hipMemcpyDeviceToHost, stream) != hipSuccess)
            fail("reading the planes failed", rows, cols);
    }
    if (hipStreamSynchronize(stream) != hipSuccess) fail("reading the planes failed", rows, cols);
    std::memcpy(&p, pinned, sizeof p);
    return p;
}

}  // namespace

const R97qWeight* device_weight_get(const R97Encoding* enc, const void* raw, int64_t rows, int64_t cols,
                                    R97IqrStream stream) {
    if (enc == nullptr) fail("no encoding", rows, cols);
    if (raw == nullptr) fail("no planes", rows, cols);
    Store& s = store();
    std::lock_guard<std::mutex> lock(s.mu);
    const Key key{enc, raw, rows, cols};
    if (!s.pinned && hipHostMalloc(reinterpret_cast<void**>(&s.pinned), sizeof(Print)) != hipSuccess) {
        s.pinned = nullptr;
        fail("pinned staging allocation failed", rows, cols);
    }
    const Print print = print_of(enc, raw, rows, cols, static_cast<hipStream_t>(stream), s.pinned);
    const auto it = s.weights.find(key);
    if (it != s.weights.end()) {
        if (same(it->second.enc, *enc) && std::memcmp(&it->second.print, &print, sizeof print) == 0)
            return &it->second.w;
        release(it->second);  // another weight at these addresses: prepare again
        s.weights.erase(it);
    }
    const float* factor = nullptr;
    const R97IqrDecodeDesc desc = describe(enc, raw, rows, cols, &factor);
    const int64_t sbytes = r97q_weight_stream_bytes(&desc);
    if (sbytes < 0) fail(std::string("form not served by the fused kernels: ") + r97q_last_error(), rows, cols);
    Entry e;
    e.enc = *enc;
    e.print = print;
    const int64_t tbytes = (cols / 128) * rows * 2;
    if (hipMalloc(&e.stream_buf, (size_t)sbytes) != hipSuccess || hipMalloc(&e.scale_buf, (size_t)tbytes) != hipSuccess) {
        release(e);
        fail("device allocation failed", rows, cols);
    }
    const int rc = r97q_weight_prepare(&desc, factor, static_cast<uint32_t*>(e.stream_buf),
                                       static_cast<uint16_t*>(e.scale_buf), &e.w, stream);
    if (rc != R97Q_OK || hipStreamSynchronize(static_cast<hipStream_t>(stream)) != hipSuccess) {
        const std::string msg = rc != R97Q_OK ? r97q_last_error() : "stream synchronisation failed";
        release(e);
        fail("preparation failed: " + msg, rows, cols);
    }
    e.bytes = sbytes + tbytes;
    return &s.weights.emplace(key, e).first->second.w;
}

const R97qWeight* device_weight_find(const R97Encoding* enc, const void* raw, int64_t rows, int64_t cols) {
    if (enc == nullptr) return nullptr;
    Store& s = store();
    std::lock_guard<std::mutex> lock(s.mu);
    const auto it = s.weights.find(Key{enc, raw, rows, cols});
    return it == s.weights.end() || !same(it->second.enc, *enc) ? nullptr : &it->second.w;
}

int64_t device_weight_count() {
    Store& s = store();
    std::lock_guard<std::mutex> lock(s.mu);
    return (int64_t)s.weights.size();
}

int64_t device_weight_bytes() {
    Store& s = store();
    std::lock_guard<std::mutex> lock(s.mu);
    int64_t b = 0;
    for (const auto& kv : s.weights) b += kv.second.bytes;
    return b;
}

void device_weight_clear() {
    Store& s = store();
    std::lock_guard<std::mutex> lock(s.mu);
    for (auto& kv : s.weights) release(kv.second);
    s.weights.clear();
}

}  // namespace r97
