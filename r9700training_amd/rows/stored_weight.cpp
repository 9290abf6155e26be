// stored_weight.cpp -- the device store of prepared IQR weights (r97/stored_weight.h).
#include "r97/stored_weight.h"

#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <tuple>

namespace r97 {
namespace {

struct Entry {
    R97qWeight w{};
    void* stream_buf = nullptr;
    void* scale_buf = nullptr;
    int64_t bytes = 0;
};
using Key = std::tuple<const void*, int64_t, int64_t>;

struct Store {
    std::mutex mu;
    std::map<Key, Entry> weights;
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

}  // namespace

const R97qWeight* device_weight_get(const IqrStoredEnc* enc, int64_t rows, int64_t cols, R97IqrStream stream) {
    if (enc == nullptr) fail("no encoding", rows, cols);
    Store& s = store();
    std::lock_guard<std::mutex> lock(s.mu);
    const Key key{enc, rows, cols};
    const auto it = s.weights.find(key);
    if (it != s.weights.end()) return &it->second.w;
    if (enc->desc.rows != rows || enc->desc.cols != cols)
        fail("the description covers [" + std::to_string(enc->desc.rows) + ", " + std::to_string(enc->desc.cols) +
                 "]",
             rows, cols);
    const int64_t sbytes = r97q_weight_stream_bytes(&enc->desc);
    if (sbytes < 0) fail(std::string("form not served by the fused kernels: ") + r97q_last_error(), rows, cols);
    Entry e;
    const int64_t tbytes = (cols / 128) * rows * 2;
    if (hipMalloc(&e.stream_buf, (size_t)sbytes) != hipSuccess || hipMalloc(&e.scale_buf, (size_t)tbytes) != hipSuccess) {
        release(e);
        fail("device allocation failed", rows, cols);
    }
    const int rc = r97q_weight_prepare(&enc->desc, enc->scale_col, static_cast<uint32_t*>(e.stream_buf),
                                       static_cast<uint16_t*>(e.scale_buf), &e.w, stream);
    if (rc != R97Q_OK || hipStreamSynchronize(static_cast<hipStream_t>(stream)) != hipSuccess) {
        const std::string msg = rc != R97Q_OK ? r97q_last_error() : "stream synchronisation failed";
        release(e);
        fail("preparation failed: " + msg, rows, cols);
    }
    e.bytes = sbytes + tbytes;
    return &s.weights.emplace(key, e).first->second.w;
}

const R97qWeight* device_weight_find(const void* enc, int64_t rows, int64_t cols) {
    Store& s = store();
    std::lock_guard<std::mutex> lock(s.mu);
    const auto it = s.weights.find(Key{enc, rows, cols});
    return it == s.weights.end() ? nullptr : &it->second.w;
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
