// r97/stored_weight.h -- the stored IQR weights the device rows read, prepared once per weight.
//
// The reference keeps a store of host-decoded grids keyed by (encoding, rows, cols)
// (src/stored_weight.h:27-55: stored_weight_put / _find / _count / _bytes / _clear), so its host
// rows can read a weight the engine holds in its own stored layout. This build's rows read the
// weight on the card instead, in the column-stream form the fused kernels decode in their
// mainloop (include/r97q.h, r97q_weight_prepare): the store here holds that form, keyed the same
// way, and is filled on a row's first use of a weight. Pointers it returns stay valid until
// device_weight_clear(); the walk that calls the rows is single-threaded, a mutex guards the map.
#pragma once

#include <cstdint>

#include "r97q.h"

namespace r97 {

// What AdValue::enc points at for a stored IQR weight in this build: the description of its
// planes (device pointers, rows_all x cols) and the optional f32 `scale.col` factor (device,
// cols/128 values; null when the weight has none).
struct IqrStoredEnc {
    R97IqrDecodeDesc desc;
    const float* scale_col = nullptr;
};

// The prepared weight `enc` names at [rows, cols]; prepares it (device memory, one
// r97q_weight_prepare on `stream`, synchronised) on first use. Throws std::runtime_error when the
// form is one the fused kernels do not serve or the preparation fails.
const R97qWeight* device_weight_get(const IqrStoredEnc* enc, int64_t rows, int64_t cols, R97IqrStream stream);
// The prepared weight, or null when no row prepared it yet.
const R97qWeight* device_weight_find(const void* enc, int64_t rows, int64_t cols);
int64_t device_weight_count();
int64_t device_weight_bytes();  // device bytes the store holds
void device_weight_clear();     // frees every prepared weight

}  // namespace r97
