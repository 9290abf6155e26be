// r97/stored_weight.h -- the stored IQR weights the device rows read, prepared once per weight.
//
// The reference keeps a store of host-decoded grids keyed by (encoding, rows, cols)
// (src/stored_weight.h:27-55: stored_weight_put / _find / _count / _bytes / _clear), so its host
// rows can read a weight the engine holds in its own stored layout. This build's rows read the
// weight on the card instead, in the form the fused kernels decode in their mainloop
// (include/r97q.h, r97q_weight_prepare): the store here holds that form, filled on a row's first use
// of a weight.
//
// A stored operand arrives as the reference's tape hands one (include/r97/adjoint.h, AdValue): `enc`
// is its encoding (here an R97Encoding, include/r97q.h) and `raw` its planes joined in one device
// buffer at the offsets r97_enc_plane_offsets gives. The row derives the decode's description from
// the encoding's plane roles (r97_iqr_desc_from_encoding, the rules of src/iqr_form.h:87-217).
//
// An entry is keyed by (enc, raw, rows, cols) and keeps a copy of the encoding it was prepared from
// and a print of its planes (the first and last 64 bytes of the codes and scale planes): a lookup
// whose encoding or print no longer matches (an encoding rebuilt, or another weight written, at
// reused addresses) prepares the weight again; the print costs one pinned round trip a lookup (its
// pieces copied on the row's stream, one synchronisation). Bytes changed elsewhere in the planes
// are not seen: a frozen weight keeps its planes, so entries persist across steps and a walk needs
// no clear at a step's end (the reference's walk clears its host store there, stored_weight_clear,
// src/step_device.cpp:1621; device_weight_clear is for a caller that wants the memory back).
// The functions are this build's own (device_weight_*), not the reference's host-store API: its
// store holds host grids for host rows, this one the card's prepared form. Pointers the store
// returns stay valid until the entry is replaced or cleared; a mutex guards the map.
#pragma once

#include <cstdint>

#include "r97q.h"

namespace r97 {

// The prepared weight the stored operand (enc, raw) names at [rows, cols]; prepares it (device
// memory, one r97q_weight_prepare on `stream`, synchronised) on first use. Throws
// std::runtime_error when the encoding is not a form the decode reads, the kernels do not serve it,
// or the preparation fails.
const R97qWeight* device_weight_get(const R97Encoding* enc, const void* raw, int64_t rows, int64_t cols,
                                    R97IqrStream stream);
// The prepared weight, or null when no row prepared it (or its encoding no longer matches; the
// print is not read here).
const R97qWeight* device_weight_find(const R97Encoding* enc, const void* raw, int64_t rows, int64_t cols);
int64_t device_weight_count();
int64_t device_weight_bytes();  // device bytes the store holds
void device_weight_clear();     // frees every prepared weight

}  // namespace r97
