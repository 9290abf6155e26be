// status.h -- the calling thread's last failure message, shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/r97q.h"

namespace r97q {

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Record a HIP runtime failure of `what` and return R97Q_ELAUNCH (or R97Q_OK when `e` is success).
inline int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return R97Q_OK;
    set_error("%s: %s", what, hipGetErrorString(e));
    return R97Q_ELAUNCH;
}

// The launch just issued on this thread: hipGetLastError after a <<<>>> launch.
inline int launch_status(const char* kernel) { return hip_status(hipGetLastError(), kernel); }

// The description's rules (src/iqr_decode.h:321-349): 0 when valid.
int32_t validate(const R97IqrDecodeDesc& d);

// Rows [d.row0, d.row0 + d.rows) of a valid description decoded into the int8-code form at
// d.out_codes (units from row row0) and d.out_scale ([cols/128][scale_ld]) (decode.hip).
int decode_tiled(const R97IqrDecodeDesc& d, int64_t scale_ld, hipStream_t s);
// n descriptions at once (one launch when they allow it), each as decode_tiled decodes it
int decode_tiled_batch(const R97IqrDecodeDesc* ds, int n, int64_t scale_ld, hipStream_t s);

}  // namespace r97q
