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

}  // namespace r97q
