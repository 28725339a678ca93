// Internal helpers for the C-ABI entry points: error recording and argument
// checks. Every entry point returns 0 on success or a negative HN_E* code, and
// hn_last_error() returns the message of the most recent failure on the thread.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/hynomas_fp8.h"

namespace hn {

void set_error(const char* fmt, ...);

inline int fail(int code, const char* msg) {
    set_error("%s", msg);
    return code;
}

inline int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
        return HN_E_LAUNCH;
    }
    return HN_OK;
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Compute units of the current device (256 if the query fails).
int device_cus();

// HN_OK if the current device is a gfx950; otherwise records "<who>: ..." and
// returns HN_E_DEVICE. The architecture is looked up once per device.
int require_gfx950(const char* who);

// Grid for the streaming kernels' grid-stride loops: `per_cu` workgroups per
// CU, fewer when there is less work. A moderate resident grid walking the
// data in order sustains more HBM bandwidth on a mixed read/write stream than
// one short-lived workgroup per unit of work.
inline int64_t stream_grid(int64_t units, int per_cu) {
    const int64_t g = (int64_t)device_cus() * per_cu;
    return units < g ? units : g;
}

}  // namespace hn

#define HN_REQUIRE(cond, code, msg) \
    do {                             \
        if (!(cond)) return ::hn::fail((code), (msg)); \
    } while (0)
