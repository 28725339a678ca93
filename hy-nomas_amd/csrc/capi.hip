// Library-wide C ABI pieces: thread-local error message and ABI version.
#include <stdarg.h>
#include <stdio.h>

#include "hn_capi_internal.h"

namespace hn {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
}

int device_cus() {
    static int cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] <= 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
            v = 256;
        cached[dev] = v;
    }
    return cached[dev];
}

}  // namespace hn

extern "C" const char* hn_last_error(void) { return hn::g_last_error; }

extern "C" int hn_abi_version(void) { return 3; }
