// Library-wide C ABI pieces: thread-local error message and ABI version.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

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

int require_gfx950(const char* who) {
    // 0: not looked up yet; 1: gfx950; -1: another architecture
    static int arch[64] = {};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
        (void)hipGetLastError();
        set_error("%s: no HIP device is available", who);
        return HN_E_DEVICE;
    }
    if (dev < 64 && arch[dev] != 0) {
        if (arch[dev] > 0) return HN_OK;
    } else {
        hipDeviceProp_t prop;
        const bool ok = hipGetDeviceProperties(&prop, dev) == hipSuccess &&
                        strncmp(prop.gcnArchName, "gfx950", 6) == 0 &&
                        (prop.gcnArchName[6] == '\0' || prop.gcnArchName[6] == ':');
        if (dev < 64) arch[dev] = ok ? 1 : -1;
        if (ok) return HN_OK;
    }
    set_error("%s: device %d is not a gfx950 (MI355X); the kernels are built for gfx950 only", who, dev);
    return HN_E_DEVICE;
}

}  // namespace hn

extern "C" const char* hn_last_error(void) { return hn::g_last_error; }

extern "C" int hn_abi_version(void) { return 4; }
