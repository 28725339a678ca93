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

}  // namespace hn

extern "C" const char* hn_last_error(void) { return hn::g_last_error; }

extern "C" int hn_abi_version(void) { return 2; }
