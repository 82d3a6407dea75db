// Error reporting and version of the C ABI (include/ava.h).
#include <stdarg.h>
#include <string.h>

#include "common.h"

namespace {
thread_local char g_err[512] = "";
}

namespace ava {

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

}  // namespace ava

extern "C" const char *ava_last_error(void) { return g_err; }

extern "C" const char *ava_version(void) { return "ava_amd 0.1 (gfx950)"; }
