// Library-wide C ABI entry points: version and thread-local error reporting.
#include <stdarg.h>
#include <stdio.h>

#include "host.h"

namespace {
thread_local char g_err[512] = "";
}

namespace sisa {
void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}
}  // namespace sisa

extern "C" int sisa_abi_version(void) { return SISA_ABI_VERSION; }

extern "C" const char* sisa_last_error(void) { return g_err; }
