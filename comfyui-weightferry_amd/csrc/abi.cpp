// C ABI housekeeping: version and the thread-local last-error message.
#include <stdarg.h>
#include <stdio.h>

#include "wf_common.h"

namespace {
thread_local char g_err[512] = "";
}

namespace wf {
void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}
}  // namespace wf

extern "C" int wf_abi_version(void) { return 1; }

extern "C" const char* wf_last_error(void) { return g_err; }
