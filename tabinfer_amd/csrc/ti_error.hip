// ti_error.hip — the thread-local last-error text behind ti_last_error (host code only;
// plain C++, so the sanitizer tests compile it with the .cpu.bin reader).
#include "ti_host.h"
#include <stdarg.h>
#include <stdio.h>

static thread_local char g_err[512] = "";

extern "C" const char* ti_last_error(void) { return g_err; }

int ti_fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}
