// ssa_capi.cpp -- library identification and per-thread error text of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "../../include/ssa_amd.h"

namespace {
thread_local char g_err[512] = "";
}

void ssa_set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

extern "C" const char *ssa_last_error(void) { return g_err; }

extern "C" const char *ssa_version(void) { return "ssa_amd 0.1 gfx950"; }
