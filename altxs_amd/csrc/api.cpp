// Library-level entry points: ABI version and per-thread error messages.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

static thread_local char g_err[512] = "";

void altxs_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

extern "C" int32_t altxs_abi_version(void) { return ALTXS_ABI_VERSION; }

extern "C" const char* altxs_last_error(void) { return g_err; }
