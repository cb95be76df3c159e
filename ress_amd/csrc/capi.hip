// C-ABI support: thread-local error string and version.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

static thread_local char g_err[512] = "";

void ress_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

RESS_API const char* ress_last_error(void) { return g_err; }

RESS_API int ress_abi_version(void) { return 4; }
