// Thread-local error text for the C ABI (sc_last_error).
#include <stdarg.h>
#include <stdio.h>

#include "sc_common.h"

static thread_local char g_last_error[512] = "";

void sc_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int sc_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

extern "C" const char* sc_last_error(void) { return g_last_error; }
extern "C" int sc_abi_version(void) { return SC_ABI_VERSION; }
