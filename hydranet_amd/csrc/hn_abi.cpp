// C-ABI housekeeping: thread-local last-error string and library version.
#include <stdarg.h>
#include <stdio.h>

static thread_local char g_hn_err[512] = "";

extern "C" void hn_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_hn_err, sizeof(g_hn_err), fmt, ap);
  va_end(ap);
}

extern "C" const char* hn_last_error_string(void) { return g_hn_err; }

extern "C" int hn_abi_version(void) { return 1; }
