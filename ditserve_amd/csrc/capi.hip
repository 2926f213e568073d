// C-ABI plumbing: per-thread error message, version, launch checks.
#include <stdarg.h>
#include <stdio.h>

#include "ditk_common.h"

namespace {
thread_local char g_err[512] = "";
}

void ditk_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int ditk_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    ditk_set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return 2;
  }
  return 0;
}

DITK_EXPORT const char* ditk_last_error(void) { return g_err; }

DITK_EXPORT int ditk_version(void) { return 1; }
