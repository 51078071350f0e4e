// Library-wide C ABI pieces: version, per-thread error message, launch check.
#include <stdarg.h>
#include <stdio.h>

#include "pkm_common.h"

namespace {
thread_local char g_last_error[1024] = "";
}

int pkm_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

// Reports a failed kernel launch (bad configuration, missing code object for
// the device) without synchronising: hipGetLastError only reads launch status.
int pkm_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return pkm_set_error(PKM_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return PKM_OK;
}

extern "C" int pkm_version(void) { return (0 << 16) | 1; }

extern "C" const char* pkm_last_error_string(void) { return g_last_error; }
