// Per-thread error reporting and version of the hexkv C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "hexkv_common.h"

namespace hexkv {

static thread_local char g_last_error[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char *what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(HEXKV_EHIP, "%s: %s", what, hipGetErrorString(err));
  return HEXKV_OK;
}

}  // namespace hexkv

extern "C" int hexkv_version(void) { return 100; /* 0.1.0 */ }

extern "C" const char *hexkv_last_error(void) { return hexkv::g_last_error; }
