// C-ABI support: thread-local error strings and launch checks.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace mxf8 {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(MXF8_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return MXF8_OK;
}

}  // namespace mxf8

extern "C" int mxf8_abi_version(void) { return 201; }

extern "C" const char* mxf8_last_error(void) { return mxf8::g_last_error; }
