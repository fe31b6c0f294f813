// Library identity and error reporting of the hi2x C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace hi2x {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = 0; }

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s launch failed: %s", what, hipGetErrorString(e));
    return HI2X_ELAUNCH;
  }
  return HI2X_OK;
}

}  // namespace hi2x

extern "C" int hi2x_version(void) { return 100; }

extern "C" const char* hi2x_last_error(void) { return hi2x::g_err; }
