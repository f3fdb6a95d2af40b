// Host-side status reporting and device queries for the C ABI.
#include <stdarg.h>
#include <stdio.h>


#include "common.hpp"

namespace ts_host {

static thread_local char g_last_error[512] = "no error";

ts_status fail(ts_status code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

ts_status check_launch(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(TS_ERR_LAUNCH, "%s: launch failed: %s", kernel, hipGetErrorString(e));
  }
  return TS_OK;
}

}  // namespace ts_host

extern "C" const char* ts_last_error(void) { return ts_host::g_last_error; }

extern "C" const char* ts_version(void) { return "trainscale_amd 0.1.0 gfx950"; }
