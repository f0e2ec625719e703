// Library-wide ABI pieces: version, thread-local last-error message, launch checks.
#include <stdarg.h>
#include <stdio.h>

#include "mi_common.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace mi {

int32_t fail(int32_t code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int32_t ok() {
  g_last_error[0] = '\0';
  return MI_OK;
}

int32_t check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(MI_ERR_DEVICE, "%s: %s", what, hipGetErrorString(err));
  return ok();
}

}  // namespace mi

extern "C" int32_t mi_abi_version(void) { return MI_PAGED_ABI_VERSION; }

extern "C" const char* mi_last_error(void) { return g_last_error; }
