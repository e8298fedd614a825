// Error channel and version of the C ABI (include/miattn.h).
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace miattn {

namespace {
thread_local char g_last_error[1024] = {0};
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

// Reads (and clears) the runtime's sticky launch error after a kernel launch.
int launch_status(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(MI_ERR_LAUNCH, "%s: HIP launch failed: %s", what, hipGetErrorString(err));
  }
  g_last_error[0] = '\0';
  return MI_OK;
}

}  // namespace miattn

extern "C" const char* mi_last_error(void) { return miattn::g_last_error; }

extern "C" int mi_abi_version(void) { return 13; }
