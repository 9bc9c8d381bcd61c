// Error reporting and version entry points of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "internal.h"

namespace bioemu {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(BIOEMU_ERR_LAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  }
  return BIOEMU_OK;
}

}  // namespace bioemu

extern "C" const char* bioemu_version(void) { return "bioemu2_mi355x 0.1 gfx950"; }

extern "C" const char* bioemu_last_error(void) { return bioemu::g_last_error; }
