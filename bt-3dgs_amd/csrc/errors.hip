// Per-thread error message and launch checking for the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "r2s_common.h"

namespace r2s {

namespace {
thread_local char g_message[1024] = "";
}

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_message, sizeof(g_message), fmt, ap);
  va_end(ap);
}

void clear_error() { g_message[0] = '\0'; }

int check_launch(const char *what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(err));
    return R2S_EHIP;
  }
  return R2S_OK;
}

}  // namespace r2s

extern "C" const char *r2s_last_error(void) { return r2s::g_message; }

// ABI revision of include/r2splat_hip.h.
extern "C" int r2s_abi_version(void) { return 10; }
