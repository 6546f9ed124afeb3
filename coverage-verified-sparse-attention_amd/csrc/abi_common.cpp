// Host-side plumbing shared by every entry point: thread-local error text,
// launch checking and the ABI version.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/cvsa_hip.h"

namespace cvsa_host {

static thread_local char g_last_error[512] = "";

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return CVSA_ERR_LAUNCH;
  }
  g_last_error[0] = '\0';
  return CVSA_OK;
}

}  // namespace cvsa_host

extern "C" const char *cvsa_last_error(void) { return cvsa_host::g_last_error; }

extern "C" int cvsa_abi_version(void) { return CVSA_ABI_VERSION; }
