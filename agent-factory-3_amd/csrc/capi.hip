// Error reporting and version query shared by every exported entry point.
// Each entry point returns 0 on success, a negative AF3_E* code for an argument
// error, or a positive hipError_t; the message is kept per host thread
// (forward runs on the caller's thread, backward on the autograd thread).
#include <stdarg.h>
#include <stdio.h>

#include "af3_common.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace af3 {

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

}  // namespace af3

extern "C" int af3_abi_version(void) { return AF3_ABI_VERSION; }

extern "C" const char* af3_last_error(void) { return g_last_error; }
