// C-ABI plumbing: thread-local last-error message and the HIP launch check shared by every entry point.
#include <stdarg.h>
#include <stdio.h>

#include "splat_common.h"

namespace splat {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(kHipError, "%s: %s", what, hipGetErrorString(e));
  return kOk;
}

}  // namespace splat

extern "C" {

const char* splat_last_error(void) { return splat::g_last_error; }

int splat_abi_version(void) { return 3; }

}  // extern "C"
