// Error reporting and version entry points of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace nkl {

static thread_local char g_last_error[512] = "no error";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(NKL_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return NKL_OK;
}

}  // namespace nkl

extern "C" int nkl_abi_version(void) { return NKL_ABI_VERSION; }

extern "C" const char* nkl_last_error_string(void) { return nkl::g_last_error; }
