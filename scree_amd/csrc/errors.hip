// Error reporting for the C ABI: a thread-local message behind scree_last_error().
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace scree {

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
    return set_error(SCREE_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  }
  return SCREE_OK;
}

}  // namespace scree

extern "C" int scree_abi_version(void) { return SCREE_ABI_VERSION; }

extern "C" const char* scree_last_error(void) { return scree::g_last_error; }
