// Error state and version of the C ABI (include/dimq_hip.h).
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace dimq {

namespace {
thread_local char g_last_error[512] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(DIMQ_ERR_HIP, "%s: HIP launch failed: %s", what, hipGetErrorString(e));
  return DIMQ_OK;
}

}  // namespace dimq

extern "C" const char* dimq_last_error(void) { return dimq::g_last_error; }

extern "C" int dimq_abi_version(void) { return 2; }
