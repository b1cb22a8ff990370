// Host-side status plumbing of the C ABI: error classes and the thread-local
// message behind mxfp4_last_error().
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace mx {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return MXFP4_OK;
  set_error("%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
  return MXFP4_ERR_HIP;
}

int launch_status(const char* what) { return hip_status(hipGetLastError(), what); }

}  // namespace mx

extern "C" const char* mxfp4_last_error(void) { return mx::g_last_error; }

extern "C" int mxfp4_abi_version(void) { return MXFP4_ABI_VERSION; }
