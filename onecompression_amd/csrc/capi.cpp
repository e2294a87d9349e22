// Error plumbing and version entry points of the C ABI.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "oc_common.h"

namespace oc {

static thread_local char g_msg[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(hipError_t e, const char* what) {
  return set_error(OC_ERR_HIP, "%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
}

}  // namespace oc

extern "C" int oc_abi_version(void) { return OC_ABI_VERSION; }

extern "C" const char* oc_last_error(void) { return oc::g_msg; }
