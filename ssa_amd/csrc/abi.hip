// ABI plumbing of libssa_hip.so: version, thread-local error text, device check.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "common.h"

namespace ssa {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return SSA_OK;
  set_error("%s: %s", what, hipGetErrorString(e));
  return SSA_ERR_HIP;
}

}  // namespace ssa

extern "C" int ssa_abi_version(void) { return SSA_ABI_VERSION; }

extern "C" const char* ssa_last_error(void) { return ssa::g_last_error; }

extern "C" int ssa_device_supported(int device) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return ssa::hip_status(e, "hipGetDeviceProperties");
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}
