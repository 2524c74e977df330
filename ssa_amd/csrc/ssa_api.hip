// Status plumbing shared by every entry point of libssa_hip.
#include <stdarg.h>
#include <stdio.h>

#include "ssa_common.h"

namespace ssa {

static thread_local char g_last_error[512] = "";

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SSA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return SSA_OK;
}

int reserve_lds(const void* kernel, size_t bytes, const char* what) {
  if (bytes <= 64 * 1024) return SSA_OK;
  int dev = 0, max_lds = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
    return fail(SSA_ERR_HIP, "%s: cannot query the LDS limit", what);
  if (bytes > static_cast<size_t>(max_lds))
    return fail(SSA_ERR_UNSUPPORTED, "%s: needs %zu bytes of LDS, device allows %d", what, bytes,
                max_lds);
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(bytes)) != hipSuccess)
    return fail(SSA_ERR_HIP, "%s: cannot reserve %zu bytes of LDS", what, bytes);
  return SSA_OK;
}

}  // namespace ssa

extern "C" int ssa_version(void) { return 1; }

extern "C" const char* ssa_status_str(int status) {
  switch (status) {
    case SSA_OK: return "ok";
    case SSA_ERR_INVALID_ARGUMENT: return "invalid argument";
    case SSA_ERR_UNSUPPORTED: return "unsupported shape or type";
    case SSA_ERR_WORKSPACE: return "workspace too small";
    case SSA_ERR_HIP: return "HIP runtime error";
    default: return "unknown status";
  }
}

extern "C" const char* ssa_last_error(void) { return ssa::g_last_error; }
