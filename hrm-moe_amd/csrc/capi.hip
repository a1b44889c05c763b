// Library-level entry points of the C ABI (version and status strings).
#include "common.h"

extern "C" int hrm_moe_abi_version(void) { return HRM_MOE_ABI_VERSION; }

extern "C" const char* hrm_moe_status_string(int status) {
  switch (status) {
    case HRM_MOE_OK: return "ok";
    case HRM_MOE_ERR_INVALID: return "invalid argument (null pointer, negative or inconsistent size)";
    case HRM_MOE_ERR_DTYPE: return "dtype not supported by this entry point";
    case HRM_MOE_ERR_UNSUPPORTED: return "shape outside the kernel limits";
    case HRM_MOE_ERR_WORKSPACE: return "workspace missing or too small";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown status";
}
