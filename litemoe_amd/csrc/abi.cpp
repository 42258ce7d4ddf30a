// Version and status strings of the C ABI, and the device address of pinned
// host memory.
#include <hip/hip_runtime.h>

#include "../../include/litemoe_amd.h"

extern "C" const char *lm_version(void) { return "litemoe_amd 0.1.0 gfx950"; }

extern "C" const char *lm_status_string(int status) {
  switch (status) {
    case LM_OK: return "ok";
    case LM_EINVAL: return "invalid argument";
    case LM_EUNSUPPORTED: return "unsupported shape";
    case LM_ELAUNCH: return "kernel launch failed";
    case LM_EWORKSPACE: return "workspace too small";
    case LM_ETOOLARGE: return "problem exceeds the static no-allocation scratch";
    default: return "unknown status";
  }
}

extern "C" int lm_host_device_pointer(void *host, void **device) {
  if (!host || !device) return LM_EINVAL;
  *device = nullptr;
  return hipHostGetDevicePointer(device, host, 0) == hipSuccess ? LM_OK : LM_EINVAL;
}
