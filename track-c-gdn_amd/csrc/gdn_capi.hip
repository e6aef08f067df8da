// Library-level C ABI helpers (version, error strings).
#include <hip/hip_runtime.h>
#include "../../include/gdn_hip.h"

extern "C" int gdn_abi_version(void) { return GDN_ABI_VERSION; }

extern "C" const char* gdn_error_string(int code) {
  switch (code) {
    case GDN_OK: return "ok";
    case GDN_ERR_NULL: return "a required pointer argument is NULL";
    case GDN_ERR_SHAPE: return "unsupported size or head configuration";
    case GDN_ERR_WORKSPACE: return "workspace missing or too small";
    default: break;
  }
  if (code < 0) return hipGetErrorString(static_cast<hipError_t>(-code));
  return "unknown gdn status code";
}
