// Library-level entry points of the C ABI (status text, ABI version).
#include "common.h"

extern "C" const char* omni_status_string(int status) {
  switch (status) {
    case OMNI_OK: return "ok";
    case OMNI_ERR_INVALID: return "invalid argument (null pointer, negative size, misaligned or short stride)";
    case OMNI_ERR_DTYPE: return "unsupported element type";
    case OMNI_ERR_SHAPE: return "shape outside what the kernels cover (head_dim, tokens, window)";
    case OMNI_ERR_WORKSPACE: return "workspace too small or not 256-byte aligned";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown status";
}

extern "C" int omni_abi_version(void) { return 3; }
