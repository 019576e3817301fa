// Version and status-text entry points of the C ABI.
#include "ndl_common.hpp"

extern "C" int ndl_abi_version(void) { return NDL_ABI_VERSION; }

extern "C" const char* ndl_strerror(int status) {
  switch (status) {
    case NDL_OK: return "ok";
    case NDL_ERR_INVALID_ARG: return "invalid argument";
    case NDL_ERR_UNSUPPORTED: return "unsupported dtype, head_dim, block_size or group size";
    case NDL_ERR_WORKSPACE: return "workspace missing or too small";
    case NDL_ERR_LAUNCH: return "kernel launch failed";
    case NDL_ERR_SCRATCH_LIMIT: return "shape needs more than the static decode scratch";
    case NDL_ERR_CAPTURE:
      return "first allocation-free call on this device made under stream capture";
    default: return "unknown status";
  }
}
