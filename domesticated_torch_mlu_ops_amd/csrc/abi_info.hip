// Version and status-text entry points of libtmo_hip.so (include/tmo_hip.h).
#include "tmo_hip.h"

extern "C" int tmo_hip_abi_version(void) { return TMO_HIP_ABI_VERSION; }

extern "C" const char* tmo_hip_status_string(int status) {
  switch (status) {
    case TMO_OK: return "ok";
    case TMO_ERR_INVALID_ARGUMENT: return "invalid argument (null pointer, size or stride)";
    case TMO_ERR_UNSUPPORTED_DTYPE: return "unsupported dtype";
    case TMO_ERR_UNSUPPORTED_MODE: return "unsupported quant_mode / quant_bit";
    case TMO_ERR_LAUNCH: return "HIP kernel launch failed";
    case TMO_ERR_SCRATCH_TOO_SMALL:
      return "the call needs more than the library's static scratch "
             "(TMO_HIP_DEQUANT_SCRATCH_BYTES); pass a workspace to the allocating entry point";
    default: return "unknown status";
  }
}
