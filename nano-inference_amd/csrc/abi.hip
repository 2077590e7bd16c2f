// Library-wide entry points of the C ABI: version and status names.
#include "common.h"

extern "C" int32_t nia_abi_version(void) { return 3; }

extern "C" const char* nia_error_string(int32_t status) {
  switch (status) {
    case NIA_OK:
      return "ok";
    case NIA_ERR_INVALID_ARGUMENT:
      return "invalid argument (null pointer, negative size or inconsistent stride)";
    case NIA_ERR_UNSUPPORTED:
      return "unsupported shape or dtype for the gfx950 attention kernels";
    case NIA_ERR_WORKSPACE:
      return "workspace missing or smaller than required";
    case NIA_ERR_LAUNCH:
      return "HIP kernel launch failed";
    case NIA_ERR_MISALIGNED:
      return "pointer or stride not aligned for 16-byte vector access";
    case NIA_ERR_SCRATCH_LIMIT:
      return "the call needs more scratch than the library's fixed decode array holds";
    default:
      return "unknown status";
  }
}
