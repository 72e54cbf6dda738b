// Library-level entry points of the C ABI: version and error text.
#include <hip/hip_runtime.h>

#include "flexengine_amd.h"

extern "C" int fe_version(void) { return 100; }  // 0.1.0

extern "C" const char* fe_error_string(int code) {
  switch (code) {
    case FE_OK:
      return "success";
    case FE_ERR_INVALID_ARGUMENT:
      return "invalid argument (null pointer, size, stride or alignment)";
    case FE_ERR_UNSUPPORTED:
      return "unsupported configuration (head_dim must be 64 or 128, group size <= 16, "
             "block_size a power of two)";
    case FE_ERR_WORKSPACE:
      return "workspace missing, misaligned or smaller than fe_paged_decode_workspace_size()";
    case FE_ERR_SCRATCH_LIMIT:
      return "the call needs more scratch than the 16 MiB fe_paged_decode_noalloc holds per "
             "GPU; call fe_paged_decode with a workspace instead";
    default:
      break;
  }
  if (code > 0) return hipGetErrorString((hipError_t)code);
  return "unknown error";
}
