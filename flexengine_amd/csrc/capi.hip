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
      return "unsupported configuration (head_dim 1-512, decode group size <= 128, "
             "group size * head_dim <= 8192, block_size a power of two; no plan or "
             "key-split prefix pass outside head_dim 64 / 128 with groups <= 16)";
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
