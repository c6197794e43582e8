// Library-level C-ABI helpers: version and error text.
#include "oa_common.h"

extern "C" int oa_abi_version(void) { return OA_ABI_VERSION; }

extern "C" const char* oa_error_string(int status) {
  if (status == 0) return "success";
  if (status == OA_EINVAL) return "invalid argument (shape, stride, size or pointer check failed)";
  if (status == OA_ENOSPC) return "request exceeds the fixed device scratch area of this entry point";
  return hipGetErrorString((hipError_t)status);
}
