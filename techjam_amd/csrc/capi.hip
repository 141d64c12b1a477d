// Version and error-string entry points of the C ABI.
#include "tj_common.h"

extern "C" int tj_abi_version(void) { return 3; }

extern "C" const char* tj_error_string(int code) {
  switch (code) {
    case TJ_OK: return "ok";
    case TJ_ERR_SHAPE: return "invalid shape or missing tensor";
    case TJ_ERR_DTYPE: return "unsupported dtype";
    case TJ_ERR_ALIGN: return "tensor not 16-byte aligned, or innermost stride != 1";
    case TJ_ERR_UNSUPPORTED: return "unsupported configuration";
    case TJ_ERR_LAUNCH: return "HIP kernel launch failed";
    case TJ_ERR_WORKSPACE: return "workspace missing or too small";
    case TJ_ERR_SCRATCH: return "request exceeds the fixed scratch of the allocation-free entry point";
    default: return "unknown error";
  }
}
