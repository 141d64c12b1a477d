// Polynomial linear attention (placeholder until the kernels land).
#include "tj_common.h"

extern "C" size_t tj_poly_workspace_bytes(int64_t, int64_t, int64_t, int64_t, int64_t) { return 0; }

extern "C" int tj_poly_attn_fwd(const void*, const void*, const void*, void*, int, int64_t, int64_t,
                                int64_t, int64_t, const int64_t*, const int64_t*, const int64_t*,
                                const int64_t*, float, int64_t, int64_t, const float*, const int32_t*,
                                void*, size_t, hipStream_t) {
  return TJ_ERR_UNSUPPORTED;
}
