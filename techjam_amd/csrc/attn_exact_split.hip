// The split-score exact-attention kernel with two query blocks per wave on
// 32-key tiles (fp32 inputs, head_dim 64: the fallback heads of the guarded
// route at long sequence lengths), in a translation unit of its own so that
// it can be built with LLVM's max-ILP machine scheduler
// (-amdgpu-sched-strategy=max-ilp, techjam_amd/build.py). With five MFMAs per
// score pair that order runs it ~2.4 % faster alone and the extreme-length
// guarded step ~2.6 % faster, outputs bit-identical; the plain kernels keep
// the default scheduler, which is the faster one for them.
#include "attn_exact_kernel.h"

namespace tj {

int launch_split_wide(const AttnArgs& a, hipStream_t stream) { return launch_qb<float, 64, 2, 32>(a, stream); }

}  // namespace tj
