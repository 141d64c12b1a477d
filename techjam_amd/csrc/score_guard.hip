// Device-side score guard of the polynomial route.
//
// The reference estimates one sigma per module from 512 sampled rows
// (src/implementations/poly_guard.py:68-93), synchronises the host with
// .item(), caches it forever (src/implementations/extreme.py:299-305) and
// routes the whole layer. Here every (b, h) gets its own estimate and flag,
// written to device memory where the polynomial and exact kernels read them,
// so the route decision never leaves the GPU.
//
// Two launches. The first has one workgroup per (b, h) and 64-row block of
// the sampled query rows: the block is staged once in LDS (fp32, transposed,
// scaled), the sampled key rows stream through LDS in 64-row blocks gathered
// with 16-byte loads, each thread forms a 4x4 tile of every 64x64 score block
// and keeps running sum, sum of squares (fp64) and max |s|; the workgroup's
// three partials go to a workspace -- the caller's, or for
// tj_score_guard_noalloc a fixed array of the library. The second launch (one thread
// per (b, h)) adds the partials of a head in a fixed order -- the result does
// not depend on scheduling -- and writes the Bessel-corrected standard
// deviation, the route flag and what the attention kernels read from it.
#include <math.h>

#include <atomic>
#include <mutex>

#include "tj_common.h"

namespace tj {
namespace {

constexpr int GT = 256;
constexpr int GB = 64;     // sampled rows per LDS block
constexpr int GMAXD = 128;

struct GuardArgs {
  const void* q;
  const void* k;
  View4 vq, vk;
  int H, S, D, n;
  float scale, ceiling;
  int exact_prefix;
  const int32_t* idx;
  float* sigma;
  float* mean;
  float* smax;
  int32_t* flags;
  float* coeffs;
  int32_t* row_limit;
  int32_t* split;
};

__host__ __device__ constexpr int guard_blocks(int n) { return (n + GB - 1) / GB; }

// Stage up to GB sampled rows, transposed: dst[d][r] = src[idx[r0 + r], d] * mul,
// 16-byte (fp32) or 8-byte (fp16) gathers of four consecutive dims.
template <typename T>
__device__ __forceinline__ void stage_rows(float (*dst)[GB + 4], const T* src, const View4& vw, int b,
                                           int h, const GuardArgs& a, int r0, float mul) {
  const int rows = min(GB, a.n - r0);
  const int q4 = a.D / 4;  // four-dim groups per row
  for (int e = threadIdx.x; e < GB * q4; e += GT) {
    const int r = e / q4, d = 4 * (e % q4);
    float x[4] = {0.f, 0.f, 0.f, 0.f};
    if (r < rows) {
      int s = a.idx[r0 + r];
      s = min(max(s, 0), a.S - 1);
      const T* p = src + vw.row(b, h, s) + d;
      if constexpr (sizeof(T) == 4) {
        const float4_t v = *reinterpret_cast<const float4_t*>(p);
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = v[j] * mul;
      } else {
        const half4_t v = *reinterpret_cast<const half4_t*>(p);
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = (float)v[j] * mul;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[d + j][r] = x[j];
  }
}

template <typename T>
__global__ __launch_bounds__(GT) void score_guard_partial_kernel(GuardArgs a, double* partials) {
  __shared__ float qs[GMAXD][GB + 4];
  __shared__ float ks[GMAXD][GB + 4];
  __shared__ double red_s[GT / kWave], red_q[GT / kWave];
  __shared__ float red_m[GT / kWave];

  const int nb = guard_blocks(a.n);
  const int id = blockIdx.x;
  const int bh = id / nb, rb = id % nb;
  const int b = bh / a.H, h = bh % a.H;
  const T* qp = reinterpret_cast<const T*>(a.q);
  const T* kp = reinterpret_cast<const T*>(a.k);
  const int t = threadIdx.x;
  // Each thread owns a 4x4 tile of the 64x64 score block: rows 4*ti.., cols 4*tj..
  const int ti = t % 16;
  const int tj = t / 16;
  const int r0 = rb * GB;
  const int nr = min(GB, a.n - r0);
  stage_rows<T>(qs, qp, a.vq, b, h, a, r0, a.scale);

  float mx = 0.f;
  double dsum = 0.0, dsq = 0.0;
  for (int c0 = 0; c0 < a.n; c0 += GB) {
    const int nc = min(GB, a.n - c0);
    __syncthreads();
    stage_rows<T>(ks, kp, a.vk, b, h, a, c0, 1.f);
    __syncthreads();
    float acc[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[r][c] = 0.f;
    for (int d = 0; d < a.D; ++d) {
      const float4_t qv = *reinterpret_cast<const float4_t*>(&qs[d][4 * ti]);
      const float4_t kv = *reinterpret_cast<const float4_t*>(&ks[d][4 * tj]);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[r][c] = fmaf(qv[r], kv[c], acc[r][c]);
    }
    float sum = 0.f, sq = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (4 * ti + r < nr && 4 * tj + c < nc) {
          const float s = acc[r][c];
          sum += s;
          sq = fmaf(s, s, sq);
          mx = fmaxf(mx, fabsf(s));
        }
      }
    dsum += sum;
    dsq += sq;
  }
  // Workgroup reduction.
  for (int off = kWave / 2; off > 0; off /= 2) {
    dsum += __shfl_xor(dsum, off, kWave);
    dsq += __shfl_xor(dsq, off, kWave);
    mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
  }
  const int w = t / kWave;
  if (t % kWave == 0) {
    red_s[w] = dsum;
    red_q[w] = dsq;
    red_m[w] = mx;
  }
  __syncthreads();
  if (t == 0) {
    double s1 = 0.0, s2 = 0.0;
    float m = 0.f;
    for (int i = 0; i < GT / kWave; ++i) {
      s1 += red_s[i];
      s2 += red_q[i];
      m = fmaxf(m, red_m[i]);
    }
    partials[3 * size_t(id) + 0] = s1;
    partials[3 * size_t(id) + 1] = s2;
    partials[3 * size_t(id) + 2] = (double)m;
  }
}

__global__ __launch_bounds__(GT) void score_guard_final_kernel(GuardArgs a, const double* partials, int bhn) {
  const int bh = blockIdx.x * GT + threadIdx.x;
  if (bh >= bhn) return;
  const int nb = guard_blocks(a.n);
  double s1 = 0.0, s2 = 0.0, m = 0.0;
  for (int i = 0; i < nb; ++i) {
    const double* p = partials + 3 * (size_t(bh) * nb + i);
    s1 += p[0];
    s2 += p[1];
    m = fmax(m, p[2]);
  }
  const double cnt = (double)a.n * (double)a.n;
  double var = cnt > 1.0 ? (s2 - s1 * s1 / cnt) / (cnt - 1.0) : 0.0;
  if (var < 0.0) var = 0.0;
  const double sigma = sqrt(var);
  const bool safe = isfinite(sigma) && sigma > 0.0 && sigma <= (double)a.ceiling;
  if (a.sigma) a.sigma[bh] = (float)sigma;
  if (a.mean) a.mean[bh] = (float)(cnt > 0.0 ? s1 / cnt : 0.0);
  if (a.smax) a.smax[bh] = (float)m;
  a.flags[bh] = safe ? 1 : 0;
  if (a.coeffs) {
    const double s2h = 0.5 * sigma * sigma;
    const double g = exp(s2h);
    a.coeffs[3 * bh + 0] = (float)(g * fmax(1.0 - s2h, 1e-3));
    a.coeffs[3 * bh + 1] = (float)g;
    a.coeffs[3 * bh + 2] = (float)(0.5 * g);
  }
  if (a.row_limit) a.row_limit[bh] = safe ? min(a.exact_prefix, a.S) : a.S;
  if (a.split) a.split[bh] = safe ? 0 : 1;
}

}  // namespace
}  // namespace tj

extern "C" size_t tj_score_guard_workspace_bytes(int64_t B, int64_t H, int64_t n_samples) {
  if (B <= 0 || H <= 0 || n_samples <= 0 || n_samples >= (int64_t(1) << 30)) return 0;
  const int64_t per_block = 3 * sizeof(double);
  const int64_t blocks = tj::guard_blocks((int)n_samples);
  if (!tjh::product_below(std::numeric_limits<int64_t>::max() / per_block, {B, H, blocks})) return 0;
  return size_t(B) * size_t(H) * size_t(blocks) * per_block;
}

// Fixed scratch of tj_score_guard_noalloc: room for the partial sums of
// B * H * ceil(n_samples / 64) workgroups (three doubles each), 1 MiB -- for
// example 5461 (b, h) at 512 samples. Every device the library runs on holds
// its own copy until the process ends.
static __device__ __align__(256) double scratch[TJ_SCORE_GUARD_SCRATCH_BYTES / sizeof(double)];

namespace {

constexpr size_t kGuardScratchBytes = TJ_SCORE_GUARD_SCRATCH_BYTES;

// Argument checks and the two launches, shared by the entry point that takes
// a caller's workspace and the one that uses the library's fixed scratch.
int guard_launch(const void* q, const void* k, int dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                 const int64_t q_strides[4], const int64_t k_strides[4], float scale, const int32_t* sample_idx,
                 int64_t n_samples, float ceiling, int64_t exact_prefix, float* sigma_out, float* mean_out,
                 float* smax_out, int32_t* flags_out, float* coeffs_out, int32_t* row_limit_out,
                 int32_t* split_out, double* partials, hipStream_t stream) {
  tj::GuardArgs a;
  a.q = q; a.k = k;
  a.vq = {q_strides[0], q_strides[1], q_strides[2]};
  a.vk = {k_strides[0], k_strides[1], k_strides[2]};
  a.H = (int)H; a.S = (int)S; a.D = (int)D; a.n = (int)n_samples;
  a.scale = scale; a.ceiling = ceiling;
  a.exact_prefix = (int)(exact_prefix < 0 ? 0 : (exact_prefix > S ? S : exact_prefix));
  a.idx = sample_idx;
  a.sigma = sigma_out; a.mean = mean_out; a.smax = smax_out; a.flags = flags_out; a.coeffs = coeffs_out;
  a.row_limit = row_limit_out;
  a.split = split_out;
  const dim3 grid((unsigned)(B * H * tj::guard_blocks(a.n)));
  if (dtype == TJ_F32)
    hipLaunchKernelGGL(tj::score_guard_partial_kernel<float>, grid, dim3(tj::GT), 0, stream, a, partials);
  else
    hipLaunchKernelGGL(tj::score_guard_partial_kernel<half_t>, grid, dim3(tj::GT), 0, stream, a, partials);
  const int rc = tjh::launch_status();
  if (rc != TJ_OK) return rc;
  const int bhn = (int)(B * H);
  hipLaunchKernelGGL(tj::score_guard_final_kernel, dim3((unsigned)((bhn + tj::GT - 1) / tj::GT)), dim3(tj::GT), 0,
                     stream, a, static_cast<const double*>(partials), bhn);
  return tjh::launch_status();
}

// Checks that need no workspace; TJ_OK when the request is well formed.
int guard_check(const void* q, const void* k, int dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                const int64_t q_strides[4], const int64_t k_strides[4], const int32_t* sample_idx,
                int64_t n_samples, const int32_t* flags_out) {
  if (dtype != TJ_F32 && dtype != TJ_F16) return TJ_ERR_DTYPE;
  if (B <= 0 || H <= 0 || S <= 0 || D <= 0 || n_samples <= 0 || n_samples > S) return TJ_ERR_SHAPE;
  if (D > tj::GMAXD || D % 4 != 0) return TJ_ERR_UNSUPPORTED;
  if (!q || !k || !sample_idx || !flags_out) return TJ_ERR_SHAPE;
  if (!q_strides || !k_strides || q_strides[3] != 1 || k_strides[3] != 1) return TJ_ERR_ALIGN;
  const int64_t elt = dtype == TJ_F32 ? 4 : 2;
  // 4-dim gathers: rows must start on 4-element boundaries of aligned bases.
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k)) % (4 * elt) != 0) return TJ_ERR_ALIGN;
  for (int i = 0; i < 3; ++i)
    if (q_strides[i] % 4 != 0 || k_strides[i] % 4 != 0) return TJ_ERR_ALIGN;
  if (!tjh::product_below(int64_t(1) << 31, {B, H}) || S >= (int64_t(1) << 31)) return TJ_ERR_SHAPE;
  const size_t need = tj_score_guard_workspace_bytes(B, H, n_samples);
  if (need == 0 || !tjh::product_below(int64_t(1) << 31, {B, H, tj::guard_blocks((int)n_samples)}))
    return TJ_ERR_SHAPE;
  return TJ_OK;
}

// Device address of `scratch` per device, looked up once per device with that
// device current. In host code the array's name is only a stand-in; kernels
// and copies must be given this address.
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mutex;

int scratch_address(hipStream_t stream, double** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return TJ_ERR_LAUNCH;
  int stream_dev = dev;
  if (stream != nullptr && hipStreamGetDevice(stream, &stream_dev) != hipSuccess) return TJ_ERR_LAUNCH;
  if (stream_dev != dev) return TJ_ERR_UNSUPPORTED;  // the scratch of another device
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return TJ_ERR_LAUNCH;
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = static_cast<double*>(p);
  return TJ_OK;
}

}  // namespace

extern "C" int tj_score_guard(const void* q, const void* k, int dtype,
                              int64_t B, int64_t H, int64_t S, int64_t D,
                              const int64_t q_strides[4], const int64_t k_strides[4],
                              float scale, const int32_t* sample_idx, int64_t n_samples,
                              float ceiling, int64_t exact_prefix,
                              float* sigma_out, float* mean_out, float* smax_out, int32_t* flags_out,
                              float* coeffs_out, int32_t* row_limit_out, int32_t* split_out,
                              void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const int rc = guard_check(q, k, dtype, B, H, S, D, q_strides, k_strides, sample_idx, n_samples, flags_out);
  if (rc != TJ_OK) return rc;
  const size_t need = tj_score_guard_workspace_bytes(B, H, n_samples);
  if (workspace == nullptr || workspace_bytes < need || !tjh::aligned16(workspace)) return TJ_ERR_WORKSPACE;
  return guard_launch(q, k, dtype, B, H, S, D, q_strides, k_strides, scale, sample_idx, n_samples, ceiling,
                      exact_prefix, sigma_out, mean_out, smax_out, flags_out, coeffs_out, row_limit_out, split_out,
                      static_cast<double*>(workspace), stream);
}

extern "C" int tj_score_guard_noalloc(const void* q, const void* k, int dtype,
                                      int64_t B, int64_t H, int64_t S, int64_t D,
                                      const int64_t q_strides[4], const int64_t k_strides[4],
                                      float scale, const int32_t* sample_idx, int64_t n_samples,
                                      float ceiling, int64_t exact_prefix,
                                      float* sigma_out, float* mean_out, float* smax_out, int32_t* flags_out,
                                      float* coeffs_out, int32_t* row_limit_out, int32_t* split_out,
                                      hipStream_t stream) {
  const int rc = guard_check(q, k, dtype, B, H, S, D, q_strides, k_strides, sample_idx, n_samples, flags_out);
  if (rc != TJ_OK) return rc;
  if (tj_score_guard_workspace_bytes(B, H, n_samples) > kGuardScratchBytes) return TJ_ERR_SCRATCH;
  double* partials = nullptr;
  const int src = scratch_address(stream, &partials);
  if (src != TJ_OK) return src;
  return guard_launch(q, k, dtype, B, H, S, D, q_strides, k_strides, scale, sample_idx, n_samples, ceiling,
                      exact_prefix, sigma_out, mean_out, smax_out, flags_out, coeffs_out, row_limit_out, split_out,
                      partials, stream);
}
