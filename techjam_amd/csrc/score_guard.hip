// Device-side score guard of the polynomial route.
//
// The reference estimates one sigma per module from 512 sampled rows
// (src/implementations/poly_guard.py:68-93), synchronises the host with
// .item(), caches it forever (src/implementations/extreme.py:299-305) and
// routes the whole layer. Here every (b, h) gets its own estimate and flag,
// written to device memory where the polynomial and exact kernels read them,
// so the route decision never leaves the GPU.
//
// One workgroup per (b, h). The sampled rows are staged in LDS as fp32 in
// 64-row blocks, transposed so that a thread reads four rows with one 16-byte
// load; each thread forms a 4x4 tile of the 64x64 scores of a block pair and
// keeps running sum, sum of squares and max |s|; a workgroup reduction in
// fp64 produces the Bessel-corrected standard deviation.
#include <math.h>

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

// Stage up to GB sampled rows, transposed: dst[d][r] = src[idx[r0 + r], d] * mul.
template <typename T>
__device__ __forceinline__ void stage_rows(float (*dst)[GB + 4], const T* src, const View4& vw, int b,
                                           int h, const GuardArgs& a, int r0, float mul) {
  const int rows = min(GB, a.n - r0);
  for (int e = threadIdx.x; e < GB * a.D; e += GT) {
    const int r = e / a.D, d = e % a.D;
    float x = 0.f;
    if (r < rows) {
      int s = a.idx[r0 + r];
      s = min(max(s, 0), a.S - 1);
      x = (float)src[vw.row(b, h, s) + d] * mul;
    }
    dst[d][r] = x;
  }
}

template <typename T>
__global__ __launch_bounds__(GT) void score_guard_kernel(GuardArgs a) {
  __shared__ float qs[GMAXD][GB + 4];
  __shared__ float ks[GMAXD][GB + 4];
  __shared__ double red_s[GT / kWave], red_q[GT / kWave];
  __shared__ float red_m[GT / kWave];

  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh % a.H;
  const T* qp = reinterpret_cast<const T*>(a.q);
  const T* kp = reinterpret_cast<const T*>(a.k);
  const int t = threadIdx.x;
  // Each thread owns a 4x4 tile of the 64x64 score block: rows 4*ti.., cols 4*tj..
  const int ti = t % 16;
  const int tj = t / 16;

  float mx = 0.f;
  double dsum = 0.0, dsq = 0.0;
  for (int r0 = 0; r0 < a.n; r0 += GB) {
    const int nr = min(GB, a.n - r0);
    for (int c0 = 0; c0 < a.n; c0 += GB) {
      const int nc = min(GB, a.n - c0);
      __syncthreads();
      stage_rows<T>(qs, qp, a.vq, b, h, a, r0, a.scale);
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
    const double cnt = (double)a.n * (double)a.n;
    double var = cnt > 1.0 ? (s2 - s1 * s1 / cnt) / (cnt - 1.0) : 0.0;
    if (var < 0.0) var = 0.0;
    const double sigma = sqrt(var);
    const bool safe = isfinite(sigma) && sigma > 0.0 && sigma <= (double)a.ceiling;
    if (a.sigma) a.sigma[bh] = (float)sigma;
    if (a.mean) a.mean[bh] = (float)(cnt > 0.0 ? s1 / cnt : 0.0);
    if (a.smax) a.smax[bh] = m;
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
}

}  // namespace
}  // namespace tj

extern "C" int tj_score_guard(const void* q, const void* k, int dtype,
                              int64_t B, int64_t H, int64_t S, int64_t D,
                              const int64_t q_strides[4], const int64_t k_strides[4],
                              float scale, const int32_t* sample_idx, int64_t n_samples,
                              float ceiling, int64_t exact_prefix,
                              float* sigma_out, float* mean_out, float* smax_out, int32_t* flags_out,
                              float* coeffs_out, int32_t* row_limit_out, int32_t* split_out,
                              hipStream_t stream) {
  if (dtype != TJ_F32 && dtype != TJ_F16) return TJ_ERR_DTYPE;
  if (B <= 0 || H <= 0 || S <= 0 || D <= 0 || n_samples <= 0 || n_samples > S) return TJ_ERR_SHAPE;
  if (D > tj::GMAXD) return TJ_ERR_UNSUPPORTED;
  if (!q || !k || !sample_idx || !flags_out) return TJ_ERR_SHAPE;
  if (!q_strides || !k_strides || q_strides[3] != 1 || k_strides[3] != 1) return TJ_ERR_ALIGN;
  if (B * H >= (int64_t(1) << 31) || S >= (int64_t(1) << 31)) return TJ_ERR_SHAPE;
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
  const dim3 grid((unsigned)(B * H));
  if (dtype == TJ_F32)
    hipLaunchKernelGGL(tj::score_guard_kernel<float>, grid, dim3(tj::GT), 0, stream, a);
  else
    hipLaunchKernelGGL(tj::score_guard_kernel<half_t>, grid, dim3(tj::GT), 0, stream, a);
  return tjh::launch_status();
}
