// Fused elementwise tails of the encoder block (torch_transformer_benchmark.py:
// 116-121, 140-145): the bias of a bias-free projection GEMM, the residual add,
// exact GELU and the zeroing of padded rows, each done in one pass over the
// activation instead of two or three.
//
//   tj_bias_residual : out = x + (row valid ? y + b : 0)          (mode 1)
//                      out = row valid ? x + y + b : 0             (mode 2)
//                      out = x + y + b                             (mode 0)
//   tj_bias_gelu     : y = gelu(y + b), exact (erf) form, in place -- or
//                      written as fp16 to a separate buffer, the operand of
//                      the next GEMM when GEMMs take fp16 operands
//   tj_bias_relu     : y = max(y + b, 0), the same two output forms (the
//                      post-norm / ReLU block variant)
//   tj_bias_residual_layernorm : one of the residual forms above, and in the
//                      same pass n = LayerNorm(out) (the next block's norm, or
//                      the final one), so that the norm does not read the
//                      residual stream again; n in fp32 or fp16. out may be
//                      null when only n is wanted: in a post-norm block the
//                      norm of the sum is the new residual stream
//
// Tensors are fp32 [rows, cols] row-major with cols % 4 == 0 and 16-byte
// aligned bases; row r = b * seq_len + s is valid iff s < valid_len[b].
#include "tj_common.h"

namespace tj {
namespace {

constexpr int ET = 256;

__device__ __forceinline__ bool row_valid(int64_t row, int64_t seq_len, const int32_t* valid_len) {
  if (valid_len == nullptr) return true;
  const int64_t b = row / seq_len, s = row % seq_len;
  return s < (int64_t)valid_len[b];
}

// Four consecutive values to element 4i of an fp32 or fp16 array.
__device__ __forceinline__ void store4(float* p, int64_t i, float4_t v) { reinterpret_cast<float4_t*>(p)[i] = v; }
__device__ __forceinline__ void store4(half_t* p, int64_t i, float4_t v) {
  reinterpret_cast<half4_t*>(p)[i] = half4_t{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
}

__global__ __launch_bounds__(ET) void bias_residual_kernel(float* out, const float* x, const float* y, const float* bias,
                                                           int64_t n4, int64_t c4, int64_t seq_len,
                                                           const int32_t* valid_len, int mode) {
  for (int64_t i = blockIdx.x * (int64_t)ET + threadIdx.x; i < n4; i += (int64_t)gridDim.x * ET) {
    const int64_t row = i / c4, c = i % c4;
    const float4_t xv = reinterpret_cast<const float4_t*>(x)[i];
    const float4_t yv = reinterpret_cast<const float4_t*>(y)[i];
    const float4_t bv = reinterpret_cast<const float4_t*>(bias)[c];
    const bool ok = mode == 0 || row_valid(row, seq_len, valid_len);
    float4_t r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float t = yv[e] + bv[e];
      r[e] = mode == 2 ? (ok ? xv[e] + t : 0.f) : xv[e] + (ok ? t : 0.f);
    }
    reinterpret_cast<float4_t*>(out)[i] = r;
  }
}

enum Act { ACT_GELU, ACT_RELU };

template <Act A>
__device__ __forceinline__ float activate(float t) {
  if constexpr (A == ACT_GELU) return 0.5f * t * (1.f + erff(t * 0.70710678118654752f));
  else return t > 0.f ? t : 0.f;
}

template <Act A, typename TO>
__global__ __launch_bounds__(ET) void bias_act_kernel(float* y, TO* out, const float* bias, int64_t n4, int64_t c4) {
  for (int64_t i = blockIdx.x * (int64_t)ET + threadIdx.x; i < n4; i += (int64_t)gridDim.x * ET) {
    const int64_t c = i % c4;
    float4_t v = reinterpret_cast<const float4_t*>(y)[i];
    const float4_t bv = reinterpret_cast<const float4_t*>(bias)[c];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = activate<A>(v[e] + bv[e]);
    store4(out, i, v);
  }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// One wave per row of N4 * 256 columns: lane l holds float4 columns l + 64 j.
// The mean and the (biased) variance are two exact passes over the row held
// in registers, as torch.nn.LayerNorm defines them.
template <int N4, typename TN>
__global__ __launch_bounds__(ET) void bias_residual_ln_kernel(float* out, TN* ln_out, const float* x, const float* y,
                                                              const float* bias, const float* gamma, const float* beta,
                                                              int64_t rows, int64_t seq_len, const int32_t* valid_len,
                                                              int mode, float eps, int zero_ln_padded) {
  const int lane = threadIdx.x % 64;
  const int64_t row = blockIdx.x * (int64_t)(ET / 64) + threadIdx.x / 64;
  if (row >= rows) return;
  constexpr int C4 = N4 * 64;  // float4 columns per row
  const bool ok = mode == 0 || row_valid(row, seq_len, valid_len);
  const float4_t* xr = reinterpret_cast<const float4_t*>(x) + row * C4;
  const float4_t* yr = reinterpret_cast<const float4_t*>(y) + row * C4;
  float4_t r[N4];
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < N4; ++j) {
    const int c = lane + 64 * j;
    const float4_t xv = xr[c], yv = yr[c];
    const float4_t bv = reinterpret_cast<const float4_t*>(bias)[c];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float t = yv[e] + bv[e];
      r[j][e] = mode == 2 ? (ok ? xv[e] + t : 0.f) : xv[e] + (ok ? t : 0.f);
      sum += r[j][e];
    }
    if (out != nullptr) reinterpret_cast<float4_t*>(out)[row * C4 + c] = r[j];
  }
  const float mean = wave_sum(sum) / (float)(C4 * 4);
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < N4; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float d = r[j][e] - mean;
      sq += d * d;
    }
  const float rstd = 1.f / sqrtf(wave_sum(sq) / (float)(C4 * 4) + eps);
  const bool zero = zero_ln_padded != 0 && !row_valid(row, seq_len, valid_len);
#pragma unroll
  for (int j = 0; j < N4; ++j) {
    const int c = lane + 64 * j;
    const float4_t gv = reinterpret_cast<const float4_t*>(gamma)[c];
    const float4_t hv = reinterpret_cast<const float4_t*>(beta)[c];
    float4_t n;
#pragma unroll
    for (int e = 0; e < 4; ++e) n[e] = zero ? 0.f : (r[j][e] - mean) * rstd * gv[e] + hv[e];
    store4(ln_out, row * C4 + c, n);
  }
}

// Element counts above this are refused (far beyond any device memory), so
// byte counts of the operands fit 64 bits.
constexpr int64_t kMaxElements = int64_t(1) << 56;

// Rows of 32, 64 or 128 columns: LPR = cols / 4 lanes per row (one float4
// each), 64 / LPR rows per wave, the mean and variance reduced over the row's
// lane group with xor shuffles (offsets below LPR stay inside the group).
// Same two exact passes as above.
template <int LPR, typename TN>
__global__ __launch_bounds__(ET) void bias_residual_ln_small_kernel(float* out, TN* ln_out, const float* x,
                                                                    const float* y, const float* bias,
                                                                    const float* gamma, const float* beta,
                                                                    int64_t rows, int64_t seq_len,
                                                                    const int32_t* valid_len, int mode, float eps,
                                                                    int zero_ln_padded) {
  constexpr int RPW = kWave / LPR;
  const int lane = threadIdx.x % kWave;
  const int c = lane % LPR;
  const int64_t row = (blockIdx.x * (int64_t)(ET / kWave) + threadIdx.x / kWave) * RPW + lane / LPR;
  const bool live = row < rows;  // every lane stays for the shuffles
  const bool ok = live && (mode == 0 || row_valid(row, seq_len, valid_len));
  float4_t r = {0.f, 0.f, 0.f, 0.f};
  float sum = 0.f;
  if (live) {
    const float4_t xv = reinterpret_cast<const float4_t*>(x)[row * LPR + c];
    const float4_t yv = reinterpret_cast<const float4_t*>(y)[row * LPR + c];
    const float4_t bv = reinterpret_cast<const float4_t*>(bias)[c];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float t = yv[e] + bv[e];
      r[e] = mode == 2 ? (ok ? xv[e] + t : 0.f) : xv[e] + (ok ? t : 0.f);
      sum += r[e];
    }
    if (out != nullptr) reinterpret_cast<float4_t*>(out)[row * LPR + c] = r;
  }
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) sum += __shfl_xor(sum, o, kWave);
  const float mean = sum / (float)(LPR * 4);
  float sq = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float d = r[e] - mean;
    sq += d * d;
  }
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) sq += __shfl_xor(sq, o, kWave);
  if (!live) return;
  const float rstd = 1.f / sqrtf(sq / (float)(LPR * 4) + eps);
  const bool zero = zero_ln_padded != 0 && !row_valid(row, seq_len, valid_len);
  const float4_t gv = reinterpret_cast<const float4_t*>(gamma)[c];
  const float4_t hv = reinterpret_cast<const float4_t*>(beta)[c];
  float4_t n;
#pragma unroll
  for (int e = 0; e < 4; ++e) n[e] = zero ? 0.f : (r[e] - mean) * rstd * gv[e] + hv[e];
  store4(ln_out, row * LPR + c, n);
}

unsigned grid_for(int64_t n4) {
  const int64_t blocks = (n4 + ET - 1) / ET;
  return (unsigned)(blocks < 256 * 32 ? blocks : 256 * 32);
}

}  // namespace
}  // namespace tj

extern "C" int tj_bias_residual(float* out, const float* x, const float* y, const float* bias, int64_t rows,
                                int64_t cols, int64_t seq_len, const int32_t* valid_len, int mode,
                                hipStream_t stream) {
  if (rows < 0 || cols <= 0 || seq_len <= 0 || mode < 0 || mode > 2) return TJ_ERR_SHAPE;
  if (!tjh::product_below(tj::kMaxElements, {rows, cols})) return TJ_ERR_SHAPE;
  if (mode != 0 && valid_len != nullptr && rows % seq_len != 0) return TJ_ERR_SHAPE;
  if (cols % 4 != 0) return TJ_ERR_UNSUPPORTED;
  if (rows == 0) return TJ_OK;
  if (!out || !x || !y || !bias) return TJ_ERR_SHAPE;
  if (!tjh::aligned16(out) || !tjh::aligned16(x) || !tjh::aligned16(y) || !tjh::aligned16(bias)) return TJ_ERR_ALIGN;
  const int64_t n4 = rows * (cols / 4);
  hipLaunchKernelGGL(tj::bias_residual_kernel, dim3(tj::grid_for(n4)), dim3(tj::ET), 0, stream, out, x, y, bias, n4,
                     cols / 4, seq_len, mode == 0 ? nullptr : valid_len, mode);
  return tjh::launch_status();
}

namespace {

template <tj::Act A>
int bias_act(float* y, const float* bias, int64_t rows, int64_t cols, void* out_f16, hipStream_t stream) {
  if (rows < 0 || cols <= 0 || !tjh::product_below(tj::kMaxElements, {rows, cols})) return TJ_ERR_SHAPE;
  if (cols % 4 != 0) return TJ_ERR_UNSUPPORTED;
  if (rows == 0) return TJ_OK;
  if (!y || !bias) return TJ_ERR_SHAPE;
  if (!tjh::aligned16(y) || !tjh::aligned16(bias) || (reinterpret_cast<uintptr_t>(out_f16) & 7u)) return TJ_ERR_ALIGN;
  const int64_t n4 = rows * (cols / 4);
  if (out_f16 != nullptr) {
    const int64_t ob = reinterpret_cast<int64_t>(out_f16), yb = reinterpret_cast<int64_t>(y);
    if (ob < yb + rows * cols * 4 && yb < ob + rows * cols * 2) return TJ_ERR_SHAPE;  // no overlap with y
    hipLaunchKernelGGL((tj::bias_act_kernel<A, half_t>), dim3(tj::grid_for(n4)), dim3(tj::ET), 0, stream, y,
                       static_cast<half_t*>(out_f16), bias, n4, cols / 4);
  } else {
    hipLaunchKernelGGL((tj::bias_act_kernel<A, float>), dim3(tj::grid_for(n4)), dim3(tj::ET), 0, stream, y, y, bias,
                       n4, cols / 4);
  }
  return tjh::launch_status();
}

}  // namespace

extern "C" int tj_bias_gelu(float* y, const float* bias, int64_t rows, int64_t cols, void* out_f16,
                            hipStream_t stream) {
  return bias_act<tj::ACT_GELU>(y, bias, rows, cols, out_f16, stream);
}

extern "C" int tj_bias_relu(float* y, const float* bias, int64_t rows, int64_t cols, void* out_f16,
                            hipStream_t stream) {
  return bias_act<tj::ACT_RELU>(y, bias, rows, cols, out_f16, stream);
}

namespace {

template <typename TN>
int launch_brl(float* out, TN* ln_out, const float* x, const float* y, const float* bias, const float* gamma,
               const float* beta, int64_t rows, int64_t cols, int64_t seq_len, const int32_t* vl, int mode, float eps,
               int zero_ln_padded, hipStream_t stream) {
  if (cols < 256) {
    const int64_t rows_per_block = (tj::ET / 64) * (64 / (cols / 4));
    const dim3 sgrid((unsigned)((rows + rows_per_block - 1) / rows_per_block));
    switch (cols) {
      case 32: hipLaunchKernelGGL((tj::bias_residual_ln_small_kernel<8, TN>), sgrid, dim3(tj::ET), 0, stream, out, ln_out, x, y, bias, gamma, beta, rows, seq_len, vl, mode, eps, zero_ln_padded); break;
      case 64: hipLaunchKernelGGL((tj::bias_residual_ln_small_kernel<16, TN>), sgrid, dim3(tj::ET), 0, stream, out, ln_out, x, y, bias, gamma, beta, rows, seq_len, vl, mode, eps, zero_ln_padded); break;
      case 128: hipLaunchKernelGGL((tj::bias_residual_ln_small_kernel<32, TN>), sgrid, dim3(tj::ET), 0, stream, out, ln_out, x, y, bias, gamma, beta, rows, seq_len, vl, mode, eps, zero_ln_padded); break;
      default: return TJ_ERR_UNSUPPORTED;
    }
    return tjh::launch_status();
  }
  const dim3 grid((unsigned)((rows + tj::ET / 64 - 1) / (tj::ET / 64)));
  switch (cols / 256) {
    case 1: hipLaunchKernelGGL((tj::bias_residual_ln_kernel<1, TN>), grid, dim3(tj::ET), 0, stream, out, ln_out, x, y, bias, gamma, beta, rows, seq_len, vl, mode, eps, zero_ln_padded); break;
    case 2: hipLaunchKernelGGL((tj::bias_residual_ln_kernel<2, TN>), grid, dim3(tj::ET), 0, stream, out, ln_out, x, y, bias, gamma, beta, rows, seq_len, vl, mode, eps, zero_ln_padded); break;
    case 4: hipLaunchKernelGGL((tj::bias_residual_ln_kernel<4, TN>), grid, dim3(tj::ET), 0, stream, out, ln_out, x, y, bias, gamma, beta, rows, seq_len, vl, mode, eps, zero_ln_padded); break;
    case 8: hipLaunchKernelGGL((tj::bias_residual_ln_kernel<8, TN>), grid, dim3(tj::ET), 0, stream, out, ln_out, x, y, bias, gamma, beta, rows, seq_len, vl, mode, eps, zero_ln_padded); break;
    default: return TJ_ERR_UNSUPPORTED;
  }
  return tjh::launch_status();
}

}  // namespace

extern "C" int tj_bias_residual_layernorm(float* out, void* ln_out, int ln_dtype, const float* x, const float* y,
                                          const float* bias, const float* gamma, const float* beta, int64_t rows,
                                          int64_t cols, int64_t seq_len, const int32_t* valid_len, int mode,
                                          float eps, int zero_ln_padded, hipStream_t stream) {
  if (rows < 0 || cols <= 0 || seq_len <= 0 || mode < 0 || mode > 2 || !(eps >= 0.f)) return TJ_ERR_SHAPE;
  if (!tjh::product_below(tj::kMaxElements, {rows, cols})) return TJ_ERR_SHAPE;
  if (ln_dtype != TJ_F32 && ln_dtype != TJ_F16) return TJ_ERR_DTYPE;
  if ((mode != 0 || zero_ln_padded) && valid_len != nullptr && rows % seq_len != 0) return TJ_ERR_SHAPE;
  if (!(cols == 32 || cols == 64 || cols == 128 || (cols % 256 == 0 && cols <= 2048))) return TJ_ERR_UNSUPPORTED;
  if (rows == 0) return TJ_OK;
  if (!ln_out || !x || !y || !bias || !gamma || !beta) return TJ_ERR_SHAPE;  // out may be null
  for (const void* p : {(const void*)out, (const void*)ln_out, (const void*)x, (const void*)y, (const void*)bias,
                        (const void*)gamma, (const void*)beta})
    if (!tjh::aligned16(p)) return TJ_ERR_ALIGN;
  const int64_t ln_bytes = rows * cols * tjh::elem_size(ln_dtype);
  // The norm output may overlap neither the inputs nor the residual output:
  // rows of an fp16 norm and of the fp32 operands differ in size, so a row's
  // store could land on a row another wave has not read yet.
  for (const void* p : {(const void*)out, (const void*)x, (const void*)y})
    if (p != nullptr && (int64_t)ln_out < (int64_t)p + rows * cols * 4 && (int64_t)p < (int64_t)ln_out + ln_bytes)
      return TJ_ERR_SHAPE;
  const int32_t* vl = (mode == 0 && !zero_ln_padded) ? nullptr : valid_len;
  if (ln_dtype == TJ_F16)
    return launch_brl(out, static_cast<half_t*>(ln_out), x, y, bias, gamma, beta, rows, cols, seq_len, vl, mode, eps,
                      zero_ln_padded, stream);
  return launch_brl(out, static_cast<float*>(ln_out), x, y, bias, gamma, beta, rows, cols, seq_len, vl, mode, eps,
                    zero_ln_padded, stream);
}
