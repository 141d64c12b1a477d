// Shared types and helpers of the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>
#include <limits>
#include <type_traits>

#include "techjam_attn.h"

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

namespace tj {

constexpr int kWave = 64;
constexpr int kNumXcd = 8;  // MI355X: 8 XCDs, workgroups dispatched round-robin

// 32x32x16 fp16 MFMA (gfx950): D = A * B + C.
//   A: lane l holds row (l % 32), k-slots 8*(l/32) .. +7
//   B: lane l holds column (l % 32), k-slots 8*(l/32) .. +7
//   C/D: lane l, register r holds row 8*(r/4) + 4*(l/32) + (r%4), column (l % 32)
// The contraction is a sum over k, so any slot -> k assignment works as long
// as A and B use the same one; the kernels rely on that to feed accumulators
// back as operands without a shuffle.
__device__ __forceinline__ float16_t mfma32(half8_t a, half8_t b, float16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Workgroup barrier without the memory fences of __syncthreads() (which also
// wait for every global load in flight): callers wait for their own LDS
// traffic explicitly (s_waitcnt) before it. The empty asm statements keep the
// compiler from moving memory accesses across.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt lgkmcnt(0) alone (vmcnt and expcnt at their maxima): this wave's
// LDS accesses are done, its global loads may stay in flight.
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// f(integral_constant<int, I>) for I = B .. E-1, each with compile-time I.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// Reductions over the lane pair (l, l ^ 32) through v_permlane32_swap, a VALU
// op on gfx950, instead of an LDS permute. With both operands equal to x, the
// swap gives every lane l the pair's two values in a fixed order: r[0] is x of
// lane l & 31 (the lower half of the wave) and r[1] is x of lane (l & 31) + 32
// (the upper half), in both lanes of the pair. So a lane can pick its partner's
// value, or the value of a given half, by index (poly_attn.hip's a_pair relies
// on this); max and sum give both lanes bitwise identical results.
__device__ __forceinline__ void pair_values(float x, float& a, float& b) {
  const unsigned u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair_max(float x) {
  float a, b;
  pair_values(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float pair_sum(float x) {
  float a, b;
  pair_values(x, a, b);
  return a + b;
}

// 16-byte vector of input elements: 4 floats or 8 halves, widened to fp32.
template <typename T>
struct Vec16;

template <>
struct Vec16<float> {
  static constexpr int N = 4;
  float4_t v;
  __device__ __forceinline__ void load(const float* p) { v = *reinterpret_cast<const float4_t*>(p); }
  __device__ __forceinline__ void zero() { v = float4_t{0.f, 0.f, 0.f, 0.f}; }
  __device__ __forceinline__ float get(int i) const { return v[i]; }
};

template <>
struct Vec16<half_t> {
  static constexpr int N = 8;
  half8_t v;
  __device__ __forceinline__ void load(const half_t* p) { v = *reinterpret_cast<const half8_t*>(p); }
  __device__ __forceinline__ void zero() { v = half8_t{0, 0, 0, 0, 0, 0, 0, 0}; }
  __device__ __forceinline__ float get(int i) const { return (float)v[i]; }
};

// Strided [B, H, S, D] view with unit D stride.
struct View4 {
  int64_t sb, sh, ss;
  __device__ __forceinline__ int64_t row(int b, int h, int s) const {
    return (int64_t)b * sb + (int64_t)h * sh + (int64_t)s * ss;
  }
};

// Swap bits 2 and 3 of a key index inside each 16-key group. The exact
// kernel stores V^T columns in this order so that the eight keys one lane
// contributes to a PV k-step sit in one 16-byte LDS word (see attn_exact.hip).
__device__ __forceinline__ int key_slot(int key) {
  return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}

}  // namespace tj

// Host-side argument checks shared by the entry points.
namespace tjh {

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int elem_size(int dtype) { return dtype == TJ_F32 ? 4 : (dtype == TJ_F16 ? 2 : 0); }

// The product of non-negative factors is below `limit`, decided without
// overflowing (a negative factor or an overflowing product is not below).
inline bool product_below(int64_t limit, std::initializer_list<int64_t> factors) {
  int64_t p = 1;
  for (int64_t f : factors)
    if (f < 0 || __builtin_mul_overflow(p, f, &p)) return false;
  return p < limit;
}

// Rows 0 .. rows-1 of `width` elements at `stride` elements per row span
// fewer than 2^31 bytes (31-bit offsets inside the kernels). rows < 2^30.
inline bool span_below_2g(int64_t rows, int64_t stride, int64_t width, int elt) {
  if (stride < 0 || stride >= (int64_t(1) << 31)) return false;
  return ((rows - 1) * stride + width) * elt < (int64_t(1) << 31);
}

// Row starts of a strided view are 16-byte aligned when the base is and every
// outer stride is a multiple of 16 bytes.
inline bool view_ok(const void* p, const int64_t st[4], int dtype) {
  const int64_t vec = 16 / elem_size(dtype);
  if (st == nullptr || st[3] != 1) return false;
  if (!aligned16(p)) return false;
  for (int i = 0; i < 3; ++i)
    if (st[i] % vec != 0) return false;
  return true;
}

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TJ_OK : TJ_ERR_LAUNCH;
}

}  // namespace tjh
