// Exact causal / right-padded scaled-dot-product attention for gfx950: the
// C ABI entry points and the choice of kernel instance per call (query rows
// per workgroup, key tile width, split scores). The kernel itself, its
// work decomposition and numerics are in attn_exact_kernel.h.
#include "attn_exact_kernel.h"

namespace tj {
namespace {

// Two query blocks per wave halve LDS operand traffic and staging per MFMA.
// They fit the register budget for head_dim <= 64 (with split scores only at
// head_dim 64 with 32-key tiles, fp32 inputs), and need sequences long enough
// to fill 256-row tiles. Launches with fewer than 1024 such tiles (two per CU)
// keep 128-row tiles: there the heaviest tile sets the time, and a 32-row
// block per wave halves its per-key-tile work.
template <typename T, int HD>
int launch(const AttnArgs& a, hipStream_t stream) {
  if constexpr (HD <= 64) {
    const int64_t wide_tiles = int64_t(a.B) * a.H * ((a.S + 255) / 256);
    if (a.S >= 512 && wide_tiles >= 1024) {
      if (a.qk_split == nullptr) return launch_qb<T, HD, 2>(a, stream);
      // Split scores carry K's low half and Q's as well: two query blocks
      // per wave fit only with 32-key tiles (fp32 inputs, head_dim 64).
      if constexpr (HD == 64 && sizeof(T) == 4) return launch_split_wide(a, stream);
    }
  }
  return launch_qb<T, HD, 1>(a, stream);
}

template <typename T>
int dispatch_hd(const AttnArgs& a, int64_t D, hipStream_t stream) {
  switch (D) {
    case 32: return launch<T, 32>(a, stream);
    case 64: return launch<T, 64>(a, stream);
    case 128: return launch<T, 128>(a, stream);
    case 256: return a.qk_split != nullptr ? TJ_ERR_UNSUPPORTED : launch<T, 256>(a, stream);
    default: return TJ_ERR_UNSUPPORTED;
  }
}

}  // namespace
}  // namespace tj

namespace {

int attn_fwd(const void* q, const void* k, const void* v, void* o, int dtype, int64_t B, int64_t H, int64_t S,
             int64_t D, const int64_t q_strides[4], const int64_t k_strides[4], const int64_t v_strides[4],
             const int64_t o_strides[4], float scale, int causal, const int32_t* valid_len,
             const int32_t* row_limit, const int32_t* qk_split, const float* q_bias, const float* v_bias,
             hipStream_t stream) {
  if (dtype != TJ_F32 && dtype != TJ_F16) return TJ_ERR_DTYPE;
  if (B < 0 || H <= 0 || S < 0 || D <= 0) return TJ_ERR_SHAPE;
  // Tile indices fit 31 bits; the launch also checks that its grid fits the
  // 32-bit dispatch size.
  if (S >= (int64_t(1) << 30) || !tjh::product_below(int64_t(1) << 31, {B, H, (S + 127) / 128})) return TJ_ERR_SHAPE;
  if (D != 32 && D != 64 && D != 128 && D != 256) return TJ_ERR_UNSUPPORTED;
  if (B == 0 || S == 0) return TJ_OK;
  if (!q || !k || !v || !o) return TJ_ERR_SHAPE;
  if (!tjh::view_ok(q, q_strides, dtype) || !tjh::view_ok(k, k_strides, dtype) ||
      !tjh::view_ok(v, v_strides, dtype) || !tjh::view_ok(o, o_strides, dtype))
    return TJ_ERR_ALIGN;
  if ((reinterpret_cast<uintptr_t>(q_bias) | reinterpret_cast<uintptr_t>(v_bias)) & 15u) return TJ_ERR_ALIGN;
  // K and V rows of one (b, h) are addressed with 31-bit byte offsets.
  for (const int64_t* st : {k_strides, v_strides})
    if (!tjh::span_below_2g(S, st[2], D, tjh::elem_size(dtype))) return TJ_ERR_UNSUPPORTED;

  tj::AttnArgs a;
  a.q = q; a.k = k; a.v = v; a.o = o;
  a.vq = {q_strides[0], q_strides[1], q_strides[2]};
  a.vk = {k_strides[0], k_strides[1], k_strides[2]};
  a.vv = {v_strides[0], v_strides[1], v_strides[2]};
  a.vo = {o_strides[0], o_strides[1], o_strides[2]};
  a.B = (int)B; a.H = (int)H; a.S = (int)S;
  a.qscale = scale * 1.4426950408889634f;
  a.causal = causal ? 1 : 0;
  a.valid_len = valid_len;
  a.row_limit = row_limit;
  a.qk_split = qk_split;
  a.q_bias = q_bias;
  a.v_bias = v_bias;
  if (dtype == TJ_F32) return tj::dispatch_hd<float>(a, D, stream);
  return tj::dispatch_hd<half_t>(a, D, stream);
}

}  // namespace

extern "C" int tj_attn_fwd(const void* q, const void* k, const void* v, void* o, int dtype,
                           int64_t B, int64_t H, int64_t S, int64_t D,
                           const int64_t q_strides[4], const int64_t k_strides[4],
                           const int64_t v_strides[4], const int64_t o_strides[4],
                           float scale, int causal, const int32_t* valid_len,
                           const int32_t* row_limit, const int32_t* qk_split, hipStream_t stream) {
  return attn_fwd(q, k, v, o, dtype, B, H, S, D, q_strides, k_strides, v_strides, o_strides, scale, causal,
                  valid_len, row_limit, qk_split, nullptr, nullptr, stream);
}

extern "C" int tj_attn_fwd_proj_bias(const void* q, const void* k, const void* v, void* o, int dtype,
                                     int64_t B, int64_t H, int64_t S, int64_t D,
                                     const int64_t q_strides[4], const int64_t k_strides[4],
                                     const int64_t v_strides[4], const int64_t o_strides[4],
                                     float scale, int causal, const int32_t* valid_len,
                                     const float* q_bias, const float* v_bias, hipStream_t stream) {
  return attn_fwd(q, k, v, o, dtype, B, H, S, D, q_strides, k_strides, v_strides, o_strides, scale, causal,
                  valid_len, nullptr, nullptr, q_bias, v_bias, stream);
}
