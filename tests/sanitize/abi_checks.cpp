// Host-side argument checks of the C ABI under AddressSanitizer and
// UndefinedBehaviorSanitizer. Every call below is one that an entry point must
// refuse before touching the HIP runtime: missing or misaligned tensors, bad
// dtypes, non-positive and huge sizes (products that overflow 64 bits), stride
// arrays with a non-unit innermost stride. The library is built for the host
// only (no device code), so a call that got as far as a launch would fail --
// and would be reported here as a wrong return code.
//
// Exit status 0 and no sanitizer report: every check held.
#include <cstdio>
#include <cstdint>
#include <cstring>
#include <limits>

#include "techjam_attn.h"

namespace {

int g_failures = 0;

void expect(const char* what, int got, int want) {
  if (got != want) {
    std::printf("FAIL %s: got %d (%s), want %d (%s)\n", what, got, tj_error_string(got), want, tj_error_string(want));
    ++g_failures;
  }
}

void expect_size(const char* what, size_t got, size_t want) {
  if (got != want) {
    std::printf("FAIL %s: got %zu, want %zu\n", what, got, want);
    ++g_failures;
  }
}

constexpr int64_t kBig = std::numeric_limits<int64_t>::max();

// Host addresses stand in for device pointers: no call below dereferences them.
alignas(256) unsigned char g_arena[1 << 16];
void* at(size_t off) { return g_arena + off; }

}  // namespace

int main() {
  expect("abi version", tj_abi_version(), 3);
  for (int c = -3; c <= 12; ++c) {
    const char* s = tj_error_string(c);
    if (s == nullptr || std::strlen(s) == 0) {
      std::printf("FAIL error string %d\n", c);
      ++g_failures;
    }
  }

  const int64_t st[4] = {16 * 4096 * 64, 4096 * 64, 64, 1};
  const int64_t st_bad_inner[4] = {16 * 4096 * 64, 4096 * 64, 64, 2};
  const int64_t st_huge_row[4] = {int64_t(1) << 60, int64_t(1) << 58, int64_t(1) << 40, 1};
  void *q = at(0), *k = at(256), *v = at(512), *o = at(768);

  // tj_attn_fwd(q, k, v, o, dtype, B, H, S, D, strides x4, scale, causal, valid_len, row_limit, qk_split, stream)
  expect("attn dtype", tj_attn_fwd(q, k, v, o, 7, 1, 1, 16, 64, st, st, st, st, 0.125f, 1, nullptr, nullptr, nullptr, nullptr), TJ_ERR_DTYPE);
  expect("attn negative B", tj_attn_fwd(q, k, v, o, TJ_F32, -1, 1, 16, 64, st, st, st, st, 0.125f, 1, nullptr, nullptr, nullptr, nullptr), TJ_ERR_SHAPE);
  expect("attn huge B*H", tj_attn_fwd(q, k, v, o, TJ_F32, kBig / 2, kBig / 2, 4096, 64, st, st, st, st, 0.125f, 1, nullptr, nullptr, nullptr, nullptr), TJ_ERR_SHAPE);
  expect("attn huge S", tj_attn_fwd(q, k, v, o, TJ_F32, 1, 1, kBig - 3, 64, st, st, st, st, 0.125f, 1, nullptr, nullptr, nullptr, nullptr), TJ_ERR_SHAPE);
  expect("attn head dim", tj_attn_fwd(q, k, v, o, TJ_F32, 1, 1, 16, 48, st, st, st, st, 0.125f, 1, nullptr, nullptr, nullptr, nullptr), TJ_ERR_UNSUPPORTED);
  expect("attn null q", tj_attn_fwd(nullptr, k, v, o, TJ_F32, 1, 1, 16, 64, st, st, st, st, 0.125f, 1, nullptr, nullptr, nullptr, nullptr), TJ_ERR_SHAPE);
  expect("attn misaligned q", tj_attn_fwd(at(8), k, v, o, TJ_F32, 1, 1, 16, 64, st, st, st, st, 0.125f, 1, nullptr, nullptr, nullptr, nullptr), TJ_ERR_ALIGN);
  expect("attn inner stride", tj_attn_fwd(q, k, v, o, TJ_F32, 1, 1, 16, 64, st, st_bad_inner, st, st, 0.125f, 1, nullptr, nullptr, nullptr, nullptr), TJ_ERR_ALIGN);
  expect("attn null strides", tj_attn_fwd(q, k, v, o, TJ_F32, 1, 1, 16, 64, st, nullptr, st, st, 0.125f, 1, nullptr, nullptr, nullptr, nullptr), TJ_ERR_ALIGN);
  expect("attn huge key stride", tj_attn_fwd(q, k, v, o, TJ_F32, 1, 1, 1 << 20, 64, st, st_huge_row, st, st, 0.125f, 1, nullptr, nullptr, nullptr, nullptr), TJ_ERR_UNSUPPORTED);
  expect("attn empty", tj_attn_fwd(nullptr, nullptr, nullptr, nullptr, TJ_F32, 0, 1, 16, 64, st, st, st, st, 0.125f, 1, nullptr, nullptr, nullptr, nullptr), TJ_OK);
  expect("attn bias alignment", tj_attn_fwd_proj_bias(q, k, v, o, TJ_F32, 1, 1, 16, 64, st, st, st, st, 0.125f, 1, nullptr, (const float*)at(4), nullptr, nullptr), TJ_ERR_ALIGN);

  // workspace sizes: 0 for invalid or overflowing requests
  expect_size("poly ws invalid", tj_poly_workspace_bytes(0, 1, 4096, 64, 512), 0);
  expect_size("poly ws huge", tj_poly_workspace_bytes(kBig / 2, kBig / 2, 4096, 64, 512), 0);
  expect_size("poly ws huge 2", tj_poly_workspace_bytes(int64_t(1) << 40, int64_t(1) << 20, 4096, 64, 512), 0);
  expect_size("guard ws invalid", tj_score_guard_workspace_bytes(1, 0, 512), 0);
  expect_size("guard ws huge", tj_score_guard_workspace_bytes(kBig / 2, kBig / 2, 512), 0);
  expect_size("guard ws huge 2", tj_score_guard_workspace_bytes(int64_t(1) << 62, 4, 1 << 29), 0);
  if (tj_poly_workspace_bytes(1, 1, 4096, 64, 512) == 0 || tj_score_guard_workspace_bytes(1, 1, 512) == 0) {
    std::printf("FAIL workspace sizes of a valid request\n");
    ++g_failures;
  }

  // tj_poly_attn_fwd(q, k, v, o, dtype, B, H, S, D, strides x4, scale, chunk, exact_prefix, coeffs, flags, ws, ws_bytes, stream)
  float coeffs[3] = {1.f, 1.f, 0.5f};
  expect("poly dtype", tj_poly_attn_fwd(q, k, v, o, 5, 1, 1, 8192, 64, st, st, st, st, 0.125f, 512, 4096, coeffs, nullptr, at(1024), 1 << 20, nullptr), TJ_ERR_DTYPE);
  expect("poly chunk", tj_poly_attn_fwd(q, k, v, o, TJ_F32, 1, 1, 8192, 64, st, st, st, st, 0.125f, 256, 4096, coeffs, nullptr, at(1024), 1 << 20, nullptr), TJ_ERR_UNSUPPORTED);
  expect("poly huge B*H", tj_poly_attn_fwd(q, k, v, o, TJ_F32, kBig / 2, kBig / 2, 8192, 64, st, st, st, st, 0.125f, 512, 4096, coeffs, nullptr, at(1024), 1 << 20, nullptr), TJ_ERR_SHAPE);
  expect("poly huge S", tj_poly_attn_fwd(q, k, v, o, TJ_F32, 1, 1, kBig - 1, 64, st, st, st, st, 0.125f, 512, 4096, coeffs, nullptr, at(1024), 1 << 20, nullptr), TJ_ERR_SHAPE);
  expect("poly null coeffs", tj_poly_attn_fwd(q, k, v, o, TJ_F32, 1, 1, 8192, 64, st, st, st, st, 0.125f, 512, 4096, nullptr, nullptr, at(1024), 1 << 20, nullptr), TJ_ERR_SHAPE);
  expect("poly huge key stride", tj_poly_attn_fwd(q, k, v, o, TJ_F32, 1, 1, 8192, 64, st, st_huge_row, st, st, 0.125f, 512, 4096, coeffs, nullptr, at(1024), 1 << 20, nullptr), TJ_ERR_UNSUPPORTED);
  expect("poly small workspace", tj_poly_attn_fwd(q, k, v, o, TJ_F32, 1, 1, 8192, 64, st, st, st, st, 0.125f, 512, 4096, coeffs, nullptr, at(1024), 1 << 20, nullptr), TJ_ERR_WORKSPACE);
  expect("poly prefix covers all", tj_poly_attn_fwd(q, k, v, o, TJ_F32, 1, 1, 4096, 64, st, st, st, st, 0.125f, 512, 4096, coeffs, nullptr, nullptr, 0, nullptr), TJ_OK);

  // tj_score_guard(q, k, dtype, B, H, S, D, qs, ks, scale, idx, n, ceiling, prefix, 7 outputs, ws, ws_bytes, stream)
  int32_t idx[4] = {0, 1, 2, 3};
  float* f = (float*)at(2048);
  int32_t* i32 = (int32_t*)at(4096);
  expect("guard dtype", tj_score_guard(q, k, 4, 1, 1, 4096, 64, st, st, 0.125f, idx, 4, 0.4f, 4096, f, f, f, i32, f, i32, i32, at(8192), 4096, nullptr), TJ_ERR_DTYPE);
  expect("guard samples > S", tj_score_guard(q, k, TJ_F32, 1, 1, 3, 64, st, st, 0.125f, idx, 4, 0.4f, 4096, f, f, f, i32, f, i32, i32, at(8192), 4096, nullptr), TJ_ERR_SHAPE);
  expect("guard huge B*H", tj_score_guard(q, k, TJ_F32, kBig / 2, kBig / 2, 4096, 64, st, st, 0.125f, idx, 4, 0.4f, 4096, f, f, f, i32, f, i32, i32, at(8192), 4096, nullptr), TJ_ERR_SHAPE);
  expect("guard huge samples", tj_score_guard(q, k, TJ_F32, 1, 1, kBig, 64, st, st, 0.125f, idx, kBig / 2, 0.4f, 4096, f, f, f, i32, f, i32, i32, at(8192), 4096, nullptr), TJ_ERR_SHAPE);
  expect("guard head dim", tj_score_guard(q, k, TJ_F32, 1, 1, 4096, 66, st, st, 0.125f, idx, 4, 0.4f, 4096, f, f, f, i32, f, i32, i32, at(8192), 4096, nullptr), TJ_ERR_UNSUPPORTED);
  expect("guard inner stride", tj_score_guard(q, k, TJ_F32, 1, 1, 4096, 64, st_bad_inner, st, 0.125f, idx, 4, 0.4f, 4096, f, f, f, i32, f, i32, i32, at(8192), 4096, nullptr), TJ_ERR_ALIGN);
  expect("guard null workspace", tj_score_guard(q, k, TJ_F32, 1, 1, 4096, 64, st, st, 0.125f, idx, 4, 0.4f, 4096, f, f, f, i32, f, i32, i32, nullptr, 0, nullptr), TJ_ERR_WORKSPACE);
  expect("guard noalloc scratch", tj_score_guard_noalloc(q, k, TJ_F32, 6000, 1, 4096, 64, st, st, 0.125f, idx, 512, 0.4f, 4096, f, f, f, i32, f, i32, i32, nullptr), TJ_ERR_SCRATCH);
  expect("guard noalloc huge", tj_score_guard_noalloc(q, k, TJ_F32, kBig / 2, 3, 4096, 64, st, st, 0.125f, idx, 4, 0.4f, 4096, f, f, f, i32, f, i32, i32, nullptr), TJ_ERR_SHAPE);

  // stand-alone polynomial kernels: [M, C, 64] operands
  const int64_t s3[3] = {512 * 64, 64, 1};
  const int64_t s3_bad[3] = {512 * 64, 64, 2};
  expect("quad_apply dtype", tj_quad_apply(q, k, o, 3, 32, 512, 64, 64, s3, s3, s3, nullptr), TJ_ERR_DTYPE);
  expect("quad_apply huge C", tj_quad_apply(q, k, o, TJ_F32, 32, kBig, 64, 64, s3, s3, s3, nullptr), TJ_ERR_SHAPE);
  expect("quad_apply huge M", tj_quad_apply(q, k, o, TJ_F32, kBig, 512, 64, 64, s3, s3, s3, nullptr), TJ_ERR_SHAPE);
  expect("quad_apply width", tj_quad_apply(q, k, o, TJ_F32, 32, 512, 32, 64, s3, s3, s3, nullptr), TJ_ERR_UNSUPPORTED);
  expect("quad_apply stride", tj_quad_apply(q, k, o, TJ_F32, 32, 512, 64, 64, s3_bad, s3, s3, nullptr), TJ_ERR_ALIGN);
  expect("quad_update huge", tj_quad_update(q, k, (float*)o, nullptr, kBig, kBig, 64, 64, s3, s3, s3, s3, nullptr), TJ_ERR_SHAPE);
  expect("quad_update shadow", tj_quad_update(q, k, (float*)o, at(6), 32, 512, 64, 64, s3, s3, s3, s3, nullptr), TJ_ERR_ALIGN);
  expect("causal_diag den stride", tj_causal_diag(q, k, v, (float*)o, (float*)at(4096), 32, 512, 64, 64, s3, s3, s3, s3, 100, nullptr), TJ_ERR_SHAPE);
  expect("causal_diag huge", tj_causal_diag(q, k, v, (float*)o, (float*)at(4096), kBig, kBig, 64, 64, s3, s3, s3, s3, 100, nullptr), TJ_ERR_SHAPE);

  // block tails: [rows, cols] fp32
  float* x = (float*)at(0);
  float* y = (float*)at(16384);
  expect("residual huge", tj_bias_residual(x, x, y, y, kBig / 2, kBig / 4, 16, nullptr, 0, nullptr), TJ_ERR_SHAPE);
  expect("residual mode", tj_bias_residual(x, x, y, y, 4, 8, 2, nullptr, 3, nullptr), TJ_ERR_SHAPE);
  expect("gelu huge", tj_bias_gelu(y, y, kBig / 2, kBig / 4, nullptr, nullptr), TJ_ERR_SHAPE);
  expect("gelu overlap", tj_bias_gelu(y, y, 4, 8, at(16384 + 64), nullptr), TJ_ERR_SHAPE);
  expect("relu huge", tj_bias_relu(y, y, kBig, 8, nullptr, nullptr), TJ_ERR_SHAPE);
  expect("layernorm huge", tj_bias_residual_layernorm(nullptr, at(32768), TJ_F32, x, y, y, y, y, kBig / 2, 256, 4, nullptr, 0, 1e-5f, 0, nullptr), TJ_ERR_SHAPE);
  expect("layernorm width", tj_bias_residual_layernorm(nullptr, at(32768), TJ_F32, x, y, y, y, y, 4, 384, 4, nullptr, 0, 1e-5f, 0, nullptr), TJ_ERR_UNSUPPORTED);
  expect("layernorm dtype", tj_bias_residual_layernorm(nullptr, at(32768), 9, x, y, y, y, y, 4, 256, 4, nullptr, 0, 1e-5f, 0, nullptr), TJ_ERR_DTYPE);
  expect("layernorm overlap", tj_bias_residual_layernorm(nullptr, at(16384 + 2048), TJ_F32, x, y, y, y, y, 4, 256, 4, nullptr, 0, 1e-5f, 0, nullptr), TJ_ERR_SHAPE);
  expect("layernorm eps", tj_bias_residual_layernorm(nullptr, at(32768), TJ_F32, x, y, y, y, y, 4, 256, 4, nullptr, 0, -1.f, 0, nullptr), TJ_ERR_SHAPE);

  if (g_failures != 0) {
    std::printf("%d check(s) failed\n", g_failures);
    return 1;
  }
  std::printf("all argument checks held\n");
  return 0;
}
