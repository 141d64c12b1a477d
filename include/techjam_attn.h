/*
 * techjam_attn.h -- C ABI of the MI355X (gfx950) attention hot path.
 *
 * Plain pointers, sizes and a HIP stream; no framework types. Every tensor is
 * described by a device pointer plus four element strides in the logical order
 * [B, H, S, D]; the innermost (D) stride must be 1. Strided views -- for
 * example the [B, S, H, D] and [B, S, 3, H, D] projection outputs seen as
 * [B, H, S, D] -- are read in place, with no hidden copies.
 *
 * Conventions shared by all entry points:
 *   - Work is enqueued on `stream`; no entry point synchronises the host.
 *   - The caller owns and allocates every buffer (the library allocates no
 *     device memory); kernels that need scratch space take a workspace.
 *   - The return value is TJ_OK or one of the TJ_ERR_* codes below;
 *     tj_error_string() names it. Argument checks happen before any launch.
 *   - Calls are reentrant: the library keeps no mutable global state, except
 *     the fixed device scratch of tj_score_guard_noalloc (see there).
 *
 * The reference implements this path in Python on top of PyTorch SDPA and three
 * Triton kernels; each declaration names the reference interface it replaces.
 */
#ifndef TECHJAM_ATTN_H
#define TECHJAM_ATTN_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes. */
#define TJ_OK 0
#define TJ_ERR_SHAPE 1       /* inconsistent or non-positive sizes            */
#define TJ_ERR_DTYPE 2       /* unsupported element type                      */
#define TJ_ERR_ALIGN 3       /* pointer/stride not aligned for vector access  */
#define TJ_ERR_UNSUPPORTED 4 /* valid request the library does not implement */
#define TJ_ERR_LAUNCH 5      /* the HIP runtime rejected a launch             */
#define TJ_ERR_WORKSPACE 6   /* workspace missing or too small                */
#define TJ_ERR_SCRATCH 7     /* request larger than a fixed library scratch   */

/* Element types of the tensor arguments. */
#define TJ_F32 0
#define TJ_F16 1

/* ABI version, bumped on any signature or semantic change. */
int tj_abi_version(void);

/* Human-readable name of a return code. Never NULL. */
const char* tj_error_string(int code);

/*
 * Exact scaled-dot-product attention, forward.
 *
 * Replaces torch.nn.functional.scaled_dot_product_attention as called by the
 * reference at src/implementations/sdpa.py:65-73 and :157-165 (strided and
 * packed-QKV views, is_causal, scale, key mask dropped under causal right
 * padding), src/implementations/extreme.py:227-236 (forced-Flash fallback)
 * and src/implementations/poly_reference.py:262-264 (exact prefix).
 *
 *   o[b,h,i,:] = sum_j softmax_j(scale * q[b,h,i,:].k[b,h,j,:]) v[b,h,j,:]
 *
 * over keys j < valid_len[b] (all keys when valid_len is NULL) and, when
 * `causal`, j <= i. Rows i >= valid_len[b] are written as zeros: those are
 * the padded query rows the model zeroes after its output projection
 * (torch_transformer_benchmark.py:120-121). When row_limit is non-NULL, only
 * rows i < row_limit[b*H + h] are computed and written; the other rows of o
 * are left untouched (the polynomial path fills them).
 *
 * Arithmetic: q, k, v are rounded to fp16 (q after multiplying by
 * scale*log2(e)); QK^T and PV run on fp16 MFMA with fp32 accumulation; the
 * online softmax runs in fp32 on base-2 exponentials; o is written in the
 * input type. Heads with qk_split[b*H + h] != 0 form QK^T from a two-term
 * fp16 expansion of q and k (three MFMAs), which keeps fp32-level score
 * accuracy for wide score ranges (sigma of the scaled scores >~ 2).
 * head_dim D must be 32, 64, 128 or 256 (256: one workgroup per CU; no
 * qk_split, which returns TJ_ERR_UNSUPPORTED).
 *
 * dtype: TJ_F32 or TJ_F16 (q, k, v and o share it).
 * valid_len: device int32[B] or NULL. row_limit, qk_split: device
 * int32[B*H] or NULL.
 * Strides are in elements with a unit innermost stride; row starts must be
 * 16-byte aligned (TJ_ERR_ALIGN otherwise). The K and V rows of one (b,h) are
 * read through 31-bit byte offsets: their sequence stride must be >= 0 and
 * ((S-1)*stride + D) * element size < 2^31 (TJ_ERR_UNSUPPORTED otherwise).
 */
int tj_attn_fwd(const void* q, const void* k, const void* v, void* o, int dtype,
                int64_t B, int64_t H, int64_t S, int64_t D,
                const int64_t q_strides[4], const int64_t k_strides[4],
                const int64_t v_strides[4], const int64_t o_strides[4],
                float scale, int causal, const int32_t* valid_len,
                const int32_t* row_limit, const int32_t* qk_split,
                hipStream_t stream);

/*
 * tj_attn_fwd with the projection biases of q and v folded in: the kernel
 * reads the bias-free projections q', k', v' and computes the attention of
 * q' + q_bias, k' + k_bias, v' + v_bias. A key bias never changes the output
 * (it adds the same q.k_bias to every score of a row, and a row's softmax is
 * invariant to that), so it has no argument; the value bias comes out as
 * + v_bias on every valid row (a row's probabilities sum to 1). Padded rows
 * stay zero. This saves the pass over the [B, S, 3D] projection output that
 * adds its bias (the packed projection of sdpa.py:127-138 through
 * torch.nn.Linear).
 *
 * q_bias, v_bias: device fp32 [H * D] (head h at h * D), 16-byte aligned,
 * or NULL. No row limits or split scores on this entry point.
 */
int tj_attn_fwd_proj_bias(const void* q, const void* k, const void* v, void* o, int dtype,
                          int64_t B, int64_t H, int64_t S, int64_t D,
                          const int64_t q_strides[4], const int64_t k_strides[4],
                          const int64_t v_strides[4], const int64_t o_strides[4],
                          float scale, int causal, const int32_t* valid_len,
                          const float* q_bias, const float* v_bias, hipStream_t stream);

/*
 * Device-side score guard of the polynomial route.
 *
 * Replaces estimate_sigma / poly_is_safe / hermite_coefficients
 * (src/implementations/poly_guard.py:68-102,
 * src/implementations/poly_reference.py:35-58) and the module-level sigma cache
 * of src/implementations/extreme.py:299-305, without the host synchronisation:
 * for every (b,h) it takes the n_samples rows listed in sample_idx (device
 * int32), forms all n_samples^2 scaled scores q_s.k_s * scale and writes
 *   sigma_out[bh]  : their Bessel-corrected standard deviation,
 *   mean_out[bh]   : their mean (with sigma, the moments pooled estimates need),
 *   smax_out[bh]   : their largest magnitude,
 *   flags_out[bh]  : 1 when 0 < sigma <= ceiling and finite (polynomial route),
 *                    0 otherwise (exact fallback),
 *   coeffs_out[3*bh..]: (c0, c1, c2) of the Hermite fit at that sigma,
 *   row_limit_out[bh]: min(exact_prefix, S) for flagged heads, S otherwise --
 *                    the rows tj_attn_fwd must compute for that head,
 *   split_out[bh]  : 1 for heads routed to the exact fallback (their score
 *                    range is wide), 0 otherwise -- tj_attn_fwd's qk_split.
 * Any output pointer except flags_out may be NULL. workspace (16-byte
 * aligned, tj_score_guard_workspace_bytes(B, H, n_samples) bytes, contents
 * irrelevant) holds per-(b,h) partial sums between the two launches; calls
 * sharing one workspace must be ordered on one stream. D must be a multiple
 * of 4 (<= 128), rows and strides multiples of 4 elements.
 */
int tj_score_guard(const void* q, const void* k, int dtype,
                   int64_t B, int64_t H, int64_t S, int64_t D,
                   const int64_t q_strides[4], const int64_t k_strides[4],
                   float scale, const int32_t* sample_idx, int64_t n_samples,
                   float ceiling, int64_t exact_prefix,
                   float* sigma_out, float* mean_out, float* smax_out, int32_t* flags_out,
                   float* coeffs_out, int32_t* row_limit_out, int32_t* split_out,
                   void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Workspace needed by tj_score_guard, in bytes (0 for invalid sizes).
 */
size_t tj_score_guard_workspace_bytes(int64_t B, int64_t H, int64_t n_samples);

/* Size of the fixed device scratch of tj_score_guard_noalloc, in bytes. */
#define TJ_SCORE_GUARD_SCRATCH_BYTES ((size_t)1 << 20)

/*
 * tj_score_guard without a workspace argument and without any allocation.
 *
 * No counterpart in the reference. It is for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops and
 * harnesses that forbid hipMalloc. Same arguments (minus the workspace),
 * checks, kernels and results (bitwise) as tj_score_guard; the per-(b,h)
 * partial sums go to a file-scope device array of the library instead,
 * TJ_SCORE_GUARD_SCRATCH_BYTES in size, which each device the library runs
 * on holds until the process ends. Requests needing more than that
 * (tj_score_guard_workspace_bytes(B, H, n_samples) > TJ_SCORE_GUARD_SCRATCH_BYTES,
 * e.g. B*H > 5461 at 512 samples) return TJ_ERR_SCRATCH before launching.
 * The caller still allocates the inputs and outputs. `stream` must belong to
 * the current device (TJ_ERR_UNSUPPORTED otherwise). Every call on one device
 * shares that device's array: calls that may overlap on one GPU (different
 * streams, or several host threads) race and must be ordered by the caller.
 * Nothing in the array needs to start at zero: each call writes every
 * partial it reads.
 */
int tj_score_guard_noalloc(const void* q, const void* k, int dtype,
                           int64_t B, int64_t H, int64_t S, int64_t D,
                           const int64_t q_strides[4], const int64_t k_strides[4],
                           float scale, const int32_t* sample_idx, int64_t n_samples,
                           float ceiling, int64_t exact_prefix,
                           float* sigma_out, float* mean_out, float* smax_out, int32_t* flags_out,
                           float* coeffs_out, int32_t* row_limit_out, int32_t* split_out,
                           hipStream_t stream);

/*
 * Workspace needed by tj_poly_attn_fwd, in bytes.
 */
size_t tj_poly_workspace_bytes(int64_t B, int64_t H, int64_t S, int64_t D, int64_t chunk);

/*
 * Causal degree-2 polynomial linear attention, rows >= exact_prefix.
 *
 * Replaces poly_attention_forward -> poly_linear_attention
 * (src/implementations/poly_attention.py:21-83,
 * src/implementations/poly_reference.py:61-265) together with the three Triton
 * kernels quad_apply / quad_update / causal_diag
 * (src/kernels/poly_attention_triton.py:420-591). With a = q*sqrt(scale) and
 * b = k*sqrt(scale), every chunk of `chunk` tokens that ends past
 * exact_prefix gets
 *   o = (c0*S_const + c1*a.S_lin + c2*phi2(a).S_quad + diag_num)
 *     / (c0*t0     + c1*a.z_lin + c2*a^T G a        + diag_den)
 * with the diagonal block exp(a_i.b_j), j <= i inside the chunk, evaluated
 * exactly (no max subtraction), and the fp32 states folded forward chunk by
 * chunk. Operands are fp16, accumulation and states fp32.
 *
 * coeffs: device float[B*H*3] (c0, c1, c2 per head). flags: device int32[B*H]
 * or NULL; heads with flags[bh] == 0 are skipped entirely. Rows < exact_prefix
 * are not written: compute them with tj_attn_fwd (row_limit from the guard).
 * Only D == 64 and chunk == 512 are implemented.
 * K and V rows of one (b,h) are read through 31-bit byte offsets, as in
 * tj_attn_fwd (TJ_ERR_UNSUPPORTED otherwise).
 */
int tj_poly_attn_fwd(const void* q, const void* k, const void* v, void* o, int dtype,
                     int64_t B, int64_t H, int64_t S, int64_t D,
                     const int64_t q_strides[4], const int64_t k_strides[4],
                     const int64_t v_strides[4], const int64_t o_strides[4],
                     float scale, int64_t chunk, int64_t exact_prefix,
                     const float* coeffs, const int32_t* flags,
                     void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Stand-alone polynomial kernels with the reference's tensor contract
 * (src/kernels/poly_attention_triton.py:420-591: quad_apply, quad_update,
 * causal_diag). The fused tj_poly_attn_fwd does not use them; they serve
 * callers of the reference's kernel-level API. Shapes are [M, rows, cols]
 * with a unit innermost stride and 16-byte aligned rows; strides are in
 * elements. Only D == V == 64 is implemented (TJ_ERR_UNSUPPORTED otherwise;
 * the Python wrappers zero-pad narrower heads).
 *
 * tj_quad_apply (quad_apply, :420-466): y[m,c,:] = sum_{i,j} a[m,c,i]
 * a[m,c,j] s[m, i*D + j, :] with a, y fp16 and s fp32 or fp16 (s_dtype); s is
 * rounded to fp16 before the products, so a master and its fp16 shadow give
 * bitwise-identical y.
 */
int tj_quad_apply(const void* a, const void* s, void* y, int s_dtype, int64_t M, int64_t C, int64_t D,
                  int64_t V, const int64_t a_strides[3], const int64_t s_strides[3],
                  const int64_t y_strides[3], hipStream_t stream);

/*
 * tj_quad_update (quad_update, :469-530): s[m, i*D + j, :] +=
 * sum_t b[m,t,i] b[m,t,j] v[m,t,:] in place, s fp32 (the running master),
 * b, v fp16. When shadow is non-NULL (fp16, shaped like s) it receives the
 * updated master rounded to fp16.
 */
int tj_quad_update(const void* b, const void* v, float* s, void* shadow, int64_t M, int64_t C, int64_t D,
                   int64_t V, const int64_t b_strides[3], const int64_t v_strides[3],
                   const int64_t s_strides[3], const int64_t shadow_strides[3], hipStream_t stream);

/*
 * tj_causal_diag (causal_diag, :533-591): w = tril(exp(a b^T)) with no max
 * subtraction; num[m,c,:] = (w v)[c] (fp32), den[m*den_stride_m + c] =
 * sum_j w[c,j] (fp32, of the fp16-rounded weights the product uses).
 * a, b, v fp16.
 */
int tj_causal_diag(const void* a, const void* b, const void* v, float* num, float* den, int64_t M,
                   int64_t C, int64_t D, int64_t V, const int64_t a_strides[3],
                   const int64_t b_strides[3], const int64_t v_strides[3],
                   const int64_t num_strides[3], int64_t den_stride_m, hipStream_t stream);

/*
 * Fused tails of the encoder block (replaces the bias add, residual add and
 * masked_fill of torch_transformer_benchmark.py:116-121 and :140-145 around a
 * bias-free projection GEMM). fp32 [rows, cols] row-major, cols % 4 == 0,
 * 16-byte aligned; rows = B * seq_len, row b*seq_len+s valid iff
 * s < valid_len[b] (valid_len NULL: every row valid).
 *   mode 0: out = x + y + bias
 *   mode 1: out = x + (valid ? y + bias : 0)    (attention output, then residual)
 *   mode 2: out = valid ? x + y + bias : 0      (FFN output, residual, row zeroing)
 * out may alias x or y.
 */
int tj_bias_residual(float* out, const float* x, const float* y, const float* bias,
                     int64_t rows, int64_t cols, int64_t seq_len, const int32_t* valid_len,
                     int mode, hipStream_t stream);

/*
 * gelu(y + bias), exact (erf) GELU -- the bias of the FFN input GEMM fused
 * with F.gelu(approximate="none") (torch_transformer_benchmark.py:145).
 * out_f16 == NULL: y is overwritten with the result (fp32). Otherwise the
 * result is written, rounded to fp16, to out_f16 ([rows, cols], 8-byte
 * aligned, not overlapping y) and y is left unchanged: the fp16 operand of
 * the FFN output GEMM when the encoder's GEMMs take fp16 operands (the fused
 * cast of the packed-projection path, src/implementations/sdpa.py:127-138,
 * applied to the block's other GEMM inputs).
 */
int tj_bias_gelu(float* y, const float* bias, int64_t rows, int64_t cols, void* out_f16, hipStream_t stream);

/*
 * max(y + bias, 0), with tj_bias_gelu's two output forms. No counterpart in
 * the reference model (pre-norm, exact GELU); it serves the optional
 * post-norm / ReLU block, torch.nn.TransformerEncoderLayer(norm_first=False,
 * activation="relu") semantics, in which the benchmark configuration of a
 * one-layer post-norm encoder with a ReLU FFN is stated.
 */
int tj_bias_relu(float* y, const float* bias, int64_t rows, int64_t cols, void* out_f16, hipStream_t stream);

/*
 * tj_bias_residual (same modes, out may alias x or y) fused with the
 * LayerNorm that reads its result next (torch_transformer_benchmark.py:140-145:
 * norm2 after the attention residual, the next block's norm1 or the final norm
 * after the FFN residual, :163-172):
 *   ln_out[r,:] = (out[r,:] - mean) / sqrt(var + eps) * gamma + beta,
 * mean and biased variance over the row, as torch.nn.LayerNorm defines them,
 * stored as ln_dtype (TJ_F32, or TJ_F16 when the norm feeds a GEMM with fp16
 * operands; the statistics are fp32 either way).
 * With zero_ln_padded, rows at or past valid_len get ln_out = 0 (the final
 * masked_fill). out may be NULL: the sum is then not stored, only its norm
 * (a post-norm block, whose residual stream is the norm of the sum). ln_out
 * must overlap none of out, x, y. cols must be 32, 64, 128, 256, 512, 1024
 * or 2048 (TJ_ERR_UNSUPPORTED otherwise); all pointers 16-byte aligned.
 */
int tj_bias_residual_layernorm(float* out, void* ln_out, int ln_dtype, const float* x, const float* y,
                               const float* bias, const float* gamma, const float* beta,
                               int64_t rows, int64_t cols, int64_t seq_len,
                               const int32_t* valid_len, int mode, float eps,
                               int zero_ln_padded, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TECHJAM_ATTN_H */
