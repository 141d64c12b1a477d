// Stand-alone polynomial-attention kernels with the reference's tensor
// contract (src/kernels/poly_attention_triton.py:420-591):
//
//   quad_apply  : y[m, c, :] = sum_{i,j} a[m,c,i] a[m,c,j] S[m, i*D + j, :]
//                 (S rounded to fp16 before the products, so an fp32 master
//                 and its fp16 shadow give bitwise-identical results);
//   quad_update : S[m, i*D + j, :] += sum_t b[m,t,i] b[m,t,j] v[m,t,:]
//                 (fp32 master in place; optional fp16 shadow = its rounding);
//   causal_diag : w = tril(exp(a b^T)); num = w v (fp32), den = rowsum(w) (fp32).
//
// Here D = V = 64 (the extreme-length configuration); the Python wrappers
// zero-pad narrower heads and value widths to 64. The fused chunk kernel in
// poly_attn.hip computes the same three quantities inside one launch with its
// own state layout; these entry points serve callers of the reference's
// kernel-level API.
//
// MFMA use follows the fused kernel: quad_apply forms y^T = S_i^T (a_i * a)^T
// with the B operand a_i * a built in registers; quad_update accumulates
// S_i^T (b_i * b) v into 32x32 accumulator blocks; causal_diag forms S^T = b a^T
// and feeds the exponentiated accumulator back as the B operand of V^T P^T.
#include "tj_common.h"

namespace tj {
namespace {

constexpr int XD = 64;        // head dim = value width
constexpr int XT = 256;       // threads per workgroup
constexpr int XLP = 72;       // padded LDS row (144 bytes)
constexpr int XAP = 66;       // padded row of the a tile (132 bytes)

struct View3 {
  int64_t sm, sr;  // strides of the outer two dims (elements); innermost is 1
  __device__ __forceinline__ int64_t at(int m, int r) const { return (int64_t)m * sm + (int64_t)r * sr; }
};

// fp16 [rows][64] tile of a [M, C, 64] fp16 tensor, 4 rows x 4 dims per thread,
// rows past C read as zeros.
struct HalfTile {
  half4_t x[4];
  __device__ __forceinline__ static void coords(int tid, int& g, int& c) {
    g = (tid >> 2) & 15;
    c = (tid & 3) | ((tid >> 6) << 2);
  }
  __device__ __forceinline__ void load(const half_t* p, const View3& vw, int m, int r0, int C, int tid) {
    int g, c;
    coords(tid, g, c);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = r0 + 4 * g + r;
      if (row < C) x[r] = *reinterpret_cast<const half4_t*>(p + vw.at(m, row) + 4 * c);
      else x[r] = half4_t{0, 0, 0, 0};
    }
  }
  // [dim][row] (rows in the order given).
  __device__ __forceinline__ void store_t(half_t (*dst)[XLP], int tid) const {
    int g, c;
    coords(tid, g, c);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      *reinterpret_cast<half4_t*>(&dst[4 * c + e][4 * g]) = half4_t{x[0][e], x[1][e], x[2][e], x[3][e]};
  }
  // [row][dim].
  __device__ __forceinline__ void store_rows(half_t (*dst)[XLP], int tid) const {
    int g, c;
    coords(tid, g, c);
#pragma unroll
    for (int r = 0; r < 4; ++r) *reinterpret_cast<half4_t*>(&dst[4 * g + r][4 * c]) = x[r];
  }
  // [dim][key_slot(row)]: V^T in the exact kernel's column order.
  __device__ __forceinline__ void store_t_slot(half_t (*dst)[XLP], int tid) const {
    int g, c;
    coords(tid, g, c);
    const int slot = key_slot(4 * g);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      *reinterpret_cast<half4_t*>(&dst[4 * c + e][slot]) = half4_t{x[0][e], x[1][e], x[2][e], x[3][e]};
  }
};

// a tile of one 128-row block: B operands (dims 16 ks + 8 hl .. +7 of row
// c0 + 32 w + ln) and the a tile in LDS for the per-i scalars.
__device__ __forceinline__ void load_a_rows(const half_t* a, const View3& va, int m, int c0, int C,
                                            half8_t aB[4], half_t (*at)[XAP]) {
  const int tid = threadIdx.x, w = tid / kWave, lane = tid % kWave, hl = lane / 32, ln = lane % 32;
  const int c = c0 + 32 * w + ln;
  const bool in = c < C;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    aB[ks] = in ? *reinterpret_cast<const half8_t*>(a + va.at(m, c) + 16 * ks + 8 * hl) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 8; j += 2)
      *reinterpret_cast<half2_t*>(&at[32 * w + ln][16 * ks + 8 * hl + j]) = half2_t{aB[ks][j], aB[ks][j + 1]};
  }
}

// ---------------------------------------------------------------------------
// quad_apply
// ---------------------------------------------------------------------------
struct ApplyArgs {
  const half_t* a;
  const void* s;
  half_t* y;
  View3 va, vs, vy;
  int M, C;
};

// The 64 x 32 half of slice S_i (rows j, the 32 columns v of one half of V)
// as loaded, 4 rows x 2 columns per thread (16 threads cover a 128-byte fp32
// half row), converted to fp16 and transposed ([v][j]) only when stored to LDS
// for the MFMA A operand -- so a load in flight holds no conversion back.
template <typename TS>
struct HalfSlice {
  using Raw = std::conditional_t<sizeof(TS) == 4, float __attribute__((ext_vector_type(2))), half2_t>;
  Raw x[4];
  // This thread's first element of slice 0: row 4 g, column 32 vh + 2 c of S[m].
  __device__ __forceinline__ static const TS* origin(const TS* s, const View3& vs, int m, int vh, int tid) {
    return s + vs.at(m, 4 * (tid >> 4)) + 32 * vh + 2 * (tid & 15);
  }
  // Slice i from the origin; the row offsets are uniform (scalar) products.
  __device__ __forceinline__ void load(const TS* o, int64_t row_stride, int i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) x[r] = *reinterpret_cast<const Raw*>(o + (int64_t)(i * XD + r) * row_stride);
  }
  __device__ __forceinline__ void store_t(half_t (*dst)[XLP], int tid) const {
    const int c = tid & 15, g = tid >> 4;
    // The empty asm pins the conversion here: left free, the scheduler
    // converts each load as soon as it is issued (two fp32 registers become
    // one), which waits for the load and empties the ring.
    Raw y[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      y[r] = x[r];
      asm volatile("" : "+v"(y[r]));
    }
#pragma unroll
    for (int e = 0; e < 2; ++e)
      *reinterpret_cast<half4_t*>(&dst[2 * c + e][4 * g]) =
          half4_t{(half_t)y[0][e], (half_t)y[1][e], (half_t)y[2][e], (half_t)y[3][e]};
  }
};

// The workgroups of one m read the same 1 MiB state: the linear block id is
// remapped so that they run on one XCD (ids are dealt round-robin over the
// XCDs) and share its L2. Returns false for padding ids.
__device__ __forceinline__ bool xcd_block(int n_rb, int M, int& m, int& rb) {
  const int total = n_rb * M;
  const int per_xcd = (total + kNumXcd - 1) / kNumXcd;
  const int id = blockIdx.x;
  const int logical = (id % kNumXcd) * per_xcd + id / kNumXcd;
  if (logical >= total) return false;
  m = logical / n_rb;
  rb = logical % n_rb;
  return true;
}

unsigned xcd_grid(int n_rb, int64_t M) {
  const int64_t total = n_rb * M;
  return (unsigned)(((total + kNumXcd - 1) / kNumXcd) * kNumXcd);
}

// Slices in flight per thread (the load of slice i is issued kApplyDepth
// slices before it is staged into LDS), and slices per barrier.
constexpr int kApplyDepth = 8;
constexpr int kApplyGroup = 4;
static_assert(kApplyDepth % kApplyGroup == 0 && XD % kApplyGroup == 0, "ring and groups must tile the slices");

// One workgroup per (m, 128 rows, half of V): y[:, 32 vh .. 32 vh + 31] of the
// rows, from the matching half of every slice S_i. Halving V doubles the
// workgroups of a launch (a launch of 32 m x 512 rows fills 256 CUs instead of
// 128); the sums run in the same order as over the whole width, so the result
// is bitwise that of a full-width tile. The slices stream through a
// kApplyDepth-deep register ring and a two-slot LDS ring (kApplyGroup slices
// per slot) separated by plain barriers, so the loads stay in flight across
// barriers. (Measured at 32 m x 512 rows: 41 -> 17 us for an fp32 state.)
template <typename TS>
__global__ __launch_bounds__(XT, 2) void quad_apply_kernel(ApplyArgs a) {
  constexpr int G = kApplyGroup, P = kApplyDepth;
  __shared__ half_t sst[2][G][32][XLP];  // [slot][slice of the group][v][j]
  __shared__ half_t at[128][XAP];
  int m, t;
  if (!xcd_block(2 * ((a.C + 127) / 128), a.M, m, t)) return;
  const int c0 = 128 * (t >> 1), vh = t & 1;
  const int tid = threadIdx.x, w = tid / kWave, lane = tid % kWave, hl = lane / 32, ln = lane % 32;
  const TS* s = reinterpret_cast<const TS*>(a.s);
  half8_t aB[4];
  load_a_rows(a.a, a.va, m, c0, a.C, aB, at);

  const TS* so = HalfSlice<TS>::origin(s, a.vs, m, vh, tid);
  const int64_t sr = a.vs.sr;
  HalfSlice<TS> ring[P];
  static_for<0, P>([&](auto p) { ring[p].load(so, sr, p); });
  static_for<0, G>([&](auto g) {
    ring[g].store_t(sst[0][g], tid);
    ring[g].load(so, sr, P + g);
  });
  wait_lds();  // the a tile and the first group are in LDS
  lds_barrier();

  half2_t arow[32];  // this lane's row of a (4-byte reads: the a tile's rows are 132 bytes)
#pragma unroll
  for (int q = 0; q < 32; ++q) arow[q] = *reinterpret_cast<const half2_t*>(&at[32 * w + ln][2 * q]);
  float16_t acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
  static_for<0, XD / G>([&](auto stc) {
    constexpr int st = decltype(stc)::value;
    static_for<0, G>([&](auto gc) {
      constexpr int g = decltype(gc)::value, i = st * G + g;
      const half_t ai = arow[i / 2][i % 2];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        half8_t bop;
#pragma unroll
        for (int j = 0; j < 8; ++j) bop[j] = aB[ks][j] * ai;
        acc = mfma32(*reinterpret_cast<const half8_t*>(&sst[st & 1][g][ln][16 * ks + 8 * hl]), bop, acc);
      }
    });
    if constexpr (st * G + G < XD) {
      // Ring entry k % P holds slice k: stage the next group into the other
      // slot (read by nobody since the last barrier), then reload the entries
      // with slices k + P.
      static_for<0, G>([&](auto gc) {
        constexpr int g = decltype(gc)::value, k = (st + 1) * G + g;
        ring[k % P].store_t(sst[(st + 1) & 1][g], tid);
        if constexpr (k + P < XD) ring[k % P].load(so, sr, k + P);
      });
      wait_lds();
      lds_barrier();
    }
  });

  const int c = c0 + 32 * w + ln;
  if (c >= a.C) return;
  half_t* yp = a.y + a.vy.at(m, c) + 32 * vh;
#pragma unroll
  for (int g = 0; g < 4; ++g)
    *reinterpret_cast<half4_t*>(yp + 8 * g + 4 * hl) =
        half4_t{(half_t)acc[4 * g], (half_t)acc[4 * g + 1], (half_t)acc[4 * g + 2], (half_t)acc[4 * g + 3]};
}

// ---------------------------------------------------------------------------
// quad_update
// ---------------------------------------------------------------------------
struct UpdateArgs {
  const half_t* b;
  const half_t* v;
  float* s;
  half_t* shadow;
  View3 vb, vv, vs, vsh;
  int M, C;
};

// One workgroup per (m, 4 consecutive i); wave w owns i = 4 blockIdx.x + w.
// Consecutive workgroups land on different XCDs: each XCD then re-reads b and
// v of the head from HBM (2x the algorithmic fetch), but the state traffic
// spreads more evenly and the launch runs ~5 % faster than with the 16
// workgroups of one m kept on one XCD.
// acc[jb][vb] holds D[j][v] of S_i, i.e. state rows i*64 + j, columns v.
__global__ __launch_bounds__(XT, 2) void quad_update_kernel(UpdateArgs a) {
  __shared__ half_t bt[2][XD][XLP];
  __shared__ half_t vt[2][XD][XLP];
  const int m = blockIdx.y;
  const int tid = threadIdx.x, w = tid / kWave, lane = tid % kWave, hl = lane / 32, ln = lane % 32;
  const int i = 4 * blockIdx.x + w;

  float16_t acc[2][2];
  {
    const float* base = a.s + a.vs.at(m, i * XD) + ln;
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int vb = 0; vb < 2; ++vb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = 32 * jb + 8 * (r / 4) + 4 * hl + (r % 4);
          acc[jb][vb][r] = base[(int64_t)j * a.vs.sr + 32 * vb];
        }
  }

  const int n_blk = (a.C + 63) / 64;
  HalfTile tb, tv;
  if (n_blk > 0) {
    tb.load(a.b, a.vb, m, 0, a.C, tid);
    tv.load(a.v, a.vv, m, 0, a.C, tid);
    tb.store_t(bt[0], tid);
    tv.store_t(vt[0], tid);
  }
  __syncthreads();
  for (int blk = 0; blk < n_blk; ++blk) {
    const int cur = blk & 1;
    if (blk + 1 < n_blk) {
      tb.load(a.b, a.vb, m, 64 * (blk + 1), a.C, tid);
      tv.load(a.v, a.vv, m, 64 * (blk + 1), a.C, tid);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int t = 16 * ks + 8 * hl;
      const half8_t bi = *reinterpret_cast<const half8_t*>(&bt[cur][i][t]);
      half8_t vv[2];
#pragma unroll
      for (int x = 0; x < 2; ++x) vv[x] = *reinterpret_cast<const half8_t*>(&vt[cur][32 * x + ln][t]);
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        const half8_t bj = *reinterpret_cast<const half8_t*>(&bt[cur][32 * jb + ln][t]);
        half8_t phi;
#pragma unroll
        for (int j = 0; j < 8; ++j) phi[j] = bj[j] * bi[j];
#pragma unroll
        for (int vb = 0; vb < 2; ++vb) acc[jb][vb] = mfma32(phi, vv[vb], acc[jb][vb]);
      }
    }
    if (blk + 1 < n_blk) {
      tb.store_t(bt[cur ^ 1], tid);
      tv.store_t(vt[cur ^ 1], tid);
    }
    __syncthreads();
  }

  float* sbase = a.s + a.vs.at(m, i * XD) + ln;
  half_t* hbase = a.shadow != nullptr ? a.shadow + a.vsh.at(m, i * XD) + ln : nullptr;
#pragma unroll
  for (int jb = 0; jb < 2; ++jb)
#pragma unroll
    for (int vb = 0; vb < 2; ++vb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = 32 * jb + 8 * (r / 4) + 4 * hl + (r % 4);
        const float x = acc[jb][vb][r];
        sbase[(int64_t)j * a.vs.sr + 32 * vb] = x;
        if (hbase != nullptr) hbase[(int64_t)j * a.vsh.sr + 32 * vb] = (half_t)x;
      }
}

// ---------------------------------------------------------------------------
// causal_diag
// ---------------------------------------------------------------------------
struct DiagArgs {
  const half_t* a;
  const half_t* b;
  const half_t* v;
  float* num;
  float* den;
  View3 va, vb, vv, vn;
  int64_t den_sm;  // den stride over m (rows are contiguous)
  int M, C;
};

// One workgroup per (m, 128 rows); keys stream in tiles of 64 up to the last
// row of the block. w = exp(a.b) with no max subtraction (the guard bounds
// the scores), rounded to fp16 for the PV MFMA; den sums the rounded weights.
__global__ __launch_bounds__(XT, 2) void causal_diag_kernel(DiagArgs a) {
  __shared__ half_t kb[2][64][XLP];
  __shared__ half_t vt[2][XD][XLP];
  __shared__ half_t at[128][XAP];
  const int m = blockIdx.y, c0 = 128 * blockIdx.x;
  const int tid = threadIdx.x, w = tid / kWave, lane = tid % kWave, hl = lane / 32, ln = lane % 32;
  half8_t aB[4];
  load_a_rows(a.a, a.va, m, c0, a.C, aB, at);
  const int qw0 = c0 + 32 * w;
  const int qi = qw0 + ln;

  float16_t accd[2];
#pragma unroll
  for (int vb = 0; vb < 2; ++vb)
#pragma unroll
    for (int r = 0; r < 16; ++r) accd[vb][r] = 0.f;
  float den = 0.f;

  const int key_end = min(a.C, c0 + 128);
  const int n_kt = (key_end + 63) / 64;
  const int wave_last = min(qw0 + 31, key_end - 1);
  HalfTile tk, tv;
  tk.load(a.b, a.vb, m, 0, key_end, tid);
  tv.load(a.v, a.vv, m, 0, key_end, tid);
  tk.store_rows(kb[0], tid);
  tv.store_t_slot(vt[0], tid);
  __syncthreads();
  for (int kt = 0; kt < n_kt; ++kt) {
    const int cur = kt & 1;
    const int kv0 = 64 * kt;
    if (kt + 1 < n_kt) {
      tk.load(a.b, a.vb, m, kv0 + 64, key_end, tid);
      tv.load(a.v, a.vv, m, kv0 + 64, key_end, tid);
    }
    if (kv0 <= wave_last) {
      float16_t sc[2];
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[kh][r] = 0.f;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          sc[kh] = mfma32(*reinterpret_cast<const half8_t*>(&kb[cur][32 * kh + ln][16 * ks + 8 * hl]), aB[ks], sc[kh]);
      }
      half8_t pf[4];
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kv0 + 32 * kh + 8 * (r / 4) + 4 * hl + (r % 4);
          const float wgt = key <= qi ? fast_exp2(sc[kh][r] * 1.4426950408889634f) : 0.f;
          const half_t wh = (half_t)wgt;
          den += (float)wh;
          pf[2 * kh + r / 8][r % 8] = wh;
        }
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int vb = 0; vb < 2; ++vb)
          accd[vb] = mfma32(*reinterpret_cast<const half8_t*>(&vt[cur][32 * vb + ln][16 * st + 8 * hl]), pf[st], accd[vb]);
    }
    if (kt + 1 < n_kt) {
      tk.store_rows(kb[cur ^ 1], tid);
      tv.store_t_slot(vt[cur ^ 1], tid);
    }
    __syncthreads();
  }
  den = pair_sum(den);
  if (qi >= a.C) return;
  float* np = a.num + a.vn.at(m, qi);
#pragma unroll
  for (int vb = 0; vb < 2; ++vb)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<float4_t*>(np + 32 * vb + 8 * g + 4 * hl) =
          float4_t{accd[vb][4 * g], accd[vb][4 * g + 1], accd[vb][4 * g + 2], accd[vb][4 * g + 3]};
  if (hl == 0) a.den[(int64_t)m * a.den_sm + qi] = den;
}

bool view3_ok(const void* p, const int64_t st[3], int elt) {
  if (p == nullptr || st == nullptr || st[2] != 1 || !tjh::aligned16(p)) return false;
  const int64_t vec = 16 / elt;
  return st[0] % vec == 0 && st[1] % vec == 0;
}

}  // namespace
}  // namespace tj

extern "C" int tj_quad_apply(const void* a, const void* s, void* y, int s_dtype, int64_t M, int64_t C, int64_t D,
                             int64_t V, const int64_t a_strides[3], const int64_t s_strides[3],
                             const int64_t y_strides[3], hipStream_t stream) {
  if (s_dtype != TJ_F32 && s_dtype != TJ_F16) return TJ_ERR_DTYPE;
  if (M < 0 || C < 0 || D <= 0 || V <= 0) return TJ_ERR_SHAPE;
  if (D != tj::XD || V != tj::XD) return TJ_ERR_UNSUPPORTED;
  if (M == 0 || C == 0) return TJ_OK;
  if (M >= 65536 || C >= (int64_t(1) << 30) || 2 * ((C + 127) / 128) * M >= (int64_t(1) << 31)) return TJ_ERR_SHAPE;
  if (!tj::view3_ok(a, a_strides, 2) || !tj::view3_ok(s, s_strides, tjh::elem_size(s_dtype)) ||
      !tj::view3_ok(y, y_strides, 2))
    return TJ_ERR_ALIGN;
  tj::ApplyArgs args;
  args.a = static_cast<const half_t*>(a);
  args.s = s;
  args.y = static_cast<half_t*>(y);
  args.va = {a_strides[0], a_strides[1]};
  args.vs = {s_strides[0], s_strides[1]};
  args.vy = {y_strides[0], y_strides[1]};
  args.M = (int)M;
  args.C = (int)C;
  const dim3 grid(tj::xcd_grid((int)(2 * ((C + 127) / 128)), M));
  if (s_dtype == TJ_F32)
    hipLaunchKernelGGL(tj::quad_apply_kernel<float>, grid, dim3(tj::XT), 0, stream, args);
  else
    hipLaunchKernelGGL(tj::quad_apply_kernel<half_t>, grid, dim3(tj::XT), 0, stream, args);
  return tjh::launch_status();
}

extern "C" int tj_quad_update(const void* b, const void* v, float* s, void* shadow, int64_t M, int64_t C, int64_t D,
                              int64_t V, const int64_t b_strides[3], const int64_t v_strides[3],
                              const int64_t s_strides[3], const int64_t shadow_strides[3], hipStream_t stream) {
  if (M < 0 || C < 0 || D <= 0 || V <= 0) return TJ_ERR_SHAPE;
  if (D != tj::XD || V != tj::XD) return TJ_ERR_UNSUPPORTED;
  if (M == 0 || C == 0) return TJ_OK;
  if (M >= 65536 || C >= (int64_t(1) << 30)) return TJ_ERR_SHAPE;
  if (!tj::view3_ok(b, b_strides, 2) || !tj::view3_ok(v, v_strides, 2) || !tj::view3_ok(s, s_strides, 4))
    return TJ_ERR_ALIGN;
  if (shadow != nullptr && !tj::view3_ok(shadow, shadow_strides, 2)) return TJ_ERR_ALIGN;
  tj::UpdateArgs args;
  args.b = static_cast<const half_t*>(b);
  args.v = static_cast<const half_t*>(v);
  args.s = s;
  args.shadow = static_cast<half_t*>(shadow);
  args.vb = {b_strides[0], b_strides[1]};
  args.vv = {v_strides[0], v_strides[1]};
  args.vs = {s_strides[0], s_strides[1]};
  args.vsh = shadow != nullptr ? tj::View3{shadow_strides[0], shadow_strides[1]} : tj::View3{0, 0};
  args.M = (int)M;
  args.C = (int)C;
  hipLaunchKernelGGL(tj::quad_update_kernel, dim3(tj::XD / 4, (unsigned)M), dim3(tj::XT), 0, stream, args);
  return tjh::launch_status();
}

extern "C" int tj_causal_diag(const void* a, const void* b, const void* v, float* num, float* den, int64_t M,
                              int64_t C, int64_t D, int64_t V, const int64_t a_strides[3],
                              const int64_t b_strides[3], const int64_t v_strides[3],
                              const int64_t num_strides[3], int64_t den_stride_m, hipStream_t stream) {
  if (M < 0 || C < 0 || D <= 0 || V <= 0) return TJ_ERR_SHAPE;
  if (D != tj::XD || V != tj::XD) return TJ_ERR_UNSUPPORTED;
  if (M == 0 || C == 0) return TJ_OK;
  if (M >= 65536 || C >= (int64_t(1) << 30)) return TJ_ERR_SHAPE;
  if (!tj::view3_ok(a, a_strides, 2) || !tj::view3_ok(b, b_strides, 2) || !tj::view3_ok(v, v_strides, 2) ||
      !tj::view3_ok(num, num_strides, 4) || den == nullptr)
    return TJ_ERR_ALIGN;
  if (den_stride_m < C) return TJ_ERR_SHAPE;
  tj::DiagArgs args;
  args.a = static_cast<const half_t*>(a);
  args.b = static_cast<const half_t*>(b);
  args.v = static_cast<const half_t*>(v);
  args.num = num;
  args.den = den;
  args.va = {a_strides[0], a_strides[1]};
  args.vb = {b_strides[0], b_strides[1]};
  args.vv = {v_strides[0], v_strides[1]};
  args.vn = {num_strides[0], num_strides[1]};
  args.den_sm = den_stride_m;
  args.M = (int)M;
  args.C = (int)C;
  hipLaunchKernelGGL(tj::causal_diag_kernel, dim3((unsigned)((C + 127) / 128), (unsigned)M), dim3(tj::XT), 0,
                     stream, args);
  return tjh::launch_status();
}
