// Exact causal / right-padded scaled-dot-product attention for gfx950.
//
// Forward pass of softmax(q k^T * scale) v with FP32 (or FP16) tensors in HBM,
// fp16 MFMA operands and fp32 accumulation; replaces the SDPA calls of the
// reference (src/implementations/sdpa.py:65-73, :157-165,
// src/implementations/extreme.py:227-236, poly_reference.py:262-264).
//
// Work decomposition
//   * One workgroup = 4 waves = a tile of 128 QB query rows of one (b, h);
//     each wave owns QB blocks of 32 consecutive rows (QB = 1 or 2) for the
//     whole key loop.
//   * Keys stream through LDS in tiles of 64 (32 for the split-score kernel
//     with two query blocks per wave) -- double buffered: K row-major, V
//     transposed, both converted to fp16 while being stored.
//   * Scores are computed transposed, S^T = K Q^T (keys x queries), so a lane
//     holds 32 keys of ONE query: the row max/sum is lane-local plus one swap
//     with lane ^ 32, the rescale factor is a per-lane scalar, and the fp32
//     accumulator converts in place into the B operand of O^T = V^T P^T -- P
//     never leaves registers.
//   * Q is pre-multiplied by scale*log2(e) before rounding, so the softmax runs
//     on exp2 with no per-score multiply.
//   * Causal tiles above the diagonal are never loaded; a wave skips the
//     compute of tiles that start after its last row. Under causal attention
//     the right-padding key mask is redundant (every valid row i only sees
//     keys j <= i < L) and is not applied; padded rows i >= L are written as 0.
//   * Grid: tile ids are remapped so that all query tiles of one (b, h) land on
//     one XCD. Each XCD takes a contiguous range of (b, h). A long range is
//     walked one (b, h) at a time, heaviest (last) query tile first, so the
//     tiles of a (b, h) start close together and share its K/V sweep in L2;
//     its last group of (b, h) (about one XCD's worth of workgroup slots) is
//     interleaved instead, heaviest tiles first across the group, so that no
//     heavy tile starts late and the XCD's tail stays short. A short range
//     (at most two such groups) is interleaved group by group throughout.
//     Launches with row limits, whose work sits on a few (b, h), and launches
//     with fewer than eight (b, h) spread every (b, h) over all XCDs.
//     The (b, h) ranges are taken in sample-fastest order, so each XCD holds
//     an even mix of the samples' valid lengths. Both walks deal their
//     heaviest-first lists in snake rounds of four, so that the XCD's four
//     shader engines, which take consecutive workgroups in turn, see equal
//     work.
//   * Heads flagged in qk_split compute QK^T from a two-term fp16 expansion of
//     q and k (x = hi + lo, both fp16) with three MFMAs -- hi.hi + hi.lo +
//     lo.hi -- which restores fp32-level score accuracy where the score range
//     is wide enough for fp16 rounding of q and k to show in the softmax, and
//     feed PV the probabilities as two fp16 parts as well (P = hi + lo, two
//     MFMAs per step), so that the only rounding left on those heads is v's
//     to fp16: an output moves by at most 2^-11 * sum_j p_j |v_j| / l.
//
// This header holds the kernel and its launch helper; attn_exact.hip
// picks the instance per call and exposes the C ABI, and
// attn_exact_split.hip builds the split-score instance with two query
// blocks per wave in a translation unit of its own (different compiler
// scheduling, see there).
#pragma once

#include "tj_common.h"

namespace tj {

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  View4 vq, vk, vv, vo;
  int B, H, S;
  float qscale;  // scale * log2(e)
  int causal;
  const int32_t* valid_len;
  const int32_t* row_limit;
  const int32_t* qk_split;
  const float* q_bias;  // [H * D] fp32 or null: added to q before scaling
  const float* v_bias;  // [H * D] fp32 or null: added to every valid output row
  int n_mtiles;
  int group;     // (b, h) per interleaved group on one XCD
  int balanced;  // spread every (b, h) over all XCDs (row limits or B*H < 8)
};

// The split-score kernel with two query blocks per wave on 32-key tiles
// (fp32 inputs, head_dim 64), built in attn_exact_split.hip.
int launch_split_wide(const AttnArgs& a, hipStream_t stream);

namespace {

constexpr int BN = 64;     // keys per tile (kernels take a tile width BNT: 64, or 32)
constexpr int NT = 256;    // threads per workgroup
constexpr int PAD = 8;     // fp16 padding per LDS row (16 bytes)
constexpr float kRescaleLog2 = 8.f;  // lazy-rescale threshold of the running max (log2 units)
constexpr int kBufferFlags = 0x00020000;  // raw (untyped) buffer resource word 3 on gfx950

template <typename T, int HD>
struct Tile {
  static constexpr int VEC = Vec16<T>::N;      // elements per 16-byte load
  static constexpr int NC = HD / VEC;          // 16-byte vectors per row
  static constexpr int UNITS = 16 * NC;        // (4-key group, vector) units
  static constexpr int UPT = (UNITS + NT - 1) / NT;
  static constexpr int KS = HD / 16;           // MFMA k-steps over head_dim
  static constexpr int DB = HD / 32;           // 32-wide output blocks
  static_assert(NC % 4 == 0, "head_dim too small for the load mapping");
};

template <int HD, int BNT>
struct SmemBase {
  half_t k[2][BNT][HD + PAD];   // K tile (high part), row-major
  half_t vt[2][HD][BNT + PAD];  // V tile, transposed, columns in key_slot order
};

// Kernels that may meet split heads also carry the low part of K.
template <int HD, bool SPLIT_OK, int BNT>
struct Smem : SmemBase<HD, BNT> {};

template <int HD, int BNT>
struct Smem<HD, true, BNT> : SmemBase<HD, BNT> {
  half_t klo[2][BNT][HD + PAD];
};

// Low fp16 parts of x0, x1 given their packed fp16 roundings h: fp16(x - h),
// one v_fma_mix per element (x * 1 - h in fp32, rounded once to fp16). x - h
// is exact in fp32, so this is the rounded fp32 difference bit for bit, in one
// instruction instead of a convert back to fp32, a subtract and a convert.
__device__ __forceinline__ uint32_t low_parts(float x0, float x1, uint32_t h) {
  uint32_t lo;
  asm("v_fma_mixlo_f16 %0, %1, 1.0, -%3 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixhi_f16 %0, %2, 1.0, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
      : "=&v"(lo)
      : "v"(x0), "v"(x1), "v"(h));
  return lo;
}

// Global -> register staging of one key tile of 16 KPU keys. Unit u covers
// keys KPU g .. KPU g + KPU - 1 of the tile (KPU = 4, or 2 for 32-key tiles)
// and one 16-byte column vector c; lanes 4n .. 4n+3 share g so a 16-lane LDS
// store phase touches KPU rows x 4 columns.
//
// K and V are read with bounds-checked buffer loads: one resource per (b, h)
// spans rows 0 .. S-1 (byte offsets fit 31 bits, checked on the host), so
// keys at or past S read as zeros without a branch, and the per-tile address
// arithmetic is scalar: lane offset (KPU g, c) + scalar offset (kv0 + r) * stride.
template <typename T, int HD, int KPU>
struct KVStage {
  using TL = Tile<T, HD>;
  static_assert(KPU == 4 || (KPU == 2 && sizeof(T) == 4), "two-key units for fp32 inputs only");
  Vec16<T> kx[TL::UPT][KPU];
  Vec16<T> vx[TL::UPT][KPU];
  __amdgpu_buffer_rsrc_t rk, rv;
  uint32_t koff[TL::UPT], voff[TL::UPT];
  uint32_t kstep, vstep;  // bytes per key row

  __device__ __forceinline__ static void unit_coords(int u, int& g, int& c) {
    g = (u >> 2) & 15;
    c = (u & 3) | ((u >> 6) << 2);
  }

  __device__ __forceinline__ void init(const AttnArgs& a, int b, int h, int tid) {
    const T* kp = reinterpret_cast<const T*>(a.k) + a.vk.row(b, h, 0);
    const T* vp = reinterpret_cast<const T*>(a.v) + a.vv.row(b, h, 0);
    kstep = (uint32_t)(a.vk.ss * (int64_t)sizeof(T));
    vstep = (uint32_t)(a.vv.ss * (int64_t)sizeof(T));
    const int kbytes = (int)((int64_t)(a.S - 1) * kstep + HD * (int64_t)sizeof(T));
    const int vbytes = (int)((int64_t)(a.S - 1) * vstep + HD * (int64_t)sizeof(T));
    rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(kp), (short)0, kbytes, kBufferFlags);
    rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(vp), (short)0, vbytes, kBufferFlags);
#pragma unroll
    for (int p = 0; p < TL::UPT; ++p) {
      int g, c;
      unit_coords(tid + p * NT, g, c);
      koff[p] = KPU * g * kstep + c * TL::VEC * (uint32_t)sizeof(T);
      voff[p] = KPU * g * vstep + c * TL::VEC * (uint32_t)sizeof(T);
    }
  }

  __device__ __forceinline__ void load(int kv0, int tid) {
#pragma unroll
    for (int p = 0; p < TL::UPT; ++p) {
      if (tid + p * NT < TL::UNITS) {
#pragma unroll
        for (int r = 0; r < KPU; ++r) {
          kx[p][r].v = __builtin_bit_cast(decltype(kx[p][r].v),
                                          __builtin_amdgcn_raw_buffer_load_b128(rk, koff[p], (kv0 + r) * kstep, 0));
          vx[p][r].v = __builtin_bit_cast(decltype(vx[p][r].v),
                                          __builtin_amdgcn_raw_buffer_load_b128(rv, voff[p], (kv0 + r) * vstep, 0));
        }
      }
    }
  }

  template <bool SPLIT, typename SM>
  __device__ __forceinline__ void store(SM& sm, int buf, int tid) const {
#pragma unroll
    for (int p = 0; p < TL::UPT; ++p) {
      const int u = tid + p * NT;
      if (u < TL::UNITS) {
        int g, c;
        unit_coords(u, g, c);
#pragma unroll
        for (int r = 0; r < KPU; ++r) {
#pragma unroll
          for (int e = 0; e < TL::VEC; e += 4) {
            half4_t hk;
#pragma unroll
            for (int j = 0; j < 4; ++j) hk[j] = (half_t)kx[p][r].get(e + j);
            *reinterpret_cast<half4_t*>(&sm.k[buf][KPU * g + r][c * TL::VEC + e]) = hk;
            if constexpr (SPLIT) {
              using u32x2 = uint32_t __attribute__((ext_vector_type(2)));
              const u32x2 hw = __builtin_bit_cast(u32x2, hk);
              const u32x2 lw = {low_parts(kx[p][r].get(e), kx[p][r].get(e + 1), hw[0]),
                                low_parts(kx[p][r].get(e + 2), kx[p][r].get(e + 3), hw[1])};
              *reinterpret_cast<half4_t*>(&sm.klo[buf][KPU * g + r][c * TL::VEC + e]) = __builtin_bit_cast(half4_t, lw);
            }
          }
        }
        const int slot = key_slot(KPU * g);
        if constexpr (KPU == 2) {
#pragma unroll
          for (int e = 0; e < TL::VEC; ++e) {
            half2_t hv = {(half_t)vx[p][0].get(e), (half_t)vx[p][1].get(e)};
            *reinterpret_cast<half2_t*>(&sm.vt[buf][c * TL::VEC + e][slot]) = hv;
          }
        } else if constexpr (sizeof(T) == 2) {
          // fp16 rows: dword m of the four key rows holds elements 2m, 2m+1;
          // byte permutes gather them column-wise (element-wise extraction
          // from a 16-byte register goes through scratch memory).
          using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
          using u32x2 = uint32_t __attribute__((ext_vector_type(2)));
#pragma unroll
          for (int m = 0; m < TL::VEC / 2; ++m) {
            uint32_t d[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) d[r] = __builtin_bit_cast(u32x4, vx[p][r].v)[m];
            const u32x2 lo = {__builtin_amdgcn_perm(d[1], d[0], 0x05040100u), __builtin_amdgcn_perm(d[3], d[2], 0x05040100u)};
            const u32x2 hi = {__builtin_amdgcn_perm(d[1], d[0], 0x07060302u), __builtin_amdgcn_perm(d[3], d[2], 0x07060302u)};
            *reinterpret_cast<half4_t*>(&sm.vt[buf][c * TL::VEC + 2 * m][slot]) = __builtin_bit_cast(half4_t, lo);
            *reinterpret_cast<half4_t*>(&sm.vt[buf][c * TL::VEC + 2 * m + 1][slot]) = __builtin_bit_cast(half4_t, hi);
          }
        } else {
#pragma unroll
          for (int e = 0; e < TL::VEC; ++e) {
            half4_t hv = {(half_t)vx[p][0].get(e), (half_t)vx[p][1].get(e),
                          (half_t)vx[p][2].get(e), (half_t)vx[p][3].get(e)};
            *reinterpret_cast<half4_t*>(&sm.vt[buf][c * TL::VEC + e][slot]) = hv;
          }
        }
      }
    }
  }
};

// One query tile of one (b, h): 4 waves x 32*QB rows. Each wave holds QB
// 32-row query blocks, so every K / V^T operand read from LDS feeds QB MFMAs.
// SPLIT selects the three-MFMA score path.
template <typename T, int HD, int QB, bool SPLIT, int BNT, typename SM>
__device__ __forceinline__ void attn_tile(const AttnArgs& a, SM& sm, int b, int h, int q0, int row_cap,
                                          int L) {
  using TL = Tile<T, HD>;
  constexpr int NKB = BNT / 32;  // 32-key score blocks per tile
  constexpr int NS = BNT / 16;   // 16-key PV steps per tile
  constexpr int WROWS = 32 * QB;
  constexpr int TROWS = 4 * WROWS;
  const int tid = threadIdx.x;
  const int w = tid / kWave;
  const int lane = tid % kWave;
  const int hl = lane / 32;
  const int ln = lane % 32;
  const int qw0 = q0 + WROWS * w;

  // Rows [q0, row_end) need keys (rows in [L, row_cap) are written as zeros
  // by the epilogue); a tile with none of them streams no keys at all.
  const int row_end = min(min(q0 + TROWS, L), row_cap);
  const int kv_end = q0 >= row_end ? 0 : (a.causal ? row_end : L);
  const int n_kv = kv_end > 0 ? (kv_end + BNT - 1) / BNT : 0;
  // Last key this wave needs (inclusive); waves whose rows are all padding
  // (or beyond row_cap) compute nothing.
  int wave_last_key = a.causal ? min(qw0 + WROWS - 1, kv_end - 1) : kv_end - 1;
  if (qw0 >= L || qw0 >= row_cap) wave_last_key = -1;

  // The first key tile's loads go out before q's, so the two latencies overlap.
  KVStage<T, HD, BNT / 16> stage;
  stage.init(a, b, h, tid);
  if (n_kv > 0) stage.load(0, tid);

  // Q^T as the B operand: lane holds query qw0 + 32*qb + ln, dims 16*ks + 8*hl .. +7.
  half8_t qf[QB][TL::KS];
  half8_t qlo[QB][SPLIT ? TL::KS : 1];
  {
    const T* qp = reinterpret_cast<const T*>(a.q);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int qi = qw0 + 32 * qb + ln;
      const bool in = qi < a.S;
      const int64_t base = a.vq.row(b, h, in ? qi : 0);
#pragma unroll
      for (int ks = 0; ks < TL::KS; ++ks) {
        const int d0 = 16 * ks + 8 * hl;
        // q bias of these eight dims (two 16-byte loads; zeros without one)
        float bq[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (a.q_bias != nullptr) {
#pragma unroll
          for (int f = 0; f < 2; ++f) {
            const float4_t t = *reinterpret_cast<const float4_t*>(a.q_bias + h * HD + d0 + 4 * f);
#pragma unroll
            for (int j = 0; j < 4; ++j) bq[4 * f + j] = t[j];
          }
        }
#pragma unroll
        for (int e = 0; e < 8; e += Vec16<T>::N) {
          Vec16<T> x;
          if (in) x.load(qp + base + d0 + e); else x.zero();
#pragma unroll
          for (int j = 0; j < Vec16<T>::N; ++j) {
            float y = (x.get(j) + bq[e + j]) * a.qscale;
            // Split heads: hi and lo must both come from this one rounded
            // fp32 y. Left free, the compiler forms the lo part's hi from the
            // exact product (one v_fma_mix rounding to fp16) and the MFMA
            // operand from the rounded y; where y rounds onto an fp16
            // midpoint the two differ by an fp16 ulp and hi + lo misses q.
            if constexpr (SPLIT) asm("" : "+v"(y));
            const half_t hi = (half_t)y;
            qf[qb][ks][e + j] = hi;
            if constexpr (SPLIT) qlo[qb][ks][e + j] = (half_t)(y - (float)hi);
          }
        }
      }
    }
  }

  float16_t oacc[QB][TL::DB];
  float m_run[QB], l_run[QB];
  // -m_run splat kept as a register block: it is the C operand of each query
  // block's first score MFMA, so the scores leave the MFMA already shifted
  // without re-initialising the accumulators every tile.
  float16_t cneg[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_run[qb] = -__builtin_inff();
    l_run[qb] = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) cneg[qb][r] = 0.f;
#pragma unroll
    for (int db = 0; db < TL::DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[qb][db][r] = 0.f;
  }

  if (n_kv > 0) stage.template store<SPLIT>(sm, 0, tid);
  __syncthreads();

  for (int kt = 0; kt < n_kv; ++kt) {
    const int cur = kt & 1;
    const int kv0 = kt * BNT;
    if (kt + 1 < n_kv) stage.load(kv0 + BNT, tid);

    if (kv0 <= wave_last_key) {
      // Scores come out of the MFMA already shifted by the running max: the
      // accumulator starts at -m_run (0 on the first tile, where m_run is set).
      const bool first = kv0 == 0;
      float16_t sacc[QB][NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int ks = 0; ks < TL::KS; ++ks) {
          const half8_t kf = *reinterpret_cast<const half8_t*>(&sm.k[cur][kb * 32 + ln][16 * ks + 8 * hl]);
          if constexpr (SPLIT) {
            const half8_t kl = *reinterpret_cast<const half8_t*>(&sm.klo[cur][kb * 32 + ln][16 * ks + 8 * hl]);
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
              sacc[qb][kb] = mfma32(kl, qf[qb][ks], ks == 0 ? cneg[qb] : sacc[qb][kb]);
              sacc[qb][kb] = mfma32(kf, qlo[qb][ks], sacc[qb][kb]);
            }
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) sacc[qb][kb] = mfma32(kf, qf[qb][ks], sacc[qb][kb]);
          } else {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) sacc[qb][kb] = mfma32(kf, qf[qb][ks], ks == 0 ? cneg[qb] : sacc[qb][kb]);
          }
        }

      half8_t pf[QB][NS];
      half8_t pl[QB][SPLIT ? NS : 1];  // split heads: p - fp16(p), rounded to fp16
      float shift[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const int qb0 = qw0 + 32 * qb;
        const int qi = qb0 + ln;
        // Mask keys past the diagonal (causal) or past the valid length.
        const bool need_mask = a.causal ? (kv0 + BNT - 1 > qb0) : (kv0 + BNT > L);
        if (need_mask) {
          const int lim = a.causal ? qi : L - 1;
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int key = kv0 + kb * 32 + 8 * (r / 4) + 4 * hl + (r % 4);
              if (key > lim) sacc[qb][kb][r] = -__builtin_inff();
            }
        }
        float t_max = sacc[qb][0][0];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) t_max = fmaxf(t_max, sacc[qb][kb][r]);
        t_max = pair_max(t_max);
        // Lazy rescaling: the reference point moves only when a row's max grows
        // by more than 2^8 (p <= 256 is exact enough in fp16 and harmless in the
        // fp32 accumulators); the first tile always sets it.
        shift[qb] = first ? t_max : (t_max > kRescaleLog2 ? t_max : 0.f);
      }
      // One wave-wide decision per tile for all query blocks (a lane or block
      // whose shift is 0 rescales by exactly 1).
      bool moved = false;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) moved |= shift[qb] != 0.f;
      if (first || __any(moved)) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const float alpha = first ? 0.f : fast_exp2(-shift[qb]);
          m_run[qb] = first ? shift[qb] : m_run[qb] + shift[qb];
          l_run[qb] *= alpha;
#pragma unroll
          for (int db = 0; db < TL::DB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[qb][db][r] *= alpha;
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[qb][kb][r] -= shift[qb];
#pragma unroll
          for (int r = 0; r < 16; ++r) cneg[qb][r] = -m_run[qb];
        }
      }
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        if constexpr (SPLIT) {
          // Split heads: P = hi + lo, both fp16 (lo = fp16(p - hi)), so the PV
          // MFMAs multiply p to about 2^-22 of its value; the row sum adds p
          // itself in fp32, consistent with that.
          float psum = 0.f;
#pragma unroll
          for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
              const float p0 = fast_exp2(sacc[qb][s / 2][8 * (s % 2) + j]);
              const float p1 = fast_exp2(sacc[qb][s / 2][8 * (s % 2) + j + 1]);
              const half2_t hi = {(half_t)p0, (half_t)p1};
              const half2_t lo = __builtin_bit_cast(half2_t, low_parts(p0, p1, __builtin_bit_cast(uint32_t, hi)));
              pf[qb][s][j] = hi[0];
              pf[qb][s][j + 1] = hi[1];
              pl[qb][s][j] = lo[0];
              pl[qb][s][j + 1] = lo[1];
              psum += p0 + p1;
            }
          l_run[qb] += psum;
        } else {
          // P = exp2(S) rounded to fp16; the row sum adds the same rounded
          // values (a dominant key's rounding then cancels in the normalisation).
#pragma unroll
          for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int j = 0; j < 8; ++j) pf[qb][s][j] = (half_t)fast_exp2(sacc[qb][s / 2][8 * (s % 2) + j]);
          float psum = 0.f;
#pragma unroll
          for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int j = 0; j < 8; j += 2)
              psum = __builtin_amdgcn_fdot2(half2_t{pf[qb][s][j], pf[qb][s][j + 1]},
                                            half2_t{(half_t)1.f, (half_t)1.f}, psum, false);
          l_run[qb] += psum;
        }
      }
      // O^T += V^T P^T over 16-key steps (split heads: V^T (P_hi + P_lo)^T).
#pragma unroll
      for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int db = 0; db < TL::DB; ++db) {
          const half8_t vf = *reinterpret_cast<const half8_t*>(&sm.vt[cur][db * 32 + ln][16 * s + 8 * hl]);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) {
            oacc[qb][db] = mfma32(vf, pf[qb][s], oacc[qb][db]);
            if constexpr (SPLIT) oacc[qb][db] = mfma32(vf, pl[qb][s], oacc[qb][db]);
          }
        }
    }

    if (kt + 1 < n_kv) stage.template store<SPLIT>(sm, cur ^ 1, tid);
    __syncthreads();
  }

  // Epilogue: combine the two half-row sums, normalise, store.
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int qi = qw0 + 32 * qb + ln;
    const float l_tot = pair_sum(l_run[qb]);
    if (qi < row_cap) {
      const bool valid = qi < L && l_tot > 0.f;
      const float inv = valid ? 1.f / l_tot : 0.f;
      // A value bias adds b_v to every valid row (its probabilities sum to 1).
      const float* vb = (valid && a.v_bias != nullptr) ? a.v_bias + h * HD : nullptr;
      T* op = reinterpret_cast<T*>(a.o) + a.vo.row(b, h, qi);
#pragma unroll
      for (int db = 0; db < TL::DB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = db * 32 + 8 * g + 4 * hl;
          const float4_t bv = vb != nullptr ? *reinterpret_cast<const float4_t*>(vb + d0) : float4_t{0.f, 0.f, 0.f, 0.f};
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = oacc[qb][db][4 * g + e] * inv + bv[e];
          if constexpr (sizeof(T) == 4) {
            *reinterpret_cast<float4_t*>(op + d0) = float4_t{y[0], y[1], y[2], y[3]};
          } else {
            *reinterpret_cast<half4_t*>(op + d0) = half4_t{(half_t)y[0], (half_t)y[1], (half_t)y[2], (half_t)y[3]};
          }
        }
    }
  }
}

template <typename T, int HD, int QB, bool SPLIT_OK, int BNT = BN>
__global__ __launch_bounds__(NT, (HD > 128 ? 1 : 2)) void attn_fwd_kernel(AttnArgs a) {
  __shared__ Smem<HD, SPLIT_OK, BNT> sm;

  // XCD-aware tile order: ids x, x+8, x+16, ... run on XCD x.
  const int id = blockIdx.x;
  int bh, mt;
  if (a.balanced) {
    // Row limits concentrate the work on a few (b, h) (e.g. the exact
    // fallback heads of the guarded polynomial route). Query tiles are then
    // issued heaviest first across all (b, h): slot s of rank mrev is id s
    // + mrev * bhn, on XCD s % 8 and, within the XCD, shader engine
    // (mrev * bhn / 8 + s / 8) % 4. With bhn a multiple of 8, (b, h) = 8 g + c
    // takes the slot whose group s / 8 is g + mrev and whose XCD is c + the
    // base-8 digit sum of g + mrev / 4: four consecutive ranks of one (b, h)
    // share an XCD (and its L2 copy of that head's K/V), every (b, h) moves
    // on to the next XCD after them, (b, h) with the same c whose g differ
    // in digit sum mod 8 (heads 0, 16, 32, 48, ...: every B-th of a
    // multiple-of-8 H) sit on different XCDs, and the shader engine turns
    // with the rank. Either way a rank's slots are a permutation of the
    // (b, h).
    const int bhn = a.B * a.H;
    const int mrev = id / bhn;
    const int s = id % bhn;
    if ((bhn & 7) == 0) {
      const int ng = bhn >> 3;
      const int g = ((s >> 3) - mrev % ng + ng) % ng;
      int digits = 0;
      for (int t = g; t > 0; t >>= 3) digits += t;
      bh = 8 * g + ((s - mrev / 4 - digits) & 7);
    } else {
      bh = (s + mrev) % bhn;
    }
    mt = a.n_mtiles - 1 - mrev;
  } else {
    // XCD x owns (b, h) bh0 .. bh0 + nb - 1 (range sizes differ by at most
    // one): the first nseq one after another, the rest in interleaved
    // groups of a.group.
    const int bhn = a.B * a.H;
    const int x = id % kNumXcd;
    const int j = id / kNumXcd;
    const int bh0 = x * bhn / kNumXcd;
    const int nb = (x + 1) * bhn / kNumXcd - bh0;
    const int nseq = nb > 2 * a.group ? nb - a.group : 0;
    int mrev;
    if (j < nseq * a.n_mtiles) {
      bh = bh0 + j / a.n_mtiles;
      mrev = j % a.n_mtiles;
      // An XCD hands consecutive workgroups to its four shader engines in
      // turn and waits for the engine whose turn it is, so each engine must
      // see the same work: heaviest-first in snake rounds of four (ranks
      // 0 1 2 3, 7 6 5 4, 8 9 10 11, ...) gives engine i ranks i, 7-i, 8+i,
      // 15-i, ..., equal sums, where plain heaviest-first gave the first
      // engine the heaviest tile of every round.
      if ((a.n_mtiles & 3) == 0) {
        const int i = j & 3;
        mrev = (mrev & ~3) + (((j >> 2) & 1) ? 3 - i : i);
      }
    } else {
      const int r = j - nseq * a.n_mtiles;
      const int per_group = a.group * a.n_mtiles;
      const int g0 = nseq + r / per_group * a.group;
      if (g0 >= nb) return;
      // Position rr of the group's heaviest-first list (rank rr / gs of
      // (b, h) rr % gs), dealt in the same snake rounds: with two (b, h) per
      // group, plain order gave two engines the heavier rank of every pair.
      int rr = r % per_group;
      if ((a.n_mtiles & 3) == 0) {
        const int i = rr & 3;
        rr = (rr & ~3) + (((rr >> 2) & 1) ? 3 - i : i);
      }
      const int gs = min(a.group, nb - g0);
      mrev = rr / gs;
      if (mrev >= a.n_mtiles) return;
      bh = bh0 + g0 + rr % gs;
    }
    mt = a.n_mtiles - 1 - mrev;
    // Logical (b, h) order runs over samples first, so every XCD's range
    // mixes the samples' valid lengths evenly.
    bh = (bh % a.B) * a.H + bh / a.B;
  }
  const int b = bh / a.H;
  const int h = bh % a.H;
  const int q0 = mt * 128 * QB;
  int row_cap = a.S;
  if (a.row_limit != nullptr) row_cap = min(row_cap, max(0, a.row_limit[bh]));
  if (q0 >= row_cap) return;
  int L = a.S;
  if (a.valid_len != nullptr) L = min(a.S, max(0, a.valid_len[b]));

  if constexpr (SPLIT_OK) {
    if (a.qk_split[bh] != 0) {
      attn_tile<T, HD, QB, true, BNT>(a, sm, b, h, q0, row_cap, L);
      return;
    }
  }
  attn_tile<T, HD, QB, false, BNT>(a, sm, b, h, q0, row_cap, L);
}

template <typename T, int HD, int QB, int BNT = BN>
int launch_qb(AttnArgs a, hipStream_t stream) {
  a.n_mtiles = (a.S + 128 * QB - 1) / (128 * QB);
  const int64_t bhn = int64_t(a.B) * a.H;
  a.balanced = a.row_limit != nullptr || bhn < kNumXcd;
  // About one XCD's worth of workgroup slots per group: 32 CUs x 2.
  a.group = max(1, 64 / a.n_mtiles);
  const int64_t per_xcd = (bhn + kNumXcd - 1) / kNumXcd;
  const int64_t grid = a.balanced ? bhn * a.n_mtiles : kNumXcd * (per_xcd + a.group - 1) * a.n_mtiles;
  if (grid * NT >= (int64_t(1) << 32)) return TJ_ERR_SHAPE;
  if constexpr ((QB == 1 && HD <= 128) || BNT == 32) {
    if (a.qk_split != nullptr) {
      hipLaunchKernelGGL((attn_fwd_kernel<T, HD, QB, true, BNT>), dim3(uint32_t(grid)), dim3(NT), 0, stream, a);
      return tjh::launch_status();
    }
  }
  hipLaunchKernelGGL((attn_fwd_kernel<T, HD, QB, false, BNT>), dim3(uint32_t(grid)), dim3(NT), 0, stream, a);
  return tjh::launch_status();
}
}  // namespace
}  // namespace tj
