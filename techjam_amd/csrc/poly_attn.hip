// Chunked causal degree-2 polynomial linear attention for gfx950 (D = 64, chunk 512).
//
// Replaces the reference's chunk scan (src/implementations/poly_reference.py:162-249)
// and its Triton kernels quad_apply / quad_update / causal_diag
// (src/kernels/poly_attention_triton.py:151-257, :420-591). With a = q*sqrt(scale),
// b = k*sqrt(scale) (fp16) and per-head coefficients (c0, c1, c2), chunk
// [t0, t1) emits for each row i
//   num = c0*S_const + c1*a.S_lin + c2*phi2(a).S_quad + sum_{t0<=j<=i} exp(a_i.b_j) v_j
//   den = c0*t0      + c1*a.z    + c2*a^T G a        + sum_{t0<=j<=i} exp(a_i.b_j)
// and the states fold in the chunk afterwards:
//   S_quad[(i,j), v] += sum_t b_ti b_tj v_tv,  S_lin[j, v] += sum_t b_tj v_tv,
//   G[i, j] += sum_t b_ti b_tj,  z[j] += sum_t b_tj,  S_const[v] += sum_t v_tv.
//
// Launches advance KG = 16 chunks at a time; in launch L every head owns 55
// workgroups with four roles:
//   * apply (2 per chunk, 256 rows each, for the KG chunks whose start
//     states the previous launch produced): quadratic term as
//       y^T = sum_i S_i^T (a_i * a^T)  (S_i = rows (i, .) of S_quad),
//     i.e. 64 MFMA GEMMs whose B operand is the fp16 product a_i*a_j built in
//     registers -- phi2(a) never exists in memory; linear and denominator terms
//     as three more small GEMMs; the exact diagonal block like the exact
//     kernel (S^T = b a^T in registers, no max subtraction).
//   * quad update (6 per head): S_i += (b_i * b)^T v over the tokens of
//     chunks [KG L, KG L + KG), accumulated straight into MFMA accumulators
//     that hold the fp32 master in its register image (the master's memory
//     layout IS the accumulator layout, so loading and storing it is straight
//     16-byte copies, once per launch). After each chunk it writes the fp16
//     shadow of the state the apply of the next chunk reads.
//   * small-state update (1 per head): S_lin, G, z, S_const, likewise.
//   * token images (KG per head): b = k*sqrt(scale) and v of the chunks the
//     next launch folds in, converted once to fp16 tiles laid out as the
//     update roles' LDS image, which those roles then stream with direct
//     global->LDS copies.
// State c (before chunk c) lives in shadow slot c % (2 KG): a launch reads
// the slots of states KG L - KG + 1 .. KG L and writes those of KG L + 1 ..
// KG L + KG, so applies and updates of one launch never touch the same slot.
// More chunks per launch load and store each master less often and need
// fewer launches (the polynomial call on 64 heads of 65536 tokens: 4 -> 8
// chunks 5.8-6.1 -> 5.4-5.5 ms; the extreme step with 8 -> 16 chunks
// 8.99-9.02 -> 8.78-8.83 ms, 10.2 MiB more workspace per head), at the
// price of a longer update chain per launch when few heads share the GPU
// (16 heads of 100 000 tokens: 2.39-2.40 -> 2.42 ms).
// Heads whose guard flag is 0 exit at once (the exact kernel covers them).
#include <type_traits>

#include "tj_common.h"

namespace tj {
namespace {

constexpr int PD = 64;         // head dim (d = dv)
constexpr int PC = 512;        // chunk length
constexpr int PT = 256;        // threads per workgroup
constexpr int NAPPLY = 2;      // apply workgroups per head and chunk (256 rows each)
constexpr int NUPD = 6;        // quad-update workgroups per head (4 for i < 32, 2 for i >= 32)
constexpr int KG = 16;         // chunks per launch (update sub-chunks, apply groups)
constexpr int NSLOT = 2 * KG;  // shadow slots: state_c lives in slot c % NSLOT
constexpr int NCONV = KG;      // token-image workgroups per head (one chunk each)
constexpr int NROLE = KG * NAPPLY + NUPD + 1 + NCONV;
constexpr int LP = 72;         // padded LDS row of 64 halves (144 bytes)
constexpr int kBufferFlags = 0x00020000;  // raw (untyped) buffer resource word 3 on gfx950

// Workspace of one head (byte offsets).
constexpr size_t kQuadImg = 0;                                   // fp32 [64 i][2 jb][2 vb][64 lanes][16]
constexpr size_t kQuadImgBytes = size_t(PD) * 4 * 64 * 16 * 4;  // 1 MiB
constexpr size_t kLinImg = kQuadImg + kQuadImgBytes;             // fp32 [2 jb][2 vb][64][16]
constexpr size_t kGramImg = kLinImg + 4 * 64 * 16 * 4;           // fp32 [2 ib][2 jb][64][16]
constexpr size_t kZsMaster = kGramImg + 4 * 64 * 16 * 4;         // fp32 z[64], S_const[64]
constexpr size_t kQuadShadow = kZsMaster + 128 * 4;              // fp16 [NSLOT][64 i][8 q][64 v][8 j]
constexpr size_t kLinShadow = kQuadShadow + NSLOT * size_t(PD) * PD * PD * 2;  // fp16 [NSLOT][64 v][64 j]
constexpr size_t kGramShadow = kLinShadow + NSLOT * PD * PD * 2;  // fp16 [NSLOT][64][64] (symmetric)
constexpr size_t kZsShadow = kGramShadow + NSLOT * PD * PD * 2;   // fp32 [NSLOT][128]
// Token images: the k (scaled) and v tiles the update roles of a launch fold
// in, written once by the previous launch as fp16 LDS images (see TokTile).
constexpr int kTileImg = 2 * PD * 64 * 2;                          // [b^T | v^T] of 64 tokens
constexpr size_t kTokImgBytes = size_t(KG) * (PC / 64) * kTileImg;  // one launch: 2 MiB
constexpr size_t kTokImg = (kZsShadow + NSLOT * 128 * 4 + 255) & ~size_t(255);  // [2][kTokImgBytes]
constexpr size_t kPerHead = kTokImg + 2 * kTokImgBytes;

// LDS: apply = quad-state ring (49152) or diagonal tiles (36864);
//      updates = two transposed token tiles, double buffered (36864).
constexpr int kRing = 3;                        // quad-state stages in flight
constexpr int kRingStage = 2 * PD * PD * 2;     // one stage: rows of two i, [2][64 v][64 j] fp16
constexpr int kStageBytes = kRing * kRingStage;
static_assert(kStageBytes >= 4 * 64 * LP * 2, "diagonal / update tiles must fit the ring area");
constexpr int kSmemBytes = kStageBytes;

struct PolyArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  View4 vq, vk, vv, vo;
  int H, S;
  float rs;             // sqrt(scale)
  int launch;           // launch index L: applies chunks (KG (L-1), KG L], updates [KG L, KG L + KG)
  int n_chunks;
  int prefix_end;       // rows below are left to the exact kernel
  const float* coeffs;  // [M][3]
  const int32_t* flags; // [M] or null
  char* ws;
  int M;                // B * H
};

__device__ __forceinline__ float4_t ld4(const float* p) { return *reinterpret_cast<const float4_t*>(p); }

template <typename T>
__device__ __forceinline__ void load_row4(const T* p, float out[4]) {
  if constexpr (sizeof(T) == 4) {
    const float4_t x = *reinterpret_cast<const float4_t*>(p);
    out[0] = x[0]; out[1] = x[1]; out[2] = x[2]; out[3] = x[3];
  } else {
    const half4_t x = *reinterpret_cast<const half4_t*>(p);
    out[0] = (float)x[0]; out[1] = (float)x[1]; out[2] = (float)x[2]; out[3] = (float)x[3];
  }
}

// Global -> registers of one 64-token x 64-dim tile of k and v. Unit =
// (4-token group g, 4-dim group c); one unit per thread. Rows are read with
// bounds-checked buffer loads (one resource per (b, h) spanning rows 0..S-1),
// so tokens at or past S read as zeros without a branch, and nothing waits
// on the loads before the tile is stored: k is scaled by rs at the store.
template <typename T>
struct TokTile {
  // Raw rows as loaded (fp32 or fp16), converted at the stores: fp16 input
  // holds half the registers.
  using Raw = std::conditional_t<sizeof(T) == 4, float4_t, half4_t>;
  Raw kx[4];
  Raw vx[4];
  __amdgpu_buffer_rsrc_t rk, rv;
  uint32_t koff, voff, kstep, vstep;
  __device__ __forceinline__ static void coords(int tid, int& g, int& c) {
    g = (tid >> 2) & 15;
    c = (tid & 3) | ((tid >> 6) << 2);
  }
  __device__ __forceinline__ void init(const PolyArgs& a, int b, int h, int tid) {
    int g, c;
    coords(tid, g, c);
    const T* kp = reinterpret_cast<const T*>(a.k) + a.vk.row(b, h, 0);
    const T* vp = reinterpret_cast<const T*>(a.v) + a.vv.row(b, h, 0);
    kstep = (uint32_t)(a.vk.ss * (int64_t)sizeof(T));
    vstep = (uint32_t)(a.vv.ss * (int64_t)sizeof(T));
    const int kbytes = (int)((int64_t)(a.S - 1) * kstep + PD * (int64_t)sizeof(T));
    const int vbytes = (int)((int64_t)(a.S - 1) * vstep + PD * (int64_t)sizeof(T));
    rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(kp), (short)0, kbytes, kBufferFlags);
    rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(vp), (short)0, vbytes, kBufferFlags);
    koff = 4 * g * kstep + 4 * c * (uint32_t)sizeof(T);
    voff = 4 * g * vstep + 4 * c * (uint32_t)sizeof(T);
  }
  __device__ __forceinline__ void load(int tok0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if constexpr (sizeof(T) == 4) {
        const float4_t x = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rk, koff, (tok0 + r) * kstep, 0));
        const float4_t y = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rv, voff, (tok0 + r) * vstep, 0));
        kx[r] = x;
        vx[r] = y;
      } else {
        const half4_t x = __builtin_bit_cast(half4_t, __builtin_amdgcn_raw_buffer_load_b64(rk, koff, (tok0 + r) * kstep, 0));
        const half4_t y = __builtin_bit_cast(half4_t, __builtin_amdgcn_raw_buffer_load_b64(rv, voff, (tok0 + r) * vstep, 0));
        kx[r] = x;
        vx[r] = y;
      }
    }
  }
  // The tile's LDS image for the update roles, stored to global memory:
  // [b^T | v^T], each 64 dim rows of 128 bytes (64 tokens), the eight
  // 16-byte pieces of row d at position piece ^ ((d >> 1) & 7) so that 16
  // lanes reading one piece column of 16 consecutive rows hit distinct banks.
  __device__ __forceinline__ void store_image(char* dst, float rs, int tid) const {
    int g, c;
    coords(tid, g, c);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = 4 * c + e;
      const int off = d * 128 + 16 * ((g >> 1) ^ ((d >> 1) & 7)) + 8 * (g & 1);
      *reinterpret_cast<half4_t*>(dst + off) =
          half4_t{(half_t)((float)kx[0][e] * rs), (half_t)((float)kx[1][e] * rs), (half_t)((float)kx[2][e] * rs),
                  (half_t)((float)kx[3][e] * rs)};
      *reinterpret_cast<half4_t*>(dst + PD * 128 + off) =
          half4_t{(half_t)vx[0][e], (half_t)vx[1][e], (half_t)vx[2][e], (half_t)vx[3][e]};
    }
  }
  // K row-major, V transposed in key_slot order: the diagonal block (as in the exact kernel).
  __device__ __forceinline__ void store_diag(half_t (*kb)[LP], half_t (*vt)[LP], float rs, int tid) const {
    int g, c;
    coords(tid, g, c);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      half4_t hk = {(half_t)((float)kx[r][0] * rs), (half_t)((float)kx[r][1] * rs), (half_t)((float)kx[r][2] * rs),
                    (half_t)((float)kx[r][3] * rs)};
      *reinterpret_cast<half4_t*>(&kb[4 * g + r][4 * c]) = hk;
    }
    const int slot = key_slot(4 * g);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      half4_t hv = {(half_t)vx[0][e], (half_t)vx[1][e], (half_t)vx[2][e], (half_t)vx[3][e]};
      *reinterpret_cast<half4_t*>(&vt[4 * c + e][slot]) = hv;
    }
  }
};

__device__ __forceinline__ half8_t mul8(half8_t x, half_t s) {
  half8_t r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = x[j] * s;
  return r;
}

// ---------------------------------------------------------------------------
// Apply role: rows [row0, row0 + 256) of the chunk; each wave owns RB = 2
// blocks of 32 consecutive rows, so every state fragment read from LDS feeds
// two MFMAs and every ring stage serves 256 rows.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void apply_role(const PolyArgs& a, const char* ws, int b, int h, int m, int c, int qt, char* smem) {
  constexpr int RB = 2;
  constexpr int WROWS = 32 * RB;
  const int t0 = c * PC, t1 = min(a.S, t0 + PC), slot = c % NSLOT;
  const int row0 = t0 + 4 * WROWS * qt;
  if (row0 >= t1 || row0 + 4 * WROWS <= a.prefix_end) return;
  auto kb = reinterpret_cast<half_t(*)[64][LP]>(smem);                  // diag: [2][64][LP]
  auto vt = reinterpret_cast<half_t(*)[64][LP]>(smem + 2 * 64 * LP * 2);  // diag: [2][64][LP]

  const int tid = threadIdx.x, w = tid / kWave, lane = tid % kWave, hl = lane / 32, ln = lane % 32;
  const int qw0 = row0 + WROWS * w;

  // a = fp16(q * rs); B operand slots (hl, j) <-> dim 16*ks + 8*hl + j.
  half8_t aB[RB][4];
  {
    const T* qp = reinterpret_cast<const T*>(a.q);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int qi = qw0 + 32 * rb + ln;
      const bool in = qi < t1;
      const int64_t base = a.vq.row(b, h, in ? qi : t0);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        float x[8];
        load_row4<T>(qp + base + 16 * ks + 8 * hl, x);
        load_row4<T>(qp + base + 16 * ks + 8 * hl + 4, x + 4);
#pragma unroll
        for (int j = 0; j < 8; ++j) aB[rb][ks][j] = in ? (half_t)(x[j] * a.rs) : (half_t)0.f;
      }
    }
  }
  // Linear denominator a.z (z = S_lin's row sums, fp32 in the slot's small
  // shadow), taken while few registers are live.
  const float* zs = reinterpret_cast<const float*>(ws + kZsShadow) + slot * 128;
  float den_l[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    float dl = 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int j = 0; j < 8; ++j) dl += (float)aB[rb][ks][j] * zs[16 * ks + 8 * hl + j];
    den_l[rb] = pair_sum(dl);
  }
  // a_i, a_i+1 (i = 2p) of this lane's query: dword p & 3 of aB[rb][p >> 3],
  // held by the lane half (p >> 2) & 1; the lane-pair swap hands it to both
  // (r[0] from the lower-half lane, r[1] from the upper, as in pair_values).
  auto a_pair = [&](int rb, int p) -> half2_t {
    using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
    const uint32_t u = __builtin_bit_cast(u32x4, aB[rb][p >> 3])[p & 3];
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(half2_t, ((p >> 2) & 1) ? r[1] : r[0]);
  };

  const half_t* qshadow = reinterpret_cast<const half_t*>(ws + kQuadShadow) + size_t(slot) * PD * PD * PD;
  // The fp16 quad shadow of one i is piece-major, [8 q][64 v][8 j]: piece q
  // holds columns j = 8q .. 8q + 7 of every row v (1 KiB contiguous per q).
  // It streams through a ring of kRing LDS stages by direct global->LDS
  // copies two stages ahead of the MFMAs (no registers held). Pair p
  // (i = 2p, 2p + 1) only reads the pieces q >= 2 ib, ib = p >> 3 (S is
  // symmetric, see the step), np = 8 - 2 ib of them per row, so a stage holds
  // G pairs (G = 1, 1, 2, 4 for ib = 0 .. 3, at most 16 KiB) as
  // [gp][q - 2 ib][ii][64 v] 16-byte pieces (1 KiB per (gp, q, ii)), filled
  // by 2 G np copy instructions (k = 2 (gp np + q - 2 ib) + ii; wave w issues
  // k = w, w + 4, ...): 37.5 % fewer bytes than whole rows, 22 stages instead
  // of 32, and 16 lanes reading one piece column of 16 consecutive rows touch
  // 256 contiguous bytes. The stages are distinct members addressed with
  // compile-time indices, so the compiler can tell the copies into one stage
  // from reads of another and does not wait for every copy in flight.
  struct Ring {
    char s0[kRingStage];
    char s1[kRingStage];
    char s2[kRingStage];
  };
  static_assert(kRing == 3, "the ring below has three members");
  Ring& ring = *reinterpret_cast<Ring*>(smem);
  auto stage_ptr = [&](auto st) -> char* {
    if constexpr (decltype(st)::value == 0) return ring.s0;
    else if constexpr (decltype(st)::value == 1) return ring.s1;
    else return ring.s2;
  };
  constexpr int kSteps = 22;
  auto step_p0 = [](int st) constexpr { return st < 16 ? st : (st < 20 ? 16 + 2 * (st - 16) : 24 + 4 * (st - 20)); };
  auto step_g = [](int st) constexpr { return st < 16 ? 1 : (st < 20 ? 2 : 4); };
  auto issue = [&](auto sc, auto st) {
    constexpr int p0 = step_p0(decltype(sc)::value), G = step_g(decltype(sc)::value);
    constexpr int ib = p0 >> 3, np = 8 - 2 * ib;
    static_assert(G * np * 2 <= 16, "a stage holds at most 16 KiB");
    char* base = stage_ptr(st);
#pragma unroll
    for (int it = 0; it < G * np / 2; ++it) {
      const int k = w + 4 * it;
      const int gp = k / (2 * np), rem = k % (2 * np);
      const int q = 2 * ib + (rem >> 1), ii = rem & 1;
      const half_t* src = qshadow + (size_t(2 * (p0 + gp) + ii) * 8 + q) * (PD * 8) + lane * 8;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                       (__attribute__((address_space(3))) void*)(base + k * 1024), 16, 0, 0);
    }
  };

  // accq: the quadratic numerator first; after the ring, scaled by c2 and
  // joined by c1 times the linear term and by the exact diagonal block.
  float16_t accq[RB][2];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int vb = 0; vb < 2; ++vb)
#pragma unroll
      for (int r = 0; r < 16; ++r) accq[rb][vb][r] = 0.f;

  // One ring step: MFMAs on the pairs of stage sc, after issuing stage sc + 2.
  auto step = [&](auto sc) {
    constexpr int si = decltype(sc)::value;
    constexpr int p0 = step_p0(si), G = step_g(si);
    constexpr int ib = p0 >> 3, np = 8 - 2 * ib;  // 16-block of every i of the stage
    if constexpr (si + 2 < kSteps) issue(std::integral_constant<int, si + 2>{}, std::integral_constant<int, (si + 2) % kRing>{});
    const char* base = stage_ptr(std::integral_constant<int, si % kRing>{});
    // phi2(a).S = sum_i a_i sum_j a_j S_ij with S_ij = S_ji (the update forms
    // both from the same fp16 products b_i b_j in the same order): the j-block
    // holding i counts once, j-blocks above it twice (a_i doubled, exact in
    // fp16), j-blocks below it not at -- 37.5 % fewer MFMAs.
#pragma unroll
    for (int gp = 0; gp < G; ++gp) {
      const int p = p0 + gp;
      half2_t ap[RB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) ap[rb] = a_pair(rb, p);
#pragma unroll
      for (int ii = 0; ii < 2; ++ii) {
#pragma unroll
        for (int ks = ib; ks < 4; ++ks) {
          const int k = 2 * (gp * np + 2 * ks + hl - 2 * ib) + ii;
          half8_t sa[2];
#pragma unroll
          for (int vb = 0; vb < 2; ++vb) sa[vb] = *reinterpret_cast<const half8_t*>(base + k * 1024 + (32 * vb + ln) * 16);
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) {
            const half_t ai = ap[rb][ii];
            const half8_t bop = mul8(aB[rb][ks], ks == ib ? ai : (half_t)(ai + ai));
#pragma unroll
            for (int vb = 0; vb < 2; ++vb) accq[rb][vb] = mfma32(sa[vb], bop, accq[rb][vb]);
          }
        }
      }
    }
    // Stage sc + 1 (this wave's copies) must have landed before the barrier;
    // stage sc + 2 (G np / 2 copies of this wave) may stay in flight. A plain
    // barrier: __syncthreads() would also wait for every copy in flight.
    if constexpr (si + 2 < kSteps) {
      constexpr int in_flight = step_g(si + 2) * (8 - 2 * (step_p0(si + 2) >> 3)) / 2;
      __builtin_amdgcn_s_waitcnt(0x0070 | in_flight);  // vmcnt(in_flight) lgkmcnt(0)
    } else {
      __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
    }
    lds_barrier();
  };
  issue(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
  issue(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
  __builtin_amdgcn_s_waitcnt(0x0074);  // stage 0 landed (stage 1: four copies in flight)
  lds_barrier();
  static_for<0, kSteps>(step);

  // Linear numerator term S_lin^T a^T and the quadratic denominator G a^T
  // (operands straight from the L2-resident shadows). G's rows are read in
  // the order that swaps bits 2 and 3 of the row index, so that accumulator
  // element r of this lane holds row 32 blk + 16 (r / 8) + 8 hl + r % 8 --
  // the dims this lane's own aB[rb][2 blk + r / 8][r % 8] holds -- and
  // a^T G a needs no other lane's a.
  const float c0 = a.coeffs[3 * m], c1 = a.coeffs[3 * m + 1], c2 = a.coeffs[3 * m + 2];
  const half_t* lsh = reinterpret_cast<const half_t*>(ws + kLinShadow) + size_t(slot) * PD * PD;
  const half_t* gsh = reinterpret_cast<const half_t*>(ws + kGramShadow) + size_t(slot) * PD * PD;
  const int grow = (ln & 0x13) | ((ln & 4) << 1) | ((ln & 8) >> 1);
  float den_q[RB], den_d[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) den_q[rb] = den_d[rb] = 0.f;
  // One 32-row block of S_lin^T (output block blk = v block) and of G at a time,
  // each fragment feeding both query blocks.
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    half8_t la[4], ga[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      la[ks] = *reinterpret_cast<const half8_t*>(lsh + (32 * blk + ln) * PD + 16 * ks + 8 * hl);
      ga[ks] = *reinterpret_cast<const half8_t*>(gsh + (32 * blk + grow) * PD + 16 * ks + 8 * hl);
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float16_t tl, tg;
#pragma unroll
      for (int r = 0; r < 16; ++r) tl[r] = tg[r] = 0.f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        tl = mfma32(la[ks], aB[rb][ks], tl);
        tg = mfma32(ga[ks], aB[rb][ks], tg);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        den_q[rb] += (float)aB[rb][2 * blk + r / 8][r % 8] * tg[r];
        accq[rb][blk][r] = c2 * accq[rb][blk][r] + c1 * tl[r];
      }
    }
  }
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) den_q[rb] = pair_sum(den_q[rb]);

  // Exact diagonal block: keys [t0, min(t1, row0 + 256)), no max subtraction;
  // the weighted values accumulate straight into accq.
  const int key_end = min(t1, row0 + 4 * WROWS);
  const int n_kt = (key_end - t0 + 63) / 64;
  TokTile<T> tile;
  tile.init(a, b, h, tid);
  tile.load(t0);
  tile.store_diag(kb[0], vt[0], a.rs, tid);
  __syncthreads();
  for (int kt = 0; kt < n_kt; ++kt) {
    const int cur = kt & 1;
    const int kv0 = t0 + 64 * kt;
    if (kt + 1 < n_kt) tile.load(kv0 + 64);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int qb0 = qw0 + 32 * rb;
      const int qi = qb0 + ln;
      // a block whose rows all precede the tile (or lie past the chunk) skips it
      if (kv0 <= min(qb0 + 31, key_end - 1)) {
        float16_t s[2];
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
#pragma unroll
          for (int r = 0; r < 16; ++r) s[kh][r] = 0.f;
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            const half8_t kf = *reinterpret_cast<const half8_t*>(&kb[cur][32 * kh + ln][16 * ks + 8 * hl]);
            s[kh] = mfma32(kf, aB[rb][ks], s[kh]);
          }
        }
        half8_t pf[4];
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kv0 + 32 * kh + 8 * (r / 4) + 4 * hl + (r % 4);
            const float wgt = key <= qi ? fast_exp2(s[kh][r] * 1.4426950408889634f) : 0.f;
            const half_t wh = (half_t)wgt;
            den_d[rb] += (float)wh;
            pf[2 * kh + r / 8][r % 8] = wh;
          }
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
          for (int vb = 0; vb < 2; ++vb) {
            const half8_t vf = *reinterpret_cast<const half8_t*>(&vt[cur][32 * vb + ln][16 * st + 8 * hl]);
            accq[rb][vb] = mfma32(vf, pf[st], accq[rb][vb]);
          }
      }
    }
    if (kt + 1 < n_kt) tile.store_diag(kb[cur ^ 1], vt[cur ^ 1], a.rs, tid);
    __syncthreads();
  }

#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int qi = qw0 + 32 * rb + ln;
    const float dd = pair_sum(den_d[rb]);
    if (qi >= t1 || qi < a.prefix_end) continue;
    const float den = c0 * (float)t0 + c1 * den_l[rb] + c2 * den_q[rb] + dd;
    const float inv = 1.f / den;
    T* op = reinterpret_cast<T*>(a.o) + a.vo.row(b, h, qi);
#pragma unroll
    for (int vb = 0; vb < 2; ++vb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int v0 = 32 * vb + 8 * g + 4 * hl;
        const float4_t sc = ld4(zs + 64 + v0);
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = (c0 * sc[e] + accq[rb][vb][4 * g + e]) * inv;
        if constexpr (sizeof(T) == 4) {
          *reinterpret_cast<float4_t*>(op + v0) = float4_t{y[0], y[1], y[2], y[3]};
        } else {
          *reinterpret_cast<half4_t*>(op + v0) = half4_t{(half_t)y[0], (half_t)y[1], (half_t)y[2], (half_t)y[3]};
        }
      }
  }
}

// ---------------------------------------------------------------------------
// Update roles: fold the chunk's tokens into the states.
// ---------------------------------------------------------------------------

// The token images of the chunks this launch folds in stream through a ring
// of three LDS stages by direct global->LDS copies issued two tiles ahead (no
// registers held). body(bT, vT) runs on every 64-token tile (b^T and v^T, 64
// dim rows of 128 bytes with XOR-placed 16-byte pieces, see img_piece);
// chunk_end(j) after the last tile of the launch's j-th chunk, once the
// workgroup has passed that tile's barrier: its global stores then complete
// under the next tile instead of holding up the wait for the copies (issued
// before them) that the barrier needs. The stages are
// distinct members addressed with compile-time indices, so the compiler can
// tell the copies into one stage from the reads of another.
struct TokRing {
  char s0[kTileImg];
  char s1[kTileImg];
  char s2[kTileImg];
};
static_assert(sizeof(TokRing) <= kStageBytes, "the token ring must fit the ring area");

// Tokens 8 pc .. 8 pc + 7 of dim row `row` of a tile image.
__device__ __forceinline__ half8_t img_piece(const half_t* base, int row, int pc) {
  return *reinterpret_cast<const half8_t*>(reinterpret_cast<const char*>(base) + row * 128 + 16 * (pc ^ ((row >> 1) & 7)));
}

template <typename Body, typename ChunkEnd>
__device__ __forceinline__ void stream_image(const char* img, int n_chunk, char* smem, Body&& body,
                                             ChunkEnd&& chunk_end) {
  constexpr int kTiles = PC / 64;
  TokRing& ring = *reinterpret_cast<TokRing*>(smem);
  const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int n = n_chunk * kTiles;
  auto stage_ptr = [&](auto st) -> char* {
    if constexpr (decltype(st)::value == 0) return ring.s0;
    else if constexpr (decltype(st)::value == 1) return ring.s1;
    else return ring.s2;
  };
  // Copy instruction `it` of wave w moves 1 KiB slot 4 it + w of the tile.
  auto issue = [&](int t, auto st) {
    char* base = stage_ptr(st);
    const char* src = img + size_t(t) * kTileImg;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int slot = 4 * it + w;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + slot * 1024 + lane * 16),
                                       (__attribute__((address_space(3))) void*)(base + slot * 1024), 16, 0, 0);
    }
  };
  // Tile t + 1 (this wave's four copies) must have landed before the barrier;
  // tile t + 2 may stay in flight (anything issued after it only makes the
  // wait longer). A plain barrier: __syncthreads() would also wait for every
  // copy in flight.
  auto wait_next = [&](int t) {
    if (t + 2 < n) __builtin_amdgcn_s_waitcnt(0x0074);  // vmcnt(4) lgkmcnt(0)
    else __builtin_amdgcn_s_waitcnt(0x0070);            // vmcnt(0) lgkmcnt(0)
    lds_barrier();
  };
  auto step = [&](int t, auto st) {
    constexpr int sv = decltype(st)::value;
    if (t + 2 < n) issue(t + 2, std::integral_constant<int, (sv + 2) % 3>{});
    const char* base = stage_ptr(st);
    body(reinterpret_cast<const half_t*>(base), reinterpret_cast<const half_t*>(base + PD * 128));
    wait_next(t);
    if ((t + 1) % kTiles == 0) chunk_end(t / kTiles);
  };
  if (n == 0) return;
  issue(0, std::integral_constant<int, 0>{});
  if (n > 1) issue(1, std::integral_constant<int, 1>{});
  wait_next(-1);
  for (int t = 0; t < n; t += 3) {
    step(t, std::integral_constant<int, 0>{});
    if (t + 1 < n) step(t + 1, std::integral_constant<int, 1>{});
    if (t + 2 < n) step(t + 2, std::integral_constant<int, 2>{});
  }
}

__device__ __forceinline__ void load_img(const float* img, float16_t& acc) {
  const int lane = threadIdx.x % kWave;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4_t x = ld4(img + lane * 16 + 4 * q);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[4 * q + e] = x[e];
  }
}

__device__ __forceinline__ void store_img(float* img, const float16_t& acc) {
  const int lane = threadIdx.x % kWave;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    *reinterpret_cast<float4_t*>(img + lane * 16 + 4 * q) = float4_t{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
}

// acc holds D[row][col] of a 32x32 block (rows 32*rb + ..., column 32*cb + ln);
// writes it transposed as fp16 into dst[col][row] (row-contiguous, 4 rows per store).
__device__ __forceinline__ void store_shadow_t(half_t* dst, const float16_t& acc, int rb, int cb) {
  const int lane = threadIdx.x % kWave, hl = lane / 32, ln = lane % 32;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int row = 32 * rb + 8 * g + 4 * hl;
    *reinterpret_cast<half4_t*>(dst + (32 * cb + ln) * PD + row) =
        half4_t{(half_t)acc[4 * g], (half_t)acc[4 * g + 1], (half_t)acc[4 * g + 2], (half_t)acc[4 * g + 3]};
  }
}

// The same block written into the piece-major quad shadow of S_i,
// [8 q][64 v][8 j] (q = j / 8), as the apply's ring reads it, from row group
// g0 on (g0 = 2 skips j = 32 rb .. 32 rb + 15).
__device__ __forceinline__ void store_quad_shadow(half_t* dst, const float16_t& acc, int rb, int cb, int g0) {
  const int lane = threadIdx.x % kWave, hl = lane / 32, ln = lane % 32;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    if (g < g0) continue;
    const int j = 32 * rb + 8 * g + 4 * hl;  // four consecutive j, one piece
    *reinterpret_cast<half4_t*>(dst + ((j >> 3) * 64 + 32 * cb + ln) * 8 + (j & 7)) =
        half4_t{(half_t)acc[4 * g], (half_t)acc[4 * g + 1], (half_t)acc[4 * g + 2], (half_t)acc[4 * g + 3]};
  }
}

// Chunks whose states this launch folds in: [c0, c1) (the final chunk's
// update is never needed).
__device__ __forceinline__ void update_range(const PolyArgs& a, int& c0, int& c1) {
  c0 = KG * a.launch;
  c1 = min(c0 + KG, a.n_chunks - 1);
}

// NI i-slices per wave, j-blocks JB0..1 (the apply never reads j < 32 for
// i >= 32: S is symmetric).
template <int NI, int JB0>
__device__ __forceinline__ void quad_update_body(const PolyArgs& a, char* ws, int i0, char* smem) {
  int c0, c1;
  update_range(a, c0, c1);
  if (c0 >= c1) return;
  constexpr int NJ = 2 - JB0;
  const int lane = threadIdx.x % kWave, hl = lane / 32, ln = lane % 32;
  float* img = reinterpret_cast<float*>(ws + kQuadImg);
  // acc[ii][jj][vb] = D[j][v] block (jb = JB0 + jj) of S_{i0+ii}. The fp32
  // master stays in these registers across the launch's chunks.
  float16_t acc[NI][NJ][2];
#pragma unroll
  for (int ii = 0; ii < NI; ++ii)
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
      for (int vb = 0; vb < 2; ++vb) load_img(img + ((size_t(i0 + ii) * 2 + JB0 + jj) * 2 + vb) * 1024, acc[ii][jj][vb]);

  const char* tok = ws + kTokImg + size_t(a.launch & 1) * kTokImgBytes;
  stream_image(
      tok, c1 - c0, smem,
      [&](const half_t* bT, const half_t* vT) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const int pc = 2 * ks + hl;  // tokens 16 ks + 8 hl .. +7 of the tile
          half8_t bj[NJ], vv[2];
#pragma unroll
          for (int jj = 0; jj < NJ; ++jj) bj[jj] = img_piece(bT, 32 * (JB0 + jj) + ln, pc);
#pragma unroll
          for (int x = 0; x < 2; ++x) vv[x] = img_piece(vT, 32 * x + ln, pc);
#pragma unroll
          for (int ii = 0; ii < NI; ++ii) {
            const half8_t bi = img_piece(bT, i0 + ii, pc);
#pragma unroll
            for (int jj = 0; jj < NJ; ++jj) {
              half8_t phi;
#pragma unroll
              for (int j = 0; j < 8; ++j) phi[j] = bj[jj][j] * bi[j];
#pragma unroll
              for (int vb = 0; vb < 2; ++vb) acc[ii][jj][vb] = mfma32(phi, vv[vb], acc[ii][jj][vb]);
            }
          }
        }
      },
      [&](int j) {
        // fp16 shadow of state_{c+1} for the applies of the next launch: only
        // the pieces the apply reads. For i in 16..31 and 48..63 it skips the
        // 16 columns j below i's own 16-block (S is symmetric), which are the
        // first half of this wave's first j-block.
        const int c = c0 + j;
        half_t* sh = reinterpret_cast<half_t*>(ws + kQuadShadow) + size_t((c + 1) % NSLOT) * PD * PD * PD;
#pragma unroll
        for (int ii = 0; ii < NI; ++ii)
#pragma unroll
          for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
            for (int vb = 0; vb < 2; ++vb)
              store_quad_shadow(sh + size_t(i0 + ii) * PD * PD, acc[ii][jj][vb], JB0 + jj, vb,
                                jj == 0 && ((i0 + ii) & 16) ? 2 : 0);
      });
#pragma unroll
  for (int ii = 0; ii < NI; ++ii)
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
      for (int vb = 0; vb < 2; ++vb) store_img(img + ((size_t(i0 + ii) * 2 + JB0 + jj) * 2 + vb) * 1024, acc[ii][jj][vb]);
}

// Quad-update workgroups 0..3: i < 32, two slices per wave, both j-blocks;
// workgroups 4..5: i >= 32, four slices per wave, j >= 32 only -- the same
// MFMA count per wave.
__device__ __forceinline__ void quad_update_role(const PolyArgs& a, char* ws, int ug, char* smem) {
  const int w = threadIdx.x / kWave;
  if (ug < 4) quad_update_body<2, 0>(a, ws, 8 * ug + 2 * w, smem);
  else quad_update_body<4, 1>(a, ws, 32 + 16 * (ug - 4) + 4 * w, smem);
}

__device__ __forceinline__ void small_update_role(const PolyArgs& a, char* ws, char* smem) {
  int c0, c1;
  update_range(a, c0, c1);
  if (c0 >= c1) return;
  const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave, hl = lane / 32, ln = lane % 32;
  float* lin_img = reinterpret_cast<float*>(ws + kLinImg);
  float* gram_img = reinterpret_cast<float*>(ws + kGramImg);
  float* zs = reinterpret_cast<float*>(ws + kZsMaster);
  float16_t acc[2][2];
  if (w < 2) {
    float* img = w == 0 ? lin_img : gram_img;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) load_img(img + (rb * 2 + cb) * 1024, acc[rb][cb]);
  }
  float z = 0.f, cs = 0.f;
  if (w == 2) {
    z = zs[lane];
    cs = zs[64 + lane];
  }
  float zsum = 0.f, csum = 0.f;
  const char* tok = ws + kTokImg + size_t(a.launch & 1) * kTokImgBytes;
  stream_image(
      tok, c1 - c0, smem,
      [&](const half_t* bT, const half_t* vT) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const int pc = 2 * ks + hl;
          if (w == 0) {  // S_lin[j][v] = sum_t b_tj v_tv
#pragma unroll
            for (int jb = 0; jb < 2; ++jb) {
              const half8_t bj = img_piece(bT, 32 * jb + ln, pc);
#pragma unroll
              for (int vb = 0; vb < 2; ++vb) acc[jb][vb] = mfma32(bj, img_piece(vT, 32 * vb + ln, pc), acc[jb][vb]);
            }
          } else if (w == 1) {  // G[i][j] = sum_t b_ti b_tj
#pragma unroll
            for (int ib = 0; ib < 2; ++ib) {
              const half8_t bi = img_piece(bT, 32 * ib + ln, pc);
#pragma unroll
              for (int jb = 0; jb < 2; ++jb) acc[ib][jb] = mfma32(bi, img_piece(bT, 32 * jb + ln, pc), acc[ib][jb]);
            }
          } else if (w == 2) {  // z[d] and S_const[d]: lane = dim, 16 tokens per step
#pragma unroll
            for (int half = 0; half < 2; ++half) {
              const half8_t bx = img_piece(bT, lane, 2 * ks + half);
              const half8_t vx = img_piece(vT, lane, 2 * ks + half);
#pragma unroll
              for (int j = 0; j < 8; ++j) {
                zsum += (float)bx[j];
                csum += (float)vx[j];
              }
            }
          }
        }
      },
      [&](int j) {
        const int nxt = (c0 + j + 1) % NSLOT;
        if (w == 0) {
          half_t* sh = reinterpret_cast<half_t*>(ws + kLinShadow) + size_t(nxt) * PD * PD;  // [v][j]
#pragma unroll
          for (int jb = 0; jb < 2; ++jb)
#pragma unroll
            for (int vb = 0; vb < 2; ++vb) store_shadow_t(sh, acc[jb][vb], jb, vb);
        } else if (w == 1) {
          half_t* sh = reinterpret_cast<half_t*>(ws + kGramShadow) + size_t(nxt) * PD * PD;  // symmetric
#pragma unroll
          for (int ib = 0; ib < 2; ++ib)
#pragma unroll
            for (int jb = 0; jb < 2; ++jb) store_shadow_t(sh, acc[ib][jb], ib, jb);
        } else if (w == 2) {
          z += zsum;
          cs += csum;
          zsum = csum = 0.f;
          float* zsh = reinterpret_cast<float*>(ws + kZsShadow) + nxt * 128;
          zsh[lane] = z;
          zsh[64 + lane] = cs;
        }
      });
  if (w == 0) {
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int vb = 0; vb < 2; ++vb) store_img(lin_img + (jb * 2 + vb) * 1024, acc[jb][vb]);
  } else if (w == 1) {
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) store_img(gram_img + (ib * 2 + jb) * 1024, acc[ib][jb]);
  } else if (w == 2) {
    zs[lane] = z;
    zs[64 + lane] = cs;
  }
}

// Token images of the chunks the next launch folds in, [KG (L+1), KG (L+1) +
// KG): chunk j of them by workgroup j, eight 64-token tiles, loads of the next
// tile in flight while the current one is stored.
template <typename T>
__device__ void image_role(const PolyArgs& a, char* ws, int b, int h, int j) {
  const int cn = KG * (a.launch + 1);
  const int c = cn + j;
  if (c >= min(cn + KG, a.n_chunks - 1)) return;
  char* dst = ws + kTokImg + size_t((a.launch + 1) & 1) * kTokImgBytes + size_t(j) * (PC / 64) * kTileImg;
  const int tid = threadIdx.x;
  TokTile<T> x0, x1;
  x0.init(a, b, h, tid);
  x1.init(a, b, h, tid);
  x0.load(c * PC);
#pragma unroll
  for (int blk = 0; blk < PC / 64; blk += 2) {
    x1.load(c * PC + 64 * (blk + 1));
    x0.store_image(dst + blk * kTileImg, a.rs, tid);
    if (blk + 2 < PC / 64) x0.load(c * PC + 64 * (blk + 2));
    x1.store_image(dst + (blk + 1) * kTileImg, a.rs, tid);
  }
}

// Roles of one head in launch L: NUPD quad-update workgroups and one
// small-state update folding in chunks [KG L, KG L + KG); KG * NAPPLY apply
// workgroups (chunk KG (L-1) + 1 + j / NAPPLY, row block j % NAPPLY; launch 0
// applies chunk 0 only); NCONV workgroups writing the token images of the
// chunks launch L + 1 folds in. Launch -1 writes only the images for launch 0.
// Head m runs on XCD m % 8 (its roles share that L2); each XCD issues the
// roles of its heads role-major in that order, longest first.
template <typename T>
__global__ __launch_bounds__(PT, 2) void poly_chunk_kernel(PolyArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[kSmemBytes];
  const int x = blockIdx.x % kNumXcd, k = blockIdx.x / kNumXcd;
  const int nh = x < a.M ? (a.M - x + kNumXcd - 1) / kNumXcd : 0;  // heads on this XCD
  if (k >= nh * NROLE) return;
  const int rr = k / nh;
  const int m = x + kNumXcd * (k % nh);
  if (a.flags != nullptr && a.flags[m] == 0) return;
  const int b = m / a.H, h = m % a.H;
  char* ws = a.ws + size_t(m) * kPerHead;
  if (rr >= NUPD + 1 + KG * NAPPLY) {
    image_role<T>(a, ws, b, h, rr - (NUPD + 1 + KG * NAPPLY));
  } else if (a.launch < 0) {
    return;
  } else if (rr < NUPD) {
    quad_update_role(a, ws, rr, smem);
  } else if (rr == NUPD) {
    small_update_role(a, ws, smem);
  } else {
    const int role = rr - (NUPD + 1);
    const int g = role / NAPPLY;
    const int c = a.launch == 0 ? (g == 0 ? 0 : -1) : KG * (a.launch - 1) + 1 + g;
    if (c >= 0 && c < a.n_chunks) apply_role<T>(a, ws, b, h, m, c, role % NAPPLY, smem);
  }
}

// Clears what must start at zero in every head's workspace: the fp32 masters
// and shadow slot 0 (state 0, read by launch 0's apply of chunk 0). Every
// other slot and the token images are written before they are read. The
// masters and quad slot 0 are one contiguous range, split over kZeroParts
// workgroups per head; part 0 also clears the small shadows' slot 0.
constexpr int kZeroParts = 8;
constexpr size_t kZeroMain = kQuadShadow + size_t(PD) * PD * PD * 2;  // masters + quad slot 0

__device__ __forceinline__ void zero_range(uint8_t* p, size_t bytes, size_t lane, size_t lanes) {
  float4_t* q = reinterpret_cast<float4_t*>(p);
  for (size_t i = lane; i < bytes / 16; i += lanes) q[i] = float4_t{0.f, 0.f, 0.f, 0.f};
}

__global__ void zero_state_kernel(uint8_t* ws, int M) {
  const int m = blockIdx.x / kZeroParts, part = blockIdx.x % kZeroParts;
  if (m >= M) return;
  uint8_t* h = ws + size_t(m) * kPerHead;
  constexpr size_t kSlice = kZeroMain / kZeroParts;
  static_assert(kZeroMain % (16 * kZeroParts) == 0, "slices of whole float4s");
  zero_range(h + part * kSlice, kSlice, threadIdx.x, blockDim.x);
  if (part == 0) {
    zero_range(h + kLinShadow, size_t(PD) * PD * 2, threadIdx.x, blockDim.x);
    zero_range(h + kGramShadow, size_t(PD) * PD * 2, threadIdx.x, blockDim.x);
    zero_range(h + kZsShadow, 128 * 4, threadIdx.x, blockDim.x);
  }
}

template <typename T>
int run(PolyArgs a, size_t ws_bytes, hipStream_t stream) {
  (void)ws_bytes;
  hipLaunchKernelGGL(zero_state_kernel, dim3(unsigned(a.M * kZeroParts)), dim3(256), 0, stream,
                     reinterpret_cast<uint8_t*>(a.ws), a.M);
  if (hipGetLastError() != hipSuccess) return TJ_ERR_LAUNCH;
  const dim3 grid(unsigned(kNumXcd * ((a.M + kNumXcd - 1) / kNumXcd) * NROLE));
  if (a.n_chunks > 1) {  // token images of the chunks launch 0 folds in
    a.launch = -1;
    hipLaunchKernelGGL(poly_chunk_kernel<T>, grid, dim3(PT), 0, stream, a);
    if (hipGetLastError() != hipSuccess) return TJ_ERR_LAUNCH;
  }
  // Launch L applies chunks (KG (L-1), KG L] and folds in chunks [KG L, KG L + KG).
  const int n_launch = 1 + (a.n_chunks - 1 + KG - 1) / KG;
  for (int L = 0; L < n_launch; ++L) {
    const int last_applied = min(KG * L, a.n_chunks - 1);
    const bool emits = min(a.S, (last_applied + 1) * PC) > a.prefix_end;
    const bool updates = KG * L < a.n_chunks - 1;
    if (!emits && !updates) continue;
    a.launch = L;
    hipLaunchKernelGGL(poly_chunk_kernel<T>, grid, dim3(PT), 0, stream, a);
    if (hipGetLastError() != hipSuccess) return TJ_ERR_LAUNCH;
  }
  return TJ_OK;
}

}  // namespace
}  // namespace tj

extern "C" size_t tj_poly_workspace_bytes(int64_t B, int64_t H, int64_t S, int64_t D, int64_t chunk) {
  (void)S;
  (void)chunk;
  if (B <= 0 || H <= 0 || D != tj::PD) return 0;
  if (!tjh::product_below(std::numeric_limits<int64_t>::max() / int64_t(tj::kPerHead), {B, H})) return 0;
  return size_t(B * H) * tj::kPerHead;
}

extern "C" int tj_poly_attn_fwd(const void* q, const void* k, const void* v, void* o, int dtype,
                                int64_t B, int64_t H, int64_t S, int64_t D,
                                const int64_t q_strides[4], const int64_t k_strides[4],
                                const int64_t v_strides[4], const int64_t o_strides[4],
                                float scale, int64_t chunk, int64_t exact_prefix,
                                const float* coeffs, const int32_t* flags,
                                void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (dtype != TJ_F32 && dtype != TJ_F16) return TJ_ERR_DTYPE;
  if (B < 0 || H <= 0 || S < 0 || D <= 0 || chunk <= 0 || exact_prefix < 0 || !(scale > 0.f)) return TJ_ERR_SHAPE;
  if (D != tj::PD || chunk != tj::PC) return TJ_ERR_UNSUPPORTED;
  if (B == 0 || S == 0 || exact_prefix >= S) return TJ_OK;
  if (S >= (int64_t(1) << 30) ||
      !tjh::product_below((int64_t(1) << 31) / tj::NROLE - tj::kNumXcd, {B, H}))
    return TJ_ERR_SHAPE;
  if (!q || !k || !v || !o || !coeffs) return TJ_ERR_SHAPE;
  if (!tjh::view_ok(q, q_strides, dtype) || !tjh::view_ok(k, k_strides, dtype) ||
      !tjh::view_ok(v, v_strides, dtype) || !tjh::view_ok(o, o_strides, dtype))
    return TJ_ERR_ALIGN;
  // K and V rows of one (b, h) are addressed with 31-bit byte offsets.
  for (const int64_t* st : {k_strides, v_strides})
    if (!tjh::span_below_2g(S, st[2], D, tjh::elem_size(dtype))) return TJ_ERR_UNSUPPORTED;
  const size_t need = size_t(B * H) * tj::kPerHead;
  if (workspace == nullptr || workspace_bytes < need || !tjh::aligned16(workspace)) return TJ_ERR_WORKSPACE;

  tj::PolyArgs a;
  a.q = q; a.k = k; a.v = v; a.o = o;
  a.vq = {q_strides[0], q_strides[1], q_strides[2]};
  a.vk = {k_strides[0], k_strides[1], k_strides[2]};
  a.vv = {v_strides[0], v_strides[1], v_strides[2]};
  a.vo = {o_strides[0], o_strides[1], o_strides[2]};
  a.H = (int)H; a.S = (int)S;
  a.rs = sqrtf(scale);
  a.prefix_end = (int)exact_prefix;
  a.coeffs = coeffs;
  a.flags = flags;
  a.ws = static_cast<char*>(workspace);
  a.M = (int)(B * H);
  a.n_chunks = (int)((S + tj::PC - 1) / tj::PC);
  if (dtype == TJ_F32) return tj::run<float>(a, need, stream);
  return tj::run<half_t>(a, need, stream);
}
