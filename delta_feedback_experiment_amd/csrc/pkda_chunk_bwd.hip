// Chunked PKDA backward for gfx950 (per-head gate).
//
// Forward chunk algebra (chunk of C = 64 tokens, entering state S0 = h,
// chunk-local cumulative log-decay G, scale s):
//   Akk[t,x] = beta_t e^{G_t-G_x} (k_t . kw_x)  (x < t),   T = (I + Akk)^-1
//   Bw = diag(beta e^G) K,  Bv = diag(beta) V,  W = T Bw,  u = T Bv
//   U = u - W S0,  Aqk[t,x] = s e^{G_t-G_x} (q_t . kw_x)  (x <= t)
//   O = Qg S0 + Aqk U,  Qg = diag(s e^G) Q;   S_C = e^{G_C} S0 + Kg^T U,  Kg = diag(e^{G_C-G}) KW
// Backward, given dO and the gradient dS_C (= dh) of the state leaving the chunk:
//   dU  = Aqk^T dO + Kg dS_C                          (reverse state pass)
//   dS0 = e^{G_C} dS_C + Qg^T dO - W^T dU             (reverse state pass)
//   dQg = dO S0^T,  dW = -dU S0^T,  dKg = U dS_C^T,  dAqk = dO U^T
//   dBw = T^T dW,  dBv = T^T dU,  dT = dW Bw^T + dU Bv^T,  dAkk = -T^T dT T^T
// and the pairwise terms of Akk and Aqk.  The gate gradient follows from
// the gradients themselves: for every row r,
//   dG_r = sum_c (q dq + k dk - kw dkw)[r, c]
// with dk the read-key and dkw the write-key gradient of this chunk, plus, on
// the chunk's last row, e^{G_C} sum(S0 * dS_C) + sum(Kg * dKg).  Two parts of
// that sum are O(1) and cancel exactly: the diagonal pairs of Aqk (decay
// e^0; s dAqk[t,t] q_t kw_t enters q dq and kw dkw alike) and the last row's
// kw dKg (decay e^{G_C - G_C}; it enters -kw dkw and sum(Kg * dKg) alike).
// Both are left out of dG, which then sums only terms that carry a decay
// factor: under strong decay dG is ~e^g smaller than its terms were, and
// forming it as the difference would lose that factor in FP32 rounding.
//
// Two kernels:
//   state_bwd -- per (document, head, BV value columns), reverse over chunks,
//                dS in MFMA accumulators; writes dh (= dS_C per chunk), dU
//                (activation dtype) and dS0 of the document.
//   fused_bwd -- per (chunk, head), 8 waves: everything else, with every
//                intermediate in LDS or registers; writes dq, dk, dkw, dv,
//                dbeta and the cumulative-gate gradient once.
// Every reduction has a fixed order: results are bitwise reproducible.
#include <type_traits>

#include "pkda_chunk_common.h"

namespace pkda {
namespace {

constexpr int kFW = 512;  // fused kernel: 8 waves

struct BwdParams {
  ChunkGeom geom;
  int H;
  const void* q;
  const void* k;
  const void* kw;
  const void* v;
  const float* gcum;
  const float* beta;
  float scale;
  const void* w;
  const void* u;    // U (the forward stores the corrected values here)
  const void* aqk;
  const void* akk;  // T = (I + Akk)^-1
  const void* h;
  const void* dO;
  const float* dht;
  void* dh;
  void* du;
  void* dq;   // dq, dk, dkw, dv: FP32 or the activation dtype (kernel template OT)
  void* dk;
  void* dkw;
  void* dv;
  float* dbeta;
  float* dgcum;
  float* dh0;
  bool kw_is_k;
  const void* qg;  // per-channel gates: s e^G q
  const void* kg;  // per-channel gates: e^{G_last - G} kw
  const float* kw32;  // per-channel gates: kw in FP32 (BF16 kw otherwise), or null
  const float* gcum_lo;  // FP32 per-channel gates, optional: gcum's FP64 remainder
  bool tri_packed;       // BF16, per-head gate, kw = k: Aqk and T as their ten lower blocks
  // BF16, per-head gate, kw = k, BF16 dq, dk, dv (the four-wave backward): the
  // reverse pass writes dv = beta dBv, the final output, instead of dBv, and
  // dBv only for rows with |beta| < 1e-20 (into du); the per-chunk kernel
  // takes dBv = dv / beta.
  bool dv_handoff;
};

// Deterministic sum of one value per thread over an NT-thread workgroup.
template <int NT>
__device__ __forceinline__ float block_sum(float x, float* s_red) {
  s_red[threadIdx.x] = x;
  __syncthreads();
  for (int off = NT / 2; off > 0; off >>= 1) {
    if (threadIdx.x < off) s_red[threadIdx.x] += s_red[threadIdx.x + off];
    __syncthreads();
  }
  const float r = s_red[0];
  __syncthreads();
  return r;
}

// Sum over the 16 lanes that share lane >> 4 (one accumulator row), fixed order.
__device__ __forceinline__ float group16_sum(float x) { return lane_group_sum<16>(x); }

// Sum over the 64 lanes of a wave, fixed order; every lane gets the result.
__device__ __forceinline__ float wave_sum(float x) {
  x = group16_sum(x);
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

// ---------------------------------------------------------------------------
// reverse state pass
//
// One workgroup per (document, head, BV value columns), chunks in reverse;
// dS [D x BV] in MFMA accumulators.  The previous chunk's tiles (KW, Q, W,
// Aqk, dO, G) are loaded into registers while the current chunk computes.
// Per chunk (decays on accumulator rows or on dO, never on loaded tiles):
//   dU = Aqk^T dO + diag(e^{G_C - G}) (KW dS)      -> du (activation dtype)
//   dS <- e^{G_C} dS + Q^T diag(s e^G) dO - W^T dU
// ---------------------------------------------------------------------------
template <typename T, int D, int BV>
struct StateBwdLayout {
  static constexpr int LD = D + Pad<T>::v;
  static constexpr int LDV = BV + Pad<T>::v;
  static constexpr int LDC = C + Pad<T>::v;
  static constexpr int off_dS = 0;                                    // [D][LDV]  dS_C slice
  static constexpr int off_KW = off_dS + D * LDV * (int)sizeof(T);    // [64][LD]
  static constexpr int off_Q = off_KW + C * LD * (int)sizeof(T);      // [64][LD]
  static constexpr int off_W = off_Q + C * LD * (int)sizeof(T);       // [64][LD]
  static constexpr int off_Aqk = off_W + C * LD * (int)sizeof(T);     // [64][LDC]
  static constexpr int off_dO = off_Aqk + C * LDC * (int)sizeof(T);   // [64][LDV]
  static constexpr int off_dOg = off_dO + C * LDV * (int)sizeof(T);   // [64][LDV]  s e^G dO
  static constexpr int off_dUn = off_dOg + C * LDV * (int)sizeof(T);  // [64][LDV]  -dU
  static constexpr int off_gam = off_dUn + C * LDV * (int)sizeof(T);
  static constexpr int off_gc = off_gam + C * 4;                       // [D] last-row G (per channel)
  static constexpr int bytes = off_gc + D * 4;
};

// PC: per-channel gate -- kg and qg come precomputed from the forward, no row
// scaling applies and dS decays row by row.
template <typename T, int D, int BV, bool PC>
__global__ __launch_bounds__(state_threads(D, BV)) void chunk_state_bwd_kernel(BwdParams p) {
  using L = StateBwdLayout<T, D, BV>;
  using E = T;
  constexpr int kSW = state_threads(D, BV);
  constexpr int NW = kSW / 64;
  constexpr int NCT = BV / 16;
  constexpr int NS = (D / 16) * NCT / NW;
  constexpr int NRT = 4 * NCT;  // 16x16 tiles of a [64 x BV] chunk operand
  static_assert(NS * NW == (D / 16) * NCT, "state tiles split evenly over the waves");
  extern __shared__ __attribute__((aligned(16))) char smem[];
  E* sdS = reinterpret_cast<E*>(smem + L::off_dS);
  E* sKW = reinterpret_cast<E*>(smem + L::off_KW);
  E* sQ = reinterpret_cast<E*>(smem + L::off_Q);
  E* sW = reinterpret_cast<E*>(smem + L::off_W);
  E* sAqk = reinterpret_cast<E*>(smem + L::off_Aqk);
  E* sdO = reinterpret_cast<E*>(smem + L::off_dO);
  E* sdOg = reinterpret_cast<E*>(smem + L::off_dOg);
  E* sdUn = reinterpret_cast<E*>(smem + L::off_dUn);
  float* sGam = reinterpret_cast<float*>(smem + L::off_gam);
  float* sGC = reinterpret_cast<float*>(smem + L::off_gc);

  const DocSlot ds = doc_slot(p.geom, p.H, D / BV);
  const int n = ds.n, h = ds.h, v0 = ds.z * BV;
  const int H = p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t gs = (int64_t)H * D;
  int first, count, dstart, dlen;
  doc_chunks(p.geom, n, first, count, dstart, dlen);

  f32x4 dS[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const int ti = wave * NS + i;
    const int rt = ti / NCT, ct = ti % NCT;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = 16 * rt + acc_row(lane, j), c = v0 + 16 * ct + acc_col(lane);
      dS[i][j] = p.dht ? p.dht[((int64_t)n * H + h) * D * D + r * D + c] : 0.f;
    }
  }
  RegTile<kSW, C, D, T> rKW, rQ, rW;
  RegTile<kSW, C, C, T> rA;
  RegTile<kSW, C, BV, T> rdO;
  float rg = 0.f;
  auto prefetch = [&](int jc) {
    const int cstart = dstart + jc * C;
    const int clen = min(C, dlen - jc * C);
    const int64_t row0 = (int64_t)cstart * H + h;
    rKW.load(static_cast<const T*>(PC ? p.kg : p.kw) + row0 * D, gs, clen);
    rQ.load(static_cast<const T*>(PC ? p.qg : p.q) + row0 * D, gs, clen);
    rW.load(static_cast<const T*>(p.w) + row0 * D, gs, clen);
    rA.load(static_cast<const T*>(p.aqk) + row0 * C, (int64_t)H * C, clen);
    rdO.load(static_cast<const T*>(p.dO) + row0 * D + v0, gs, clen);
    if (PC) {
      if (tid < D) rg = p.gcum[((int64_t)(cstart + clen - 1) * H + h) * D + tid];
    } else if (tid < C) {
      rg = p.gcum[(int64_t)(cstart + min(tid, clen - 1)) * H + h];
    }
  };
  if (count > 0) prefetch(count - 1);
  const float scale = p.scale;
  for (int jc = count - 1; jc >= 0; --jc) {
    const int cid = first + jc;
    const int cstart = dstart + jc * C;
    const int clen = min(C, dlen - jc * C);
    const int64_t row0 = (int64_t)cstart * H + h;
    // publish this chunk's operands and dS_C; checkpoint dS_C
    rKW.store(sKW, L::LD);
    rQ.store(sQ, L::LD);
    rW.store(sW, L::LD);
    rA.store(sAqk, L::LDC);
    rdO.store(sdO, L::LDV);
    if (PC) {
      if (tid < D) sGC[tid] = rg;
    } else if (tid < C) {
      sGam[tid] = rg;
    }
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int ti = wave * NS + i;
      const int rt = ti / NCT, ct = ti % NCT;
      store_acc_lds(sdS, L::LDV, dS[i], 16 * rt, 16 * ct, lane);
      T* hb = static_cast<T*>(p.dh) + ((int64_t)cid * H + h) * D * D;
      store_acc_tile(hb + tile_offset(D, rt, v0 / 16 + ct), dS[i], lane);
    }
    __syncthreads();
    if (jc > 0) prefetch(jc - 1);
    const float gC = PC ? 0.f : sGam[C - 1];
    // s e^G dO (elementwise, for Q^T diag(s e^G) dO)
    if (!PC) {
      for (int i = tid; i < C * BV; i += kSW) {
        const int r = i / BV, c = i - r * BV;
        sdOg[r * L::LDV + c] = to_e<E>(scale * exp_fast(sGam[r]) * from_e<E>(sdO[r * L::LDV + c]));
      }
    }
    // dU = Aqk^T dO + diag(e^{G_C - G}) KW dS     (tile ti: row block ti % 4, column tile ti / 4)
    T* du_out = static_cast<T*>(p.du) + row0 * D + v0;
#pragma unroll
    for (int ti = wave; ti < NRT; ti += NW) {
      const int r0 = 16 * (ti & 3), ct = ti >> 2;
      float egc[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) egc[e] = PC ? 1.f : exp_fast(gC - sGam[r0 + acc_row(lane, e)]);
      f32x4 a1 = zero4(), a2 = zero4();
      mma_tile_range<E, COL, ROW>(a1, sAqk, L::LDC, r0, sdO, L::LDV, 16 * ct, kfloor<E>(r0), C, lane);
      mma_tile<E, ROW, ROW>(a2, sKW, L::LD, r0, sdS, L::LDV, 16 * ct, D, lane);
      f32x4 du;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        du[e] = a1[e] + egc[e] * a2[e];
        sdUn[(r0 + acc_row(lane, e)) * L::LDV + 16 * ct + acc_col(lane)] = to_e<E>(-du[e]);
      }
      store_acc_global<T>(du_out, gs, du, r0, 16 * ct, clen, lane);
    }
    __syncthreads();
    // dS <- e^{G_C} dS + Q^T (s e^G dO) - W^T dU   (per-channel: diag(e^{G_C}) dS + qg^T dO - W^T dU)
    const float decay = exp_fast(gC);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int ti = wave * NS + i;
      const int rt = ti / NCT, ct = ti % NCT;
      if (PC) {
#pragma unroll
        for (int j = 0; j < 4; ++j) dS[i][j] *= exp_fast(sGC[16 * rt + acc_row(lane, j)]);
      } else {
        dS[i] = dS[i] * decay;
      }
      mma_tile<E, COL, ROW>(dS[i], sQ, L::LD, 16 * rt, PC ? sdO : sdOg, L::LDV, 16 * ct, C, lane);
      mma_tile<E, COL, ROW>(dS[i], sW, L::LD, 16 * rt, sdUn, L::LDV, 16 * ct, C, lane);
    }
    __syncthreads();
  }
  if (p.dh0) {
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int ti = wave * NS + i;
      const int rt = ti / NCT, ct = ti % NCT;
      store_acc_global<float>(p.dh0 + ((int64_t)n * H + h) * D * D + v0, D, dS[i], 16 * rt, 16 * ct, D, lane);
    }
  }
}
// ---------------------------------------------------------------------------
// fused per-chunk backward
//
// With dBv = T^T dU, the WY backward needs neither dW nor dT: since
// dW = -dU S0^T and (Bv - Bw S0) = T^-1 U,
//   dBw  = T^T dW = -dBv S0^T
//   dT   = dW Bw^T + dU Bv^T = dU (T^-1 U)^T   so   dAkk = -T^T dT T^T = -dBv U^T.
// Phases (8 waves, wave (rb, ch): row block rb, column half ch):
//   1  dBv = T^T dU -> dv (BF16 with a per-head gate: the reverse pass has
//      formed dBv and hands it over instead of dU);  dQg = dO S0^T;
//      dAqk = dO U^T -> P2
//   2  dBv to LDS over dU
//   3  dBw = -dBv S0^T;  dAkk = -dBv U^T -> P1r = dAkk E, P1 = beta_t P1r
//   4  dS_C replaces S0; sum(S0 * dS_C)
//   5  dKg = U dS_C^T
//   6  pairwise terms with K, Q, KW; outputs
// ---------------------------------------------------------------------------
template <typename T, int D>
struct FusedBwdLayout {
  static constexpr int LD = D + Pad<T>::v;
  static constexpr int LDC = C + Pad<T>::v;
  static constexpr int RT = C * LD * (int)sizeof(T);    // one [64][LD] tile
  static constexpr int CT = C * LDC * (int)sizeof(T);   // one [64][LDC] tile
  static constexpr int off_U = 0;                       // U, then K
  static constexpr int off_dO = off_U + RT;             // dO, then Q
  static constexpr int off_dU = off_dO + RT;            // dU, then dBv
  static constexpr int off_V = off_dU + RT;             // V, then KW
  static constexpr int off_H = off_V + RT;              // S0, then dS_C [D][LD]
  static constexpr int off_T = off_H + D * LD * (int)sizeof(T);  // T, then P1r = dAkk E
  static constexpr int off_P2 = off_T + CT;             // s dAqk E
  static constexpr int off_P1 = off_P2 + CT;            // beta_t dAkk E
  static constexpr int off_gam = off_P1 + CT;
  static constexpr int off_beta = off_gam + C * 4;
  static constexpr int off_p2d = off_beta + C * 4;      // [64] s dAqk[t,t], FP32
  static constexpr int off_red = off_p2d + C * 4;       // [kFW] floats
  static constexpr int bytes = off_red + kFW * 4;
};

template <typename T, int D, typename OT, typename OK, bool ALIAS>
__global__ __launch_bounds__(kFW) void chunk_fused_bwd_kernel(BwdParams p) {
  using L = FusedBwdLayout<T, D>;
  using E = T;
  // BF16 with a per-head gate: the reverse pass hands over dBv = T^T dU in du
  constexpr bool kDbv = implicit_w<T>();
  constexpr int HCT = D / 32;  // column tiles per wave of a [64 x D] output
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int H = p.H;
  const ChunkHead wg = chunk_head<true>(H);
  if (wg.cid >= p.geom.num_chunks) return;
  const ChunkInfo ci = chunk_info(p.geom, wg.cid);
  if (ci.len <= 0) return;
  const int cid = wg.cid, hh = wg.h;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int rb = wave & 3, ch = wave >> 2;
  const int r0 = 16 * rb;
  const int len = ci.len;
  const int64_t gs = (int64_t)H * D;
  const int64_t row0 = (int64_t)ci.start * H + hh;

  E* sU = reinterpret_cast<E*>(smem + L::off_U);
  E* sK = sU;
  E* sdO = reinterpret_cast<E*>(smem + L::off_dO);
  E* sQ = sdO;
  E* sdU = reinterpret_cast<E*>(smem + L::off_dU);
  E* sdBv = sdU;
  E* sV = reinterpret_cast<E*>(smem + L::off_V);
  E* sKW = sV;
  E* sH = reinterpret_cast<E*>(smem + L::off_H);
  E* sT = reinterpret_cast<E*>(smem + L::off_T);
  E* sP1r = sT;
  E* sP2 = reinterpret_cast<E*>(smem + L::off_P2);
  E* sP1 = reinterpret_cast<E*>(smem + L::off_P1);
  float* sGam = reinterpret_cast<float*>(smem + L::off_gam);
  float* sBeta = reinterpret_cast<float*>(smem + L::off_beta);
  float* sP2d = reinterpret_cast<float*>(smem + L::off_p2d);
  float* sRed = reinterpret_cast<float*>(smem + L::off_red);

  const T* hsrc = static_cast<const T*>(p.h) + ((int64_t)cid * H + hh) * D * D;
  const T* dhsrc = static_cast<const T*>(p.dh) + ((int64_t)cid * H + hh) * D * D;
  const float scale = p.scale;

  if (tid < C) {
    const int64_t idx = (int64_t)(ci.start + min(tid, len - 1)) * H + hh;
    sGam[tid] = p.gcum[idx];
    sBeta[tid] = tid < len ? p.beta[(int64_t)(ci.start + tid) * H + hh] : 0.f;
  }
  // every global load of the phase is issued before the first LDS store, so
  // the tiles share one memory round trip
  {
    RegTile<kFW, C, D, T> rU, rdO, rdU, rV;
    RegTile<kFW, C, C, T> rT;
    TiledTile<kFW, D, T> rH;
    rU.load(static_cast<const T*>(p.u) + row0 * D, gs, len);
    rdO.load(static_cast<const T*>(p.dO) + row0 * D, gs, len);
    rdU.load(static_cast<const T*>(p.du) + row0 * D, gs, len);
    rV.load(static_cast<const T*>(p.v) + row0 * D, gs, len);
    if (!kDbv) rT.load(static_cast<const T*>(p.akk) + row0 * C, (int64_t)H * C, len);
    rH.load(hsrc);
    rU.store(sU, L::LD);
    rdO.store(sdO, L::LD);
    rdU.store(sdU, L::LD);
    rV.store(sV, L::LD);
    if (!kDbv) rT.store(sT, L::LDC);
    rH.store(sH, L::LD);
  }
  __syncthreads();
  const float gC = sGam[C - 1];
  // T, P1 and P2 hold exact zeros above the diagonal (and K, Q, KW, U zero
  // rows past the chunk's end), so products over the chunk's tokens run over
  // all 64: the extra k-steps add zeros and the loops unroll.

  f32x4 dq[HCT], dkb[HCT], dkws[HCT], dBv[HCT];
  float db[4] = {0.f, 0.f, 0.f, 0.f};
  // dv in the activation dtype leaves through V's region, free after phase 1
  // when the write key is the read key (16-byte stores)
  constexpr bool vStage = sizeof(OT) == sizeof(T) && ALIAS;
  OT* dvo = static_cast<OT*>(p.dv) + row0 * D;
  // ---- phase 1: dBv = T^T dU (-> dv), dQg = dO S0^T, dAqk = dO U^T ------------
#pragma unroll
  for (int j = 0; j < HCT; ++j) {
    const int ct = ch * HCT + j;
    const int c = 16 * ct + acc_col(lane);
    f32x4 acv = zero4();
    if constexpr (kDbv) {
#pragma unroll
      for (int e = 0; e < 4; ++e) acv[e] = from_e<E>(sdU[(r0 + acc_row(lane, e)) * L::LD + c]);
    } else {
      mma_tile<E, COL, ROW>(acv, sT, L::LDC, r0, sdU, L::LD, 16 * ct, C, lane);
    }
    dBv[j] = acv;
#pragma unroll
    for (int e = 0; e < 4; ++e) db[e] += acv[e] * from_e<E>(sV[(r0 + acc_row(lane, e)) * L::LD + c]);
    if constexpr (!vStage) {
      f32x4 dv;
#pragma unroll
      for (int e = 0; e < 4; ++e) dv[e] = sBeta[r0 + acc_row(lane, e)] * acv[e];
      store_acc_global<OT>(dvo, gs, dv, r0, 16 * ct, len, lane);  // final
    }
    f32x4 acc = zero4();
    mma_tile<E, ROW, COL>(acc, sdO, L::LD, r0, sH, L::LD, 16 * ct, D, lane);
#pragma unroll
    for (int e = 0; e < 4; ++e) dq[j][e] = scale * exp_fast(sGam[r0 + acc_row(lane, e)]) * acc[e];
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int ct = 2 * ch + j;
    f32x4 acc = zero4();
    if (ct <= rb) mma_tile<E, ROW, COL>(acc, sdO, L::LD, r0, sU, L::LD, 16 * ct, D, lane);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = r0 + acc_row(lane, e), s = 16 * ct + acc_col(lane);
      // the diagonal (decay e^0) is kept apart, in FP32: its two halves of
      // the gate gradient (q dq and kw dkw) cancel exactly and stay out of it
      const float val = (s < t && t < len) ? scale * exp_fast(sGam[t] - sGam[s]) * acc[e] : 0.f;
      sP2[t * L::LDC + s] = to_e<E>(val);
      if (s == t) sP2d[t] = t < len ? scale * acc[e] : 0.f;
    }
  }
  __syncthreads();
  // ---- phase 2: dBv over dU; Q, KW, dS_C and K start their way in ---------
  RegTile<kFW, C, D, T> rQ, rKW, rK;
  TiledTile<kFW, D, T> rdH;
  rQ.load(static_cast<const T*>(p.q) + row0 * D, gs, len);
  if (!ALIAS) rKW.load(static_cast<const T*>(p.kw) + row0 * D, gs, len);
  rdH.load(dhsrc);
  rK.load(static_cast<const T*>(p.k) + row0 * D, gs, len);  // waits in registers until U's region frees
#pragma unroll
  for (int j = 0; j < HCT; ++j) {
    if constexpr (!kDbv) store_acc_lds(sdBv, L::LD, dBv[j], r0, 16 * (ch * HCT + j), lane);
    if constexpr (vStage) {
      f32x4 dv;
#pragma unroll
      for (int e = 0; e < 4; ++e) dv[e] = sBeta[r0 + acc_row(lane, e)] * dBv[j][e];
      store_acc_lds(sV, L::LD, dv, r0, 16 * (ch * HCT + j), lane);
    }
  }
  __syncthreads();
  if constexpr (vStage) store_tile<kFW, C, D>(dvo, gs, sV, L::LD, len);  // final
  // ---- phase 3: dBw = -dBv S0^T, dAkk = -dBv U^T --------------------------------
#pragma unroll
  for (int j = 0; j < HCT; ++j) {
    const int ct = ch * HCT + j;
    f32x4 acc = zero4();
    mma_tile<E, ROW, COL>(acc, sdBv, L::LD, r0, sH, L::LD, 16 * ct, D, lane);
#pragma unroll
    for (int e = 0; e < 4; ++e) dkb[j][e] = -exp_fast(sGam[r0 + acc_row(lane, e)]) * acc[e];  // e^G dBw
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int ct = 2 * ch + j;
    f32x4 acc = zero4();
    if (ct <= rb) mma_tile<E, ROW, COL>(acc, sdBv, L::LD, r0, sU, L::LD, 16 * ct, D, lane);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = r0 + acc_row(lane, e), s = 16 * ct + acc_col(lane);
      const float raw = (s < t && t < len) ? -acc[e] * exp_fast(sGam[t] - sGam[s]) : 0.f;
      sP1r[t * L::LDC + s] = to_e<E>(raw);
      sP1[t * L::LDC + s] = to_e<E>(sBeta[t] * raw);
    }
  }
  // Q and KW regions (dO, V) have been free since phase 1
  rQ.store(sQ, L::LD);
  if (!ALIAS) rKW.store(sKW, L::LD);
  __syncthreads();
  // ---- phase 4: dS_C replaces S0; sum(S0 * dS_C) ------------------------------
  float hd = 0.f;
  {
    constexpr int V = Vec16<T>::N;
#pragma unroll
    for (int i = 0; i < TiledTile<kFW, D, T>::ITER; ++i) {
      int r, c;
      rdH.pos(i, r, c);
      float x[V], hv[V];
      Vec16<T>::unpack(rdH.r[i], x);
      lds_vec<V>(sH + r * L::LD + c, hv);
#pragma unroll
      for (int j = 0; j < V; ++j) hd += hv[j] * x[j];
      *reinterpret_cast<uint4*>(sH + r * L::LD + c) = rdH.r[i];  // this thread's own slots
    }
  }
  __syncthreads();
  // ---- phase 5: dKg = U dS_C^T (write-key gradient of the state path) ---------
#pragma unroll
  for (int j = 0; j < HCT; ++j) {
    const int ct = ch * HCT + j;
    f32x4 acc = zero4();
    mma_tile<E, ROW, COL>(acc, sU, L::LD, r0, sH, L::LD, 16 * ct, D, lane);
#pragma unroll
    for (int e = 0; e < 4; ++e) dkws[j][e] = exp_fast(gC - sGam[r0 + acc_row(lane, e)]) * acc[e];
  }
  __syncthreads();
  rK.store(sK, L::LD);
  __syncthreads();
  const E* sKWr = ALIAS ? sK : sKW;
  // ---- phase 6: pairwise terms ------------------------------------------------
  float gsum[4] = {0.f, 0.f, 0.f, 0.f};
  float kgd = 0.f;
  OT* dqo = static_cast<OT*>(p.dq) + row0 * D;
  OK* dko = static_cast<OK*>(p.dk) + row0 * D;
  // outputs in the activation dtype with the write-key gradient folded into
  // dk leave through LDS (16-byte stores)
  constexpr bool kStage = sizeof(OT) == sizeof(T) && sizeof(OK) == sizeof(T) && ALIAS;
#pragma unroll
  for (int j = 0; j < HCT; ++j) {
    const int ct = ch * HCT + j;
    const int c = 16 * ct + acc_col(lane);
    f32x4 ak = zero4(), aq = zero4(), aw = zero4();
    mma_tile<E, ROW, ROW>(ak, sP1r, L::LDC, r0, sKWr, L::LD, 16 * ct, C, lane);    // sum_x P1r kw
    mma_tile<E, ROW, ROW>(aq, sP2, L::LDC, r0, sKWr, L::LD, 16 * ct, C, lane);     // sum_x P2 kw
    mma_tile<E, COL, ROW>(aw, sP1, L::LDC, r0, sK, L::LD, 16 * ct, C, lane);       // sum_t P1 k
    mma_tile<E, COL, ROW>(aw, sP2, L::LDC, r0, sQ, L::LD, 16 * ct, C, lane);       // sum_t P2 q
    f32x4 dk, dkw;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = r0 + acc_row(lane, e);
      const float kv = from_e<E>(sK[r * L::LD + c]);
      const float qv = from_e<E>(sQ[r * L::LD + c]);
      const float wv = from_e<E>(sKWr[r * L::LD + c]);
      const float tk = dkb[j][e] + ak[e];  // e^G dBw + sum_x P1r kw
      const float pd = sP2d[r];
      dk[e] = sBeta[r] * tk;
      db[e] += kv * tk;
      dq[j][e] += aq[e];
      // Every term of the gate gradient carries a decay factor: the Aqk
      // diagonal and the last row's state-path term (e^{G_C - G_C} = 1)
      // appear once with each sign and are left out of both.
      const float dkwg = (r == len - 1 ? 0.f : dkws[j][e]) + aw[e];
      if (r != len - 1) kgd += wv * dkws[j][e];
      gsum[e] += qv * dq[j][e] + kv * dk[e] - wv * dkwg;
      dq[j][e] += pd * wv;
      dkw[e] = dkws[j][e] + aw[e] + pd * qv;
    }
    if constexpr (kStage) {  // S0's and dBv's regions are free: stage for 16-byte stores
      store_acc_lds(sH, L::LD, dq[j], r0, 16 * ct, lane);
      store_acc_lds(sdBv, L::LD, dk + dkw, r0, 16 * ct, lane);
    } else {
      store_acc_global<OT>(dqo, gs, dq[j], r0, 16 * ct, len, lane);
      if (ALIAS) {
        store_acc_global<OK>(dko, gs, dk + dkw, r0, 16 * ct, len, lane);
      } else {
        store_acc_global<OK>(dko, gs, dk, r0, 16 * ct, len, lane);
        store_acc_global<OK>(static_cast<OK*>(p.dkw) + row0 * D, gs, dkw, r0, 16 * ct, len, lane);
      }
    }
  }
  // row sums over the two column halves; wave sums of the last-row terms
  float* sRowG = sRed;              // [2][64]
  float* sRowB = sRed + 2 * C;      // [2][64]
  float* sWave = sRed + 4 * C;      // [2][8]
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float g = group16_sum(gsum[e]);
    const float b = group16_sum(db[e]);
    if ((lane & 15) == 0) {
      sRowG[ch * C + r0 + acc_row(lane, e)] = g;
      sRowB[ch * C + r0 + acc_row(lane, e)] = b;
    }
  }
  hd = wave_sum(hd);
  kgd = wave_sum(kgd);
  if (lane == 0) {
    sWave[wave] = hd;
    sWave[kFW / 64 + wave] = kgd;
  }
  __syncthreads();
  if constexpr (kStage) {
    store_tile<kFW, C, D>(dqo, gs, reinterpret_cast<const OT*>(sH), L::LD, len);
    store_tile<kFW, C, D>(dko, gs, reinterpret_cast<const OT*>(sdBv), L::LD, len);
  }
  if (tid < len) {
    const int64_t idx = (int64_t)(ci.start + tid) * H + hh;
    float g = sRowG[tid] + sRowG[C + tid];
    if (tid == len - 1) {
      float hd_sum = 0.f, kg_sum = 0.f;
#pragma unroll
      for (int w = 0; w < kFW / 64; ++w) {
        hd_sum += sWave[w];
        kg_sum += sWave[kFW / 64 + w];
      }
      g += exp_fast(gC) * hd_sum + kg_sum;
    }
    p.dgcum[idx] = g;
    p.dbeta[idx] = sRowB[tid] + sRowB[C + tid];
  }
}

// ---------------------------------------------------------------------------
// fused per-chunk backward, BF16 with a per-head gate and kw = k: the
// four-wave form, two workgroups per compute unit.
//
// The same products and gate-gradient terms as chunk_fused_bwd_kernel with
// the work laid out so that a workgroup needs ~64 KB of LDS instead of
// ~132 KB: while one workgroup waits for its tiles, the other computes.
//   * Wave w owns output columns [D w / 4, D (w + 1) / 4) of every row, so
//     the contractions over the value index (dO S0^T, dBv S0^T, U dS_C^T)
//     take S0 and dS_C rows of its own columns only: they come from the
//     tile-major checkpoints straight into registers as MFMA B operands
//     (never through LDS), and sum(S0 * dS_C) is formed there too.
//   * dv = beta dBv and dbeta = sum_c dBv U / beta are formed on the loaded
//     registers (V is not read: see below) and dv never touches LDS.
//   * Two [64 x D] LDS regions hold U and dO, then U and dBv, then K and Q;
//     the pair matrices (s dAqk E, dAkk E, beta dAkk E) have their own.
// Passes: (1) dQg = dO S0^T, dAqk = dO U^T -> P2;  (2) dBw = -dBv S0^T,
// dAkk = -dBv U^T -> P1r, P1, dKg = U dS_C^T;  (3) the pair terms with K and
// Q, row block by row block, and the outputs.
// ---------------------------------------------------------------------------
constexpr int kW4 = 256;

template <int D>
struct FusedW4Layout {
  static constexpr int LD = D + Pad<bf16_t>::v;
  static constexpr int LDC = C + Pad<bf16_t>::v;
  static constexpr int RT = C * LD * 2;
  static constexpr int CT = C * LDC * 2;
  static constexpr int off_R0 = 0;               // U, then K
  static constexpr int off_R1 = off_R0 + RT;     // dO, then dBv, then Q
  static constexpr int off_P2 = off_R1 + RT;     // s dAqk E (strictly lower)
  static constexpr int off_P1r = off_P2 + CT;    // dAkk E (strictly lower)
  static constexpr int off_P1 = off_P1r + CT;    // beta_t dAkk E
  static constexpr int off_gam = off_P1 + CT;    // [64] G
  static constexpr int off_beta = off_gam + C * 4;
  static constexpr int off_p2d = off_beta + C * 4;   // [64] s dAqk[t,t], FP32, then 64 dummy slots
  static constexpr int off_db1 = off_p2d + 2 * C * 4;  // [64] sum_c dBv U
  static constexpr int off_dbv = off_db1 + C * 4;    // [64] sum_c dBv V (rows with |beta| < 1e-20 only)
  static constexpr int off_rowg = off_dbv + C * 4;   // [4][64] per-wave row sums of the gate gradient
  static constexpr int off_rowb = off_rowg + 4 * C * 4;  // [4][64] per-wave row sums of dbeta
  static constexpr int off_wave = off_rowb + 4 * C * 4;  // [2][4] sum(S0 dS_C), sum(kw dKg) per wave
  // dq's last PARK tiles (row blocks 2-3) between passes 1 and 3 (FP32, one
  // 16-byte slot per lane and tile): at D = 128 the accumulators of passes 2
  // and 3 fit the 256 registers of two workgroups per compute unit only
  // without them
  static constexpr int PARK = D == 128 ? 3 : 0;  // tiles per wave
  static constexpr int off_park = off_wave + 8 * 4;
  static constexpr int bytes = off_park + 4 * PARK * 64 * 16;
  static_assert(2 * bytes <= 160 * 1024, "two workgroups per compute unit");
};


// The body for one chunk; `len` is a literal C for whole chunks (every chunk
// of a document but its last), so every row test folds away and no branch
// splits the code.
template <int D>
__device__ __forceinline__ void fused_bwd_w4(const BwdParams& p, const ChunkInfo ci, const int len, char* smem) {
  using L = FusedW4Layout<D>;
  using E = bf16_t;
  using M = Mma<bf16_t>;
  constexpr int NJ = D / 64;  // column tiles per wave
  constexpr int KV = D / 32;  // k steps over the value index
  const int H = p.H;
  const ChunkHead wg = chunk_head<true>(H);
  const int cid = wg.cid, hh = wg.h;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int q = lane >> 4, il = lane & 15;
  const int64_t gs = (int64_t)H * D;
  const int64_t row0 = (int64_t)ci.start * H + hh;
  const float scale = p.scale;

  E* sR0 = reinterpret_cast<E*>(smem + L::off_R0);
  E* sR1 = reinterpret_cast<E*>(smem + L::off_R1);
  E* sP2 = reinterpret_cast<E*>(smem + L::off_P2);
  E* sP1r = reinterpret_cast<E*>(smem + L::off_P1r);
  E* sP1 = reinterpret_cast<E*>(smem + L::off_P1);
  float* sGam = reinterpret_cast<float*>(smem + L::off_gam);
  float* sBeta = reinterpret_cast<float*>(smem + L::off_beta);
  float* sP2d = reinterpret_cast<float*>(smem + L::off_p2d);
  float* sDb1 = reinterpret_cast<float*>(smem + L::off_db1);
  float* sDbV = reinterpret_cast<float*>(smem + L::off_dbv);
  float* sRowG = reinterpret_cast<float*>(smem + L::off_rowg);
  float* sRowB = reinterpret_cast<float*>(smem + L::off_rowb);
  float* sWave = reinterpret_cast<float*>(smem + L::off_wave);
  f32x4* sPark = reinterpret_cast<f32x4*>(smem + L::off_park) + wave * L::PARK * 64 + lane;

  // the first passes' loads go out before the first LDS store, in the order
  // the passes need them; the gate and beta first, so that their LDS stores
  // wait for those loads only
  const int64_t gidx = (int64_t)(ci.start + min(tid & (C - 1), len - 1)) * H + hh;
  const float gval = p.gcum[gidx];  // rows past the end repeat the last gate
  const float bval = p.beta[gidx];
  RegTile<kW4, C, D, E> rU, rdO, rdBv, rK, rQ;
  s16x8_t S0f[NJ][KV], dSf[NJ][KV];  // B operands: rows of this wave's columns, k over the value index
  const E* hsrc = static_cast<const E*>(p.h) + ((int64_t)cid * H + hh) * D * D;
  const E* dhsrc = static_cast<const E*>(p.dh) + ((int64_t)cid * H + hh) * D * D;
  rU.load(static_cast<const E*>(p.u) + row0 * D, gs, len);
  rdO.load(static_cast<const E*>(p.dO) + row0 * D, gs, len);
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int kk = 0; kk < KV; ++kk) {
      // tile-major [D x D]: B[k = v][n = c] = S0[c][v], c = 16 ct + il, v = 32 kk + 8 q .. + 7
      const int ct = NJ * wave + j;
      const int64_t off = tile_offset(D, ct, 2 * kk + (q >> 1)) + il * 16 + 8 * (q & 1);
      S0f[j][kk] = *reinterpret_cast<const s16x8_t*>(hsrc + off);
    }
  rdBv.load(static_cast<const E*>(p.dv_handoff ? p.dv : p.du) + row0 * D, gs, len);  // dBv, or dv (final)
  // every thread writes (the C rows' values, repeated): no branch
  sGam[tid & (C - 1)] = gval;
  sBeta[tid & (C - 1)] = (tid & (C - 1)) < len ? bval : 0.f;
  rU.store(sR0, L::LD);
  rdO.store(sR1, L::LD);
  __syncthreads();

  // dv = beta dBv (final) and sum_c dBv U on the registers: the 16 pieces of
  // a row sit in 16 consecutive lanes.
  // dbeta: every beta-dependent quantity of the chunk (Bv, Bw and the rows of
  // Akk) is row t scaled by beta_t, so (I + Akk) U = Bv - Bw S0 reads
  // U_t = beta_t r_t with r_t independent of beta_t, and the adjoint of the
  // right-hand side being dBv = T^T dU, dL/dbeta_t = sum_c dBv[t,c] r_t[c]
  // = sum_c dBv[t,c] U[t,c] / beta_t.  (The three-term form -- dBv V, the Bw
  // part and the Akk part -- is the same sum; it needs V, which this kernel
  // then does not read.)  A row with |beta_t| < 1e-20 (where U_t no longer
  // carries r_t) takes the three-term form, with V loaded for that row only.
  {
    constexpr int V = Vec16<E>::N;
    constexpr int PER_ROW = D / V;
    static_assert(PER_ROW == 16 || PER_ROW == 8, "row pieces fill 16 or 8 lanes");
    E* dvo = static_cast<E*>(p.dv) + row0 * D;
#pragma unroll
    for (int i = 0; i < RegTile<kW4, C, D, E>::ITER; ++i) {
      const int idx = tid + i * kW4;
      const int r = idx / PER_ROW, c = (idx % PER_ROW) * V;
      float b[V], u[V];
      Vec16<E>::unpack(rdBv.r[i], b);
      Vec16<E>::unpack(rU.r[i], u);
      const float br = sBeta[r];
      const bool tiny_row = !(fabsf(br) >= 1e-20f);
      if (p.dv_handoff) {  // b holds dv (already written): dBv = dv / beta, or dBv itself for a tiny beta
        if (tiny_row && r < len) {
          Vec16<E>::load(static_cast<const E*>(p.du) + row0 * D + r * gs + c, b);
        } else {
          const float rb = 1.f / br;
#pragma unroll
          for (int e = 0; e < V; ++e) b[e] = tiny_row ? 0.f : b[e] * rb;
        }
        rdBv.r[i] = pack_vec16<E>(b);  // the dBv operand of passes 2-3
      }
      float part = 0.f, pv = 0.f;
#pragma unroll
      for (int e = 0; e < V; ++e) part += b[e] * u[e];
      if (r < len && !(fabsf(br) >= 1e-20f)) {  // rare: the value part from V itself
        float v[V];
        Vec16<E>::load(static_cast<const E*>(p.v) + row0 * D + r * gs + c, v);
#pragma unroll
        for (int e = 0; e < V; ++e) pv += b[e] * v[e];
      }
      part = lane_group_sum<PER_ROW>(part);
      // pv is zero on every lane unless a row of this wave's pieces has a
      // vanishing beta (one wave-uniform test)
      if (__builtin_expect(__ballot(r < len && !(fabsf(br) >= 1e-20f)) != 0, 0)) pv = lane_group_sum<PER_ROW>(pv);
      sDb1[r] = part;  // the row's lanes all hold the sums: unconditional, no branch
      sDbV[r] = pv;
      if (!p.dv_handoff) {
#pragma unroll
        for (int e = 0; e < V; ++e) b[e] *= br;
        if (r < len) store_vec<V>(dvo + r * gs + c, b);
      }
    }
  }

  // ---- pass 1: dQg = dO S0^T (-> s e^G dQg), dAqk = dO U^T -> P2, P2d ---------
  f32x4 dq[4][NJ];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) dq[rb][j] = zero4();
#pragma unroll
    for (int kk = 0; kk < KV; ++kk) {
      const s16x8_t a = M::frag_a<ROW>(sR1 + 16 * rb * L::LD, L::LD, 32 * kk, lane);
#pragma unroll
      for (int j = 0; j < NJ; ++j) M::mfma(dq[rb][j], a, S0f[j][kk]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float f = scale * exp_fast(sGam[16 * rb + 4 * q + e]);
#pragma unroll
      for (int j = 0; j < NJ; ++j) dq[rb][j][e] *= f;
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {  // parked until pass 3 (this lane's own slots)
      const int slot = rb * NJ + j - (4 * NJ - L::PARK);
      if (slot >= 0) sPark[slot * 64] = dq[rb][j];
    }
  }
  // pair tiles of this wave: lower tiles w, w + 4, w + 8; waves 2 and 3 also
  // write the six upper tiles' zeros (of P2 here, of P1r and P1 in pass 2)
  auto upper_zero = [&](E* P) {
    if (wave >= 2) {
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        const int k = 3 * (wave - 2) + u;  // 0..5: (0,1) (0,2) (0,3) (1,2) (1,3) (2,3)
        const int tb = k < 3 ? 0 : k < 5 ? 1 : 2;
        const int sb = k < 3 ? k + 1 : k < 5 ? k - 1 : 3;
#pragma unroll
        for (int e = 0; e < 4; ++e) P[(16 * tb + 4 * q + e) * L::LDC + 16 * sb + il] = to_e<E>(0.f);
      }
    }
  };
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    const int i = wave + 4 * u;
    if (i < 10) {
      int tb, sb;
      lower_block(i, tb, sb);
      f32x4 acc = zero4();
#pragma unroll
      for (int kk = 0; kk < KV; ++kk)
        M::mfma(acc, M::frag_a<ROW>(sR1 + 16 * tb * L::LD, L::LD, 32 * kk, lane),
                M::frag_b<COL>(sR0 + 16 * sb * L::LD, L::LD, 32 * kk, lane));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = 16 * tb + 4 * q + e, s = 16 * sb + il;
        // the diagonal (decay e^0) is kept apart, in FP32: its two halves of
        // the gate gradient (q dq and kw dkw) cancel exactly and stay out of it
        const float val = (s < t && t < len) ? scale * exp_fast(sGam[t] - sGam[s]) * acc[e] : 0.f;
        sP2[t * L::LDC + s] = to_e<E>(val);
        // the diagonal lane writes P2d[t], the others their own dummy slot
        sP2d[s == t ? t : C + lane] = t < len ? scale * acc[e] : 0.f;
      }
    }
  }
  upper_zero(sP2);
  __syncthreads();  // every wave is done with dO
  rdBv.store(sR1, L::LD);
  __syncthreads();

  // ---- pass 2: dBw = -dBv S0^T (-> -e^G dBv S0^T), dAkk = -dBv U^T -> P1r, P1,
  //      dKg = U dS_C^T (-> e^{G_C - G} dKg), sum(S0 dS_C) ----------------------
  f32x4 tk[4][NJ], dkws[4][NJ];
  const float gC = sGam[C - 1];
  // dS_C's rows of this wave's columns (loaded here: S0's and dS_C's operands
  // are not in registers together through pass 1)
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int kk = 0; kk < KV; ++kk) {
      const int ct = NJ * wave + j;
      const int64_t off = tile_offset(D, ct, 2 * kk + (q >> 1)) + il * 16 + 8 * (q & 1);
      dSf[j][kk] = *reinterpret_cast<const s16x8_t*>(dhsrc + off);
    }
  // tk from S0 first; sum(S0 dS_C) is S0's last use, before dS_C's products
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) tk[rb][j] = zero4();
#pragma unroll
    for (int kk = 0; kk < KV; ++kk) {
      const s16x8_t a = M::frag_a<ROW>(sR1 + 16 * rb * L::LD, L::LD, 32 * kk, lane);
#pragma unroll
      for (int j = 0; j < NJ; ++j) M::mfma(tk[rb][j], a, S0f[j][kk]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float fb = -exp_fast(sGam[16 * rb + 4 * q + e]);
#pragma unroll
      for (int j = 0; j < NJ; ++j) tk[rb][j][e] *= fb;  // e^G dBw
    }
  }
  float hd = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int kk = 0; kk < KV; ++kk) {
      const uint4 a = __builtin_bit_cast(uint4, S0f[j][kk]), b = __builtin_bit_cast(uint4, dSf[j][kk]);
      float x[8], y[8];
      Vec16<E>::unpack(a, x);
      Vec16<E>::unpack(b, y);
#pragma unroll
      for (int e = 0; e < 8; ++e) hd += x[e] * y[e];
    }
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) dkws[rb][j] = zero4();
#pragma unroll
    for (int kk = 0; kk < KV; ++kk) {
      const s16x8_t u = M::frag_a<ROW>(sR0 + 16 * rb * L::LD, L::LD, 32 * kk, lane);
#pragma unroll
      for (int j = 0; j < NJ; ++j) M::mfma(dkws[rb][j], u, dSf[j][kk]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float fs = exp_fast(gC - sGam[16 * rb + 4 * q + e]);
#pragma unroll
      for (int j = 0; j < NJ; ++j) dkws[rb][j][e] *= fs;
    }
  }
  // K and Q go out now (in registers until U's and dBv's regions free); the
  // fence keeps the scheduler from hoisting them into the loops above, where
  // their registers would push the pass past 256
  __builtin_amdgcn_sched_barrier(0);
  rK.load(static_cast<const E*>(p.k) + row0 * D, gs, len);
  rQ.load(static_cast<const E*>(p.q) + row0 * D, gs, len);
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    const int i = wave + 4 * u;
    if (i < 10) {
      int tb, sb;
      lower_block(i, tb, sb);
      f32x4 acc = zero4();
#pragma unroll
      for (int kk = 0; kk < KV; ++kk)
        M::mfma(acc, M::frag_a<ROW>(sR1 + 16 * tb * L::LD, L::LD, 32 * kk, lane),
                M::frag_b<COL>(sR0 + 16 * sb * L::LD, L::LD, 32 * kk, lane));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = 16 * tb + 4 * q + e, s = 16 * sb + il;
        const float raw = (s < t && t < len) ? -acc[e] * exp_fast(sGam[t] - sGam[s]) : 0.f;
        sP1r[t * L::LDC + s] = to_e<E>(raw);
        sP1[t * L::LDC + s] = to_e<E>(sBeta[t] * raw);
      }
    }
  }
  upper_zero(sP1r);
  upper_zero(sP1);
  hd = wave_sum(hd);
  __syncthreads();  // every wave is done with U and dBv; the pair matrices are complete
  rK.store(sR0, L::LD);
  rQ.store(sR1, L::LD);
  __syncthreads();

  // ---- pass 3: pair terms, row block by row block; outputs ----------------------
  //   (a) dq += P2 K -> dq out, its gate-gradient term q dq;
  //   (b) tk += P1r K (tk = e^G dBw + sum_x P1r kw; dk = beta tk) and
  //       dkw = dkws + P1^T K + P2^T Q -> dk + dkw out, the other terms
  E* dqo = static_cast<E*>(p.dq) + row0 * D;
  E* dko = static_cast<E*>(p.dk) + row0 * D;
  s16x8_t Kf[2][NJ];  // B operands K[x][c] over the chunk's tokens
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int j = 0; j < NJ; ++j) Kf[kt][j] = M::frag_b<ROW>(sR0 + 16 * (NJ * wave + j), L::LD, 32 * kt, lane);
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const int r0 = 16 * rb;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int slot = rb * NJ + j - (4 * NJ - L::PARK);
      if (slot >= 0) dq[rb][j] = sPark[slot * 64];
    }
    // P2 is zero above the diagonal: rows of block rb reach k < 16 rb + 16
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      if (32 * kt < r0 + 16) {
        const s16x8_t a2 = M::frag_a<ROW>(sP2 + r0 * L::LDC, L::LDC, 32 * kt, lane);
#pragma unroll
        for (int j = 0; j < NJ; ++j) M::mfma(dq[rb][j], a2, Kf[kt][j]);
      }
    }
    float gq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = 16 * (NJ * wave + j) + il;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = r0 + 4 * q + e;
        gq[e] += from_e<E>(sR1[r * L::LD + c]) * dq[rb][j][e];
        dq[rb][j][e] += sP2d[r] * from_e<E>(sR0[r * L::LD + c]);  // the diagonal, after the gate term
      }
      store_acc_global<E>(dqo, gs, dq[rb][j], r0, 16 * (NJ * wave + j), len, lane);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) sRowG[wave * C + r0 + 4 * q + e] = group16_sum(gq[e]);  // same value from 16 lanes
  }
  s16x8_t Qf[2][NJ];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int j = 0; j < NJ; ++j) Qf[kt][j] = M::frag_b<ROW>(sR1 + 16 * (NJ * wave + j), L::LD, 32 * kt, lane);
  float kgd = 0.f;
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const int r0 = 16 * rb;
    f32x4 aw[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) aw[j] = zero4();
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      if (32 * kt < r0 + 16) {
        const s16x8_t a1 = M::frag_a<ROW>(sP1r + r0 * L::LDC, L::LDC, 32 * kt, lane);
#pragma unroll
        for (int j = 0; j < NJ; ++j) M::mfma(tk[rb][j], a1, Kf[kt][j]);
      }
      // columns x of block rb take rows t > x: k >= 16 rb
      if (32 * kt + 32 > r0) {
        const s16x8_t b1 = M::frag_a<COL>(sP1 + r0, L::LDC, 32 * kt, lane);
        const s16x8_t b2 = M::frag_a<COL>(sP2 + r0, L::LDC, 32 * kt, lane);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          M::mfma(aw[j], b1, Kf[kt][j]);
          M::mfma(aw[j], b2, Qf[kt][j]);
        }
      }
    }
    float gsum[4] = {0.f, 0.f, 0.f, 0.f}, db[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = 16 * (NJ * wave + j) + il;
      f32x4 dk, dkw;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = r0 + 4 * q + e;
        const float kv = from_e<E>(sR0[r * L::LD + c]);
        const float qv = from_e<E>(sR1[r * L::LD + c]);
        const float t_ = tk[rb][j][e];
        dk[e] = sBeta[r] * t_;
        db[e] += kv * t_;
        // Every term of the gate gradient carries a decay factor: the Aqk
        // diagonal and the last row's state-path term (e^{G_C - G_C} = 1)
        // appear once with each sign and are left out of both.
        const float dkwg = (r == len - 1 ? 0.f : dkws[rb][j][e]) + aw[j][e];
        if (r != len - 1) kgd += kv * dkws[rb][j][e];
        gsum[e] += kv * dk[e] - kv * dkwg;
        dkw[e] = dkws[rb][j][e] + aw[j][e] + sP2d[r] * qv;
      }
      store_acc_global<E>(dko, gs, dk + dkw, r0, 16 * (NJ * wave + j), len, lane);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float g = group16_sum(gsum[e]);
      const float b = group16_sum(db[e]);
      // the 16 lanes of the row all read the q dq part (a) wrote, then all
      // write the same sum
      sRowG[wave * C + r0 + 4 * q + e] += g;
      sRowB[wave * C + r0 + 4 * q + e] = b;
    }
  }
  kgd = wave_sum(kgd);
  sWave[wave] = hd;  // every lane holds the wave sums
  sWave[4 + wave] = kgd;
  __syncthreads();
  if (tid < len) {
    const int64_t idx = (int64_t)(ci.start + tid) * H + hh;
    const float bt = sBeta[tid];
    float g = 0.f, b3 = sDbV[tid];  // the three-term form (|beta| < 1e-20)
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      g += sRowG[w * C + tid];
      b3 += sRowB[w * C + tid];
    }
    const float b = fabsf(bt) >= 1e-20f ? sDb1[tid] / bt : b3;
    if (tid == len - 1) {
      float hd_sum = 0.f, kg_sum = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        hd_sum += sWave[w];
        kg_sum += sWave[4 + w];
      }
      g += exp_fast(gC) * hd_sum + kg_sum;
    }
    p.dgcum[idx] = g;
    p.dbeta[idx] = b;
  }
}

template <int D>
__global__ __launch_bounds__(kW4, 2) void chunk_fused_bwd_w4_kernel(BwdParams p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const ChunkHead wg = chunk_head<true>(p.H);
  if (wg.cid >= p.geom.num_chunks) return;
  const ChunkInfo ci = chunk_info(p.geom, wg.cid);
  if (ci.len == C) fused_bwd_w4<D>(p, ci, C, smem);
  else if (ci.len > 0) fused_bwd_w4<D>(p, ci, ci.len, smem);
}

// ---------------------------------------------------------------------------
// fused per-chunk backward, per-channel gate (G [64][D] per chunk).
//
// The WY backward of the per-head kernel (dBv = T^T dU, dBw = -dBv S0^T,
// dAkk = -dBv U^T), with the decay inside every key contraction:
//   dq  = s e^G (dO S0^T) + sum_{x<=t} s dAqk[t,x] kw[x] e^{G[t]-G[x]}
//   dk  = beta e^G dBw + beta_t sum_{x<t} dAkk[t,x] kw[x] e^{G[t]-G[x]}
//   dkw = e^{G_C-G} (U dS_C^T) + sum_{t>x} beta_t dAkk[t,x] k[t] e^{G[t]-G[x]}
//                              + sum_{t>=x} s dAqk[t,x] q[t] e^{G[t]-G[x]}
// (channel by channel).  Pairs in different 16-row blocks go through MFMA
// with the decay split at the block boundary -- every factor <= 1 -- and
// pairs inside a block are summed exactly (dAqk's blocks there in FP32, the
// write key in FP32 when the caller has it).  dG[t,c] = q dq + k dk - kw dkw
// per element, plus e^{G_C[c]} sum_v S0[c,v] dS_C[c,v] + sum_t kg dkg on the
// last row, with the two parts that cancel exactly (the Aqk diagonal and
// the last row's kg dkg) left out, and each pair's two halves formed from
// the same rounded factors.
// ---------------------------------------------------------------------------
template <typename T, int D>
struct FusedBwdPcLayout {
  static constexpr int LD = D + Pad<T>::v;
  static constexpr int LDC = C + Pad<T>::v;
  static constexpr int LDG = D + 4;
  static constexpr int RT = C * LD * (int)sizeof(T);
  static constexpr int CT = C * LDC * (int)sizeof(T);
  static constexpr int HT = D * LD * (int)sizeof(T);
  static constexpr int LDW = D + 4;                     // FP32 write-key tile
  static constexpr int KWF_BYTES = C * LDW * 4;
  static constexpr bool KWF_IN_H = KWF_BYTES <= HT;
  static constexpr int off_U = 0;                       // U      } phase 3: G [64][LDG], then the
  static constexpr int off_V = off_U + RT;              // V      }   transposed diagonal blocks
  static constexpr int off_T = off_V + RT;              // T      }
  static constexpr int off_dO = off_T + CT;             // dO, then K
  static constexpr int off_dU = off_dO + RT;            // dU, then dBv, then Q
  static constexpr int off_H = off_dU + RT;             // h, then dH, then kw in FP32 (when it fits)
  static constexpr int off_P2 = off_H + HT;             // s dAqk (strictly lower)
  static constexpr int off_P1 = off_P2 + CT;            // dAkk (strictly lower)
  static constexpr int off_beta = off_P1 + CT;
  static constexpr int off_p2d = off_beta + C * 4;      // [64] s dAqk[t,t], FP32
  static constexpr int off_hd = off_p2d + C * 4;        // [D]
  static constexpr int off_kg = off_hd + D * 4;         // [4][D]
  static constexpr int off_red = off_kg + 4 * D * 4;    // [kFW]
  // BF16: s dAqk's diagonal 16 x 16 blocks also in FP32, [4][16 t][16 x] then
  // [4][16 x][16 t] (FP32 tiles read them from P2 and its transposed copy)
  static constexpr bool P2B = sizeof(T) < 4;
  static constexpr int off_P2B = off_red + kFW * 4;
  static constexpr int off_KWf = KWF_IN_H ? off_H : off_P2B + (P2B ? 2 * 4 * 256 * 4 : 0);
  static constexpr int bytes = off_P2B + (P2B ? 2 * 4 * 256 * 4 : 0) + (KWF_IN_H ? 0 : KWF_BYTES);
  static constexpr int off_Q = off_dU;
  // phase 3, after G: the diagonal 16 x 16 blocks of dAkk and dAqk transposed, [4][16 x][16 t] each
  static constexpr int G_BYTES = C * LDG * 4;
  static constexpr int off_P1T = off_U + G_BYTES;
  static constexpr int off_P2T = off_P1T + 4 * 256 * (int)sizeof(T);
  static_assert(G_BYTES + 8 * 256 * (int)sizeof(T) <= off_dO, "G and the transposed blocks fit the U..T region");
  // FP32: the gate's FP64 remainder beside G (pair decays from hi and lo)
  static constexpr bool GLO = sizeof(T) == 4;
  static constexpr int off_Glo = off_P2T + 4 * 256 * (int)sizeof(T);
  static_assert(!GLO || off_Glo + G_BYTES <= off_dO, "G's remainder fits the U..T region");
  static_assert(bytes <= 160 * 1024, "LDS of one compute unit");
  static_assert(D * (D / Vec16<T>::N) * 4 <= CT, "row partials of sum(h * dH) fit the T region");
};

// The body for one chunk; `len` is a literal C for whole chunks (every row
// test of the tile loads folds away, so no branch holds a load back).
template <typename T, int D, typename OT, typename OK>
__device__ __forceinline__ void fused_bwd_pc(const BwdParams& p, const ChunkInfo ci, const int len, char* smem) {
  using L = FusedBwdPcLayout<T, D>;
  using E = T;
  using F = FragK<E>;
  constexpr int HCT = D / 32;
  const int H = p.H;
  const ChunkHead wg = chunk_head<false>(H);
  const int cid = wg.cid, hh = wg.h;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  // waves w and w + 4 share a SIMD: they take row blocks rb and 3 - rb, whose
  // cross-block pair work (later blocks for small rb, earlier ones for large)
  // adds up to the same on every SIMD
  const int ch = wave >> 2, rb = ch ? 3 - (wave & 3) : (wave & 3);
  const int r0 = 16 * rb;
  const int64_t gs = (int64_t)H * D;
  const int64_t row0 = (int64_t)ci.start * H + hh;

  E* sU = reinterpret_cast<E*>(smem + L::off_U);
  float* sG = reinterpret_cast<float*>(smem + L::off_U);
  E* sT = reinterpret_cast<E*>(smem + L::off_T);
  E* sdO = reinterpret_cast<E*>(smem + L::off_dO);
  E* sK = sdO;
  E* sdU = reinterpret_cast<E*>(smem + L::off_dU);
  E* sdBv = sdU;
  E* sH = reinterpret_cast<E*>(smem + L::off_H);
  E* sQ = reinterpret_cast<E*>(smem + L::off_Q);
  float* sKWf = reinterpret_cast<float*>(smem + L::off_KWf);
  E* sP2 = reinterpret_cast<E*>(smem + L::off_P2);
  E* sP1r = reinterpret_cast<E*>(smem + L::off_P1);
  E* sP1T = reinterpret_cast<E*>(smem + L::off_P1T);
  E* sP2T = reinterpret_cast<E*>(smem + L::off_P2T);
  float* sP2B = reinterpret_cast<float*>(smem + L::off_P2B);
  float* sP2BT = sP2B + 4 * 256;
  float* sBeta = reinterpret_cast<float*>(smem + L::off_beta);
  float* sP2d = reinterpret_cast<float*>(smem + L::off_p2d);
  float* sHD = reinterpret_cast<float*>(smem + L::off_hd);
  float* sKG = reinterpret_cast<float*>(smem + L::off_kg);
  float* sRed = reinterpret_cast<float*>(smem + L::off_red);
  float* sGlo = reinterpret_cast<float*>(smem + L::off_Glo);  // FP32, phase 3
  // G's remainder at (row, column) of the phase 3 tile (0 unless FP32)
  auto glo = [&](int r, int c) -> float {
    if constexpr (L::GLO) return sGlo[r * L::LDG + c];
    else return 0.f;
  };

  const T* hsrc = static_cast<const T*>(p.h) + ((int64_t)cid * H + hh) * D * D;
  const T* dhsrc = static_cast<const T*>(p.dh) + ((int64_t)cid * H + hh) * D * D;
  const T* kg_ = static_cast<const T*>(p.k) + row0 * D;
  const T* kwg = static_cast<const T*>(p.kw) + row0 * D;
  const float* kw32g = p.kw32 ? p.kw32 + row0 * D : nullptr;
  const float* gg = p.gcum + row0 * D;        // G rows, stride gs
  const float* ggl = p.gcum_lo ? p.gcum_lo + row0 * D : nullptr;  // FP32: G's remainder
  const float* gC = gg + (int64_t)(len - 1) * gs;
  const float scale = p.scale;

  // G at this lane's accumulator positions (rows r0 + 4 (lane / 16) + e,
  // column 16 (ch HCT + j) + lane % 16) is read there by phases 1 to 2b: loaded
  // where phase 1 first needs it and kept.  K waits in registers behind the
  // first tiles and takes dO's region once phase 1 is done with it.  (A wait
  // for a load covers every load issued before it, so loads go in the order
  // they are needed.)
  const int rq = 4 * (lane >> 4);
  float Gl[HCT][4], gCl[HCT];
  float Gll[HCT][4], gCll[HCT];  // FP32: the remainders (zero without gcum_lo)
  RegTile<kFW, C, D, T> rK;
  // beta first: its LDS store below then waits for this load only
  const float bval = p.beta[(int64_t)(ci.start + min(tid & (C - 1), len - 1)) * H + hh];
  {
    RegTile<kFW, C, D, T> rU, rdO, rdU;
    RegTile<kFW, C, C, T> rT;
    TiledTile<kFW, D, T> rH;
    rU.load(static_cast<const T*>(p.u) + row0 * D, gs, len);
    rdO.load(static_cast<const T*>(p.dO) + row0 * D, gs, len);
    rdU.load(static_cast<const T*>(p.du) + row0 * D, gs, len);
    rT.load(static_cast<const T*>(p.akk) + row0 * C, (int64_t)H * C, len);
    rH.load(hsrc);
    rK.load(kg_, gs, len);
    // every thread writes (the C rows' values, repeated): no branch to hold
    // the tile loads after it behind this load
    sBeta[tid & (C - 1)] = (tid & (C - 1)) < len ? bval : 0.f;
    rU.store(sU, L::LD);
    rdO.store(sdO, L::LD);
    rdU.store(sdU, L::LD);
    rT.store(sT, L::LDC);
    rH.store(sH, L::LD);
  }
  __syncthreads();

  f32x4 dq[HCT], dk[HCT], dv[HCT], dkws[HCT];
  // dbeta_t = sum_c dBv[t,c] U[t,c] / beta_t (every beta-dependent quantity of
  // the chunk is row t scaled by beta_t, so U_t = beta_t r_t and the adjoint
  // of the row is dBv_t); db gathers the three-term form (dBv V, the Bw and
  // the Akk parts), which rows with |beta_t| < 1e-20 take, their V alone read
  float db[4] = {0.f, 0.f, 0.f, 0.f}, dbu[4] = {0.f, 0.f, 0.f, 0.f};
  bool tiny[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int r = r0 + acc_row(lane, e);
    tiny[e] = r < len && !(fabsf(sBeta[r]) >= 1e-20f);
  }
  const int kbeg = kfloor<E>(r0);
  // ---- phase 1: dQg = dO S0^T, dAqk = dO U^T, dBv = T^T dU ------------------------
  // (dk's WY part goes through dBv too: with (Bv - Bw S0) = T^-1 U,
  //   dBw = T^T dW = -dBv S0^T  and  dAkk = -T^T dT T^T = -dBv U^T,
  // so neither dW nor dT is formed.)
#pragma unroll
  for (int j = 0; j < HCT; ++j) {
    const int ct = ch * HCT + j;
    const int c = 16 * ct + acc_col(lane);
    f32x4 acc = zero4();
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      Gl[j][e] = gg[(int64_t)min(r0 + rq + e, len - 1) * gs + c];
      if constexpr (L::GLO) Gll[j][e] = ggl ? ggl[(int64_t)min(r0 + rq + e, len - 1) * gs + c] : 0.f;
    }
    mma_tile<E, ROW, COL>(acc, sdO, L::LD, r0, sH, L::LD, 16 * ct, D, lane);
#pragma unroll
    for (int e = 0; e < 4; ++e) dq[j][e] = scale * exp_fast(Gl[j][e]) * acc[e];
    f32x4 acv = zero4();
    mma_tile_range<E, COL, ROW>(acv, sT, L::LDC, r0, sdU, L::LD, 16 * ct, kbeg, C, lane);  // dBv = T^T dU
    dv[j] = acv;  // dBv until it is in LDS
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = r0 + acc_row(lane, e);
      dbu[e] += acv[e] * from_e<E>(sU[r * L::LD + c]);
      if (tiny[e]) db[e] += acv[e] * io<T>::load(static_cast<const T*>(p.v) + row0 * D + (int64_t)r * gs + c);
    }
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int ct = 2 * ch + j;
    f32x4 acc = zero4();
    if (ct <= rb) mma_tile<E, ROW, COL>(acc, sdO, L::LD, r0, sU, L::LD, 16 * ct, D, lane);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = r0 + acc_row(lane, e), s = 16 * ct + acc_col(lane);
      // the diagonal is kept apart in FP32 (its gate-gradient terms cancel)
      const float val = (s < t && t < len) ? scale * acc[e] : 0.f;
      sP2[t * L::LDC + s] = to_e<E>(val);
      if (s == t) sP2d[t] = t < len ? scale * acc[e] : 0.f;
      // In-block pairs are summed exactly from FP32 values: their gate terms
      // carry the largest decay factors, and a BF16 copy of dAqk there moves
      // dA_log by ~1e-2.
      if (L::P2B && ct == rb) {
        sP2B[(16 * rb + t - r0) * 16 + s - r0] = val;
        sP2BT[(16 * rb + s - r0) * 16 + t - r0] = val;
      }
    }
  }
  __syncthreads();
  // the next phases' operands start their way in: G_C, dH and the write key at
  // this lane's positions (0 past the chunk).  The eight waves' Gl and Wl
  // cover the [64 x D] tiles once, so phase 3 takes its LDS copies of G and
  // the write key from them rather than from global memory again.
#pragma unroll
  for (int j = 0; j < HCT; ++j) {
    gCl[j] = gC[16 * (ch * HCT + j) + (lane & 15)];
    if constexpr (L::GLO) gCll[j] = ggl ? ggl[(int64_t)(len - 1) * gs + 16 * (ch * HCT + j) + (lane & 15)] : 0.f;
  }
  TiledTile<kFW, D, T> rdH;
  rdH.load(dhsrc);
  // (rows clamped into the chunk and every load unconditional, so the
  // sixteen go out together; rows past the chunk are zeroed where phase 3
  // stores them)
  float Wl[HCT][4];
  if (kw32g) {
#pragma unroll
    for (int j = 0; j < HCT; ++j) {
      const int c = 16 * (ch * HCT + j) + (lane & 15);
#pragma unroll
      for (int e = 0; e < 4; ++e) Wl[j][e] = kw32g[(int64_t)min(r0 + rq + e, len - 1) * gs + c];
    }
  } else {
#pragma unroll
    for (int j = 0; j < HCT; ++j) {
      const int c = 16 * (ch * HCT + j) + (lane & 15);
#pragma unroll
      for (int e = 0; e < 4; ++e) Wl[j][e] = io<T>::load(kwg + (int64_t)min(r0 + rq + e, len - 1) * gs + c);
    }
  }
  rK.store(sK, L::LD);  // dO's region: phase 1 is done with it
  // dBv over dU (every wave has read dU); dv = beta dBv
#pragma unroll
  for (int j = 0; j < HCT; ++j) {
    store_acc_lds(sdBv, L::LD, dv[j], r0, 16 * (ch * HCT + j), lane);
#pragma unroll
    for (int e = 0; e < 4; ++e) dv[j][e] *= sBeta[r0 + acc_row(lane, e)];
  }
  __syncthreads();
  // ---- phase 2: dBw = -dBv S0^T (-> dk), dAkk = -dBv U^T ------------------------
#pragma unroll
  for (int j = 0; j < HCT; ++j) {
    const int ct = ch * HCT + j;
    const int c = 16 * ct + acc_col(lane);
    f32x4 acc = zero4();
    mma_tile<E, ROW, COL>(acc, sdBv, L::LD, r0, sH, L::LD, 16 * ct, D, lane);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int s = r0 + acc_row(lane, e);
      const float eg = exp_fast(Gl[j][e]);
      dk[j][e] = -sBeta[s] * eg * acc[e];
      db[e] -= acc[e] * eg * from_e<E>(sK[s * L::LD + c]);
    }
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int ct = 2 * ch + j;
    f32x4 acc = zero4();
    if (ct <= rb) mma_tile<E, ROW, COL>(acc, sdBv, L::LD, r0, sU, L::LD, 16 * ct, D, lane);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = r0 + acc_row(lane, e), s = 16 * ct + acc_col(lane);
      sP1r[t * L::LDC + s] = to_e<E>((s < t && t < len) ? -acc[e] : 0.f);  // dAkk
    }
  }
  __syncthreads();
  // ---- phase 2b: dH replaces S0; per-row sum(S0 * dH); dKg = U dH^T --------------
  // phase 3's Q starts its way in (its region, dBv's, is dead)
  RegTile<kFW, C, D, T> rQ;
  rQ.load(static_cast<const T*>(p.q) + row0 * D, gs, len);
  // (dH arrives tile-major: per-piece partial sums go through the T region,
  // dead since phase 1, and are summed per row in a fixed order)
  {
    constexpr int V = Vec16<T>::N;
    constexpr int PPR = D / V;  // pieces per row
    float* sPart = reinterpret_cast<float*>(smem + L::off_T);
#pragma unroll
    for (int i = 0; i < TiledTile<kFW, D, T>::ITER; ++i) {
      int r, c;
      rdH.pos(i, r, c);
      float x[V], hv[V];
      Vec16<T>::unpack(rdH.r[i], x);
      lds_vec<V>(sH + r * L::LD + c, hv);
      float part = 0.f;
#pragma unroll
      for (int j = 0; j < V; ++j) part += hv[j] * x[j];
      *reinterpret_cast<uint4*>(sH + r * L::LD + c) = rdH.r[i];  // this thread's own slots
      sPart[r * PPR + c / V] = part;
    }
    __syncthreads();
    if (tid < D) {
      float sum = 0.f;
      for (int k = 0; k < PPR; ++k) sum += sPart[tid * PPR + k];
      sHD[tid] = sum;
    }
  }
#pragma unroll
  for (int j = 0; j < HCT; ++j) {
    const int ct = ch * HCT + j;
    f32x4 acc = zero4();
    mma_tile<E, ROW, COL>(acc, sU, L::LD, r0, sH, L::LD, 16 * ct, D, lane);
    float col = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float gdc = gCl[j] - Gl[j][e];
      if constexpr (L::GLO) gdc += gCll[j] - Gll[j][e];
      dkws[j][e] = exp_fast(gdc) * acc[e];
      // the last row's term (decay e^0) cancels against its own -kw dkw: left out
      col += (r0 + rq + e < len - 1 ? Wl[j][e] : 0.f) * dkws[j][e];
    }
    col += __shfl_xor(col, 16);
    col += __shfl_xor(col, 32);
    if (lane < 16) sKG[rb * D + 16 * ct + lane] = col;
  }
  __syncthreads();
  // ---- phase 3: pairwise terms with the decay inside the contraction ----------
  // dAkk is held once (unscaled); beta_t multiplies the other factor, so the
  // two halves of each (t, x) pair's gate term see the same rounded value.
  // G (rows past the chunk repeat its last) and the write key in FP32 (kw32,
  // else kw or k widened; zero rows past the chunk) from this lane's Gl, Wl.
  rQ.store(sQ, L::LD);
#pragma unroll
  for (int j = 0; j < HCT; ++j) {
    const int c = 16 * (ch * HCT + j) + (lane & 15);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sG[(r0 + rq + e) * L::LDG + c] = L::GLO ? Gl[j][e] : Gl[j][e] * kLog2e;
      if constexpr (L::GLO) sGlo[(r0 + rq + e) * L::LDG + c] = Gll[j][e];
      sKWf[(r0 + rq + e) * L::LDW + c] = r0 + rq + e < len ? Wl[j][e] : 0.f;
    }
  }
  if (ch == 0) {  // this row block's diagonal blocks, transposed
    for (int i = lane; i < 256; i += 64) {
      const int xo = i >> 4, to = i & 15;
      sP1T[(16 * rb + xo) * 16 + to] = sP1r[(r0 + to) * L::LDC + r0 + xo];
      if (!L::P2B) sP2T[(16 * rb + xo) * 16 + to] = sP2[(r0 + to) * L::LDC + r0 + xo];
    }
  }
  __syncthreads();
  const int rlo = r0 - 1;   // last row before this row block (G[-1] = 0)
  // Pairs (t, x) in different row blocks go through MFMA with the decay split
  // at R = (first row of t's block) - 1: e^{G[t]-G[x]} = e^{G[t]-G[R]} e^{G[R]-G[x]},
  // each factor <= 1.  The row side (t) takes kw[x] e^{G[R]-G[x]} as its B
  // operand, the column side (x) takes q[t] e^{G[t]-G[R]} (or beta k) -- both
  // rounded to the MFMA's input type.  The gate gradient of a pair enters row t
  // and row x with opposite signs and must cancel in the chunk's reverse sum:
  // both halves are formed from the same two rounded factors (a row half
  // a(t) * sum_x P b(x), a column half b(x) * sum_t P a(t)).  Formed from the
  // unrounded factor on one side, the halves differ by the operand's rounding
  // and dA_log, a sum of the gate gradient over the whole head, moves by ~4e-2.
  auto rnd = [](float x) { return from_e<E>(to_e<E>(x)); };
  OT* dqo = static_cast<OT*>(p.dq) + row0 * D;
  OK* dko = static_cast<OK*>(p.dk) + row0 * D;
  OK* dkwo = p.dkw ? static_cast<OK*>(p.dkw) + row0 * D : nullptr;
  OT* dvo = static_cast<OT*>(p.dv) + row0 * D;
#pragma unroll
  for (int j = 0; j < HCT; ++j) store_acc_global<OT>(dvo, gs, dv[j], r0, 16 * (ch * HCT + j), len, lane);
  // Each pass works on slot 0 of dq, dk and dkws, which hold column tile
  // ch HCT + j at pass j.  dq, dk and dkw leave two adjacent column tiles of
  // a row block together, so each BF16 row piece is a 64-byte span (one tile
  // alone would write 32-byte pieces, half a cache line, one pass apart).
  TileGroupStore<OT, 2> st_q;
  TileGroupStore<OK, 2> st_k, st_w;
#pragma unroll 1
  for (int j = 0; j < HCT; ++j) {
    const int ct = ch * HCT + j;
    const int c = 16 * ct + acc_col(lane);
    const int nn = 16 * ct + (lane & 15);  // this lane's B column (== c)
    float gr[4], grl[4], kv[4], qv[4], wv[4];
    f32x4 dg, dkwj;
    // the decay between two rows: G[a] - G[b] from hi and (FP32) the remainders
    auto gdv = [&](float a, float al, float b, float bl) -> float {
      if constexpr (L::GLO) return (a - b) + (al - bl);
      else return a - b;
    };
    // e^d for a difference d of staged G values: without the FP32 remainders
    // G is staged times log2 e, so each exponential is one exp2 (the multiply
    // by log2 e done once per element at staging, not once per pair)
    auto exg = [](float d) -> float {
      if constexpr (L::GLO) return exp_fast(d);
      else return exp2_fast(d);
    };
    {
      float kgc = 0.f;
#pragma unroll
      for (int b = 0; b < 4; ++b) kgc += sKG[b * D + c];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = r0 + rq + e;
        gr[e] = sG[r * L::LDG + c];
        grl[e] = glo(r, c);
        kv[e] = from_e<E>(sK[r * L::LD + c]);
        qv[e] = from_e<E>(sQ[r * L::LD + c]);
        wv[e] = sKWf[r * L::LDW + c];
        const float pd = sP2d[r];
        // terms without a pair: the state parts of dq, dk and dkw; the Aqk
        // diagonal and the last row's state-path write-key term (decay e^0)
        // enter two of q dq, kw dkw and sum(kg dkg) with opposite signs and
        // are left out of the gate gradient
        dg[e] = qv[e] * dq[0][e] + kv[e] * dk[0][e] - (r == len - 1 ? 0.f : wv[e] * dkws[0][e]);
        if (r == len - 1) dg[e] += exg(sG[(C - 1) * L::LDG + c]) * sHD[c] + kgc;
        dq[0][e] += pd * wv[e];
        dkwj[e] = dkws[0][e] + pd * qv[e];
      }
    }
    // (1) rows t_e = r0 + rq + e of this block, x <= t_e inside it, exactly
    // (pairs with x > t_e vanish: dAkk and dAqk are zero on and above the
    // diagonal, dAqk's diagonal being held apart).  For x <= t_0 the decay
    // factors as e^{G[t_e]-G[x]} = R_e E(x), R_e = e^{G[t_e]-G[t_0]},
    // E(x) = e^{G[t_0]-G[x]} the running product of the per-token decays
    // e^{G[y]-G[y-1]} from x + 1 to t_0 (every factor <= 1, so no overflow for
    // any gate); the pairs with x in (t_0, t_e] take their factor directly.
    {
      f32x4 ak = zero4(), aq = zero4();
#pragma unroll
      for (int u = 1; u < 3; ++u) {  // x = t_u, rows e > u
        float p1[4], p2[4];
        lds4(sP1T + (16 * rb + rq + u) * 16 + rq, p1);
        if constexpr (L::P2B) lds4(sP2BT + (16 * rb + rq + u) * 16 + rq, p2);
        else lds4(sP2T + (16 * rb + rq + u) * 16 + rq, p2);
#pragma unroll
        for (int e = u + 1; e < 4; ++e) {
          const float w = wv[u] * exg(gdv(gr[e], grl[e], gr[u], grl[u]));
          ak[e] += p1[e] * w;
          aq[e] += p2[e] * w;
        }
      }
      float ak0[4] = {0.f, 0.f, 0.f, 0.f}, aq0[4] = {0.f, 0.f, 0.f, 0.f};
      {  // x = t_0: the product starts at 1
        float p1[4], p2[4];
        lds4(sP1T + (16 * rb + rq) * 16 + rq, p1);
        if constexpr (L::P2B) lds4(sP2BT + (16 * rb + rq) * 16 + rq, p2);
        else lds4(sP2T + (16 * rb + rq) * 16 + rq, p2);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ak0[e] += p1[e] * wv[0];
          aq0[e] += p2[e] * wv[0];
        }
      }
      // x in the block's earlier 4-row groups (x < t_0): FP32 MFMA steps, one
      // per (row group g, key group j < g), the decay split at t_0 of group g:
      // B = kw[x] e^{G[t_0(g)]-G[x]} (<= 1), A = the rows of group g (the other
      // rows zero), so the lanes of group g receive exactly their rows' sums.
      {
        const int mrow = lane & 15, kq = lane >> 4, ag = mrow >> 2;
        float g0[4], g0l[4];
#pragma unroll
        for (int g = 1; g < 4; ++g) {
          g0[g] = sG[(r0 + 4 * g) * L::LDG + nn];
          g0l[g] = glo(r0 + 4 * g, nn);
        }
        f32x4 mk = zero4(), mq = zero4();
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const int x = r0 + 4 * j + kq;  // this lane's B row
          const float gx = sG[x * L::LDG + nn], gxl = glo(x, nn);
          const float kwx = sKWf[x * L::LDW + nn];
          const float a1 = from_e<E>(sP1r[(r0 + mrow) * L::LDC + x]);
          float a2;
          if constexpr (L::P2B) a2 = sP2B[(16 * rb + mrow) * 16 + 4 * j + kq];
          else a2 = from_e<E>(sP2[(r0 + mrow) * L::LDC + x]);
#pragma unroll
          for (int g = j + 1; g < 4; ++g) {
            const float bx = kwx * exg(gdv(g0[g], g0l[g], gx, gxl));
            Mma<float>::mfma(mk, ag == g ? a1 : 0.f, bx);
            Mma<float>::mfma(mq, ag == g ? a2 : 0.f, bx);
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ak0[e] += mk[e];
          aq0[e] += mq[e];
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float R = e == 0 ? 1.f : exg(gdv(gr[e], grl[e], gr[0], grl[0]));
        ak[e] += R * ak0[e];
        aq[e] += R * aq0[e];
        const float bk = sBeta[r0 + rq + e] * ak[e];
        dk[0][e] += bk;
        db[e] += kv[e] * ak[e];
        dq[0][e] += aq[e];
        dg[e] += qv[e] * aq[e] + kv[e] * bk;
      }
    }
    // (2) rows t of this block, x in earlier blocks: split at rlo
    if (rb > 0) {
      f32x4 akX = zero4(), aqX = zero4();
      const float grlo = sG[rlo * L::LDG + nn], grlo_l = glo(rlo, nn);
      if constexpr (sizeof(E) == 2) {
        // 16-deep steps cover exactly the earlier blocks: A = rows of dAkk and
        // s dAqk (four consecutive x, one 8-byte read each), B = kw e^{G[R]-G[x]}
        for (int k0 = 0; k0 < r0; k0 += 16) {
          const int kk = k0 + 4 * (lane >> 4);
          const s16x4_t a1 = *reinterpret_cast<const s16x4_t*>(sP1r + (r0 + (lane & 15)) * L::LDC + kk);
          const s16x4_t a2 = *reinterpret_cast<const s16x4_t*>(sP2 + (r0 + (lane & 15)) * L::LDC + kk);
          float bx[4];
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int x = kk + jj;
            bx[jj] = sKWf[x * L::LDW + nn] * exg(grlo - sG[x * L::LDG + nn]);
          }
          const s16x4_t b = pack_bf16x4(bx);
          mfma16_bf16(akX, a1, b);
          mfma16_bf16(aqX, a2, b);
        }
      } else for (int k0 = 0; k0 < kceil<E>(r0); k0 += Mma<E>::KS) {
        const int kk = k0 + F::off(lane);
        float a1[F::N], a2[F::N], bx[F::N];
#pragma unroll
        for (int jj = 0; jj < F::N; ++jj) {
          const int x = kk + jj;
          a1[jj] = from_e<E>(sP1r[(r0 + (lane & 15)) * L::LDC + x]);
          a2[jj] = from_e<E>(sP2[(r0 + (lane & 15)) * L::LDC + x]);
          bx[jj] = x <= rlo ? sKWf[x * L::LDW + nn] * exg(gdv(grlo, grlo_l, sG[x * L::LDG + nn], glo(x, nn)))
                            : 0.f;
        }
        F::mfma(akX, a1, bx);
        F::mfma(aqX, a2, bx);
      }
      const float grlo_c = sG[rlo * L::LDG + c], grlo_cl = glo(rlo, c);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float sb = sBeta[r0 + rq + e];
        const float dlo = exg(gdv(gr[e], grl[e], grlo_c, grlo_cl));  // e^{G[t]-G[R]}
        dk[0][e] += sb * dlo * akX[e];
        db[e] += kv[e] * dlo * akX[e];
        dq[0][e] += dlo * aqX[e];
        // the column side's B operands of these pairs: beta k e^{G[t]-G[R]}, q e^{G[t]-G[R]}
        dg[e] += rnd(sb * kv[e] * dlo) * akX[e] + rnd(qv[e] * dlo) * aqX[e];
      }
    }
    // (3) rows x_e = r0 + rq + e of this block as the key, t > x_e inside it,
    // exactly, as (1): for t > t_3, e^{G[t]-G[x_e]} = E'(t) R'_e with
    // E'(t) = e^{G[t]-G[t_3]} (running product from t_3 + 1) and
    // R'_e = e^{G[t_3]-G[x_e]}; t in (x_e, t_3] directly.
    {
      f32x4 aw = zero4();
#pragma unroll
      for (int u = 1; u < 4; ++u) {  // t = t_u, keys e < u
        const int t = r0 + rq + u;
        float p1[4], p2[4];
        lds4(sP1r + t * L::LDC + r0 + rq, p1);
        if constexpr (L::P2B) lds4(sP2B + (16 * rb + rq + u) * 16 + rq, p2);
        else lds4(sP2 + t * L::LDC + r0 + rq, p2);
        const float kx = sBeta[t] * kv[u], qx = qv[u];
#pragma unroll
        for (int e = 0; e < u; ++e) aw[e] += (p1[e] * kx + p2[e] * qx) * exg(gdv(gr[u], grl[u], gr[e], grl[e]));
      }
      // t in the block's later 4-row groups (t > t_3): FP32 MFMA steps, one per
      // (key group g, row group i > g), the decay split at t_3 of group g:
      // B = beta k[t] e^{G[t]-G[t_3(g)]} and q[t] e^{G[t]-G[t_3(g)]} (<= 1),
      // A = dAkk and s dAqk columns of group g (the other columns zero).
      float aw0[4] = {0.f, 0.f, 0.f, 0.f};
      {
        const int mrow = lane & 15, kq = lane >> 4, ag = mrow >> 2;
        float g3[3], g3l[3];
#pragma unroll
        for (int g = 0; g < 3; ++g) {
          g3[g] = sG[(r0 + 4 * g + 3) * L::LDG + nn];
          g3l[g] = glo(r0 + 4 * g + 3, nn);
        }
        f32x4 mw = zero4();
#pragma unroll
        for (int i = 1; i < 4; ++i) {
          const int t = r0 + 4 * i + kq;  // this lane's B row
          const float gt = sG[t * L::LDG + nn], gtl = glo(t, nn);
          const float kt = sBeta[t] * from_e<E>(sK[t * L::LD + nn]);
          const float qt = from_e<E>(sQ[t * L::LD + nn]);
          const float a1 = from_e<E>(sP1r[t * L::LDC + r0 + mrow]);
          float a2;
          if constexpr (L::P2B) a2 = sP2B[(16 * rb + 4 * i + kq) * 16 + mrow];
          else a2 = from_e<E>(sP2[t * L::LDC + r0 + mrow]);
#pragma unroll
          for (int g = 0; g < i; ++g) {
            const float f = exg(gdv(gt, gtl, g3[g], g3l[g]));
            Mma<float>::mfma(mw, ag == g ? a1 : 0.f, kt * f);
            Mma<float>::mfma(mw, ag == g ? a2 : 0.f, qt * f);
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) aw0[e] = mw[e];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        aw[e] += (e == 3 ? 1.f : exg(gdv(gr[3], grl[3], gr[e], grl[e]))) * aw0[e];
        dkwj[e] += aw[e];
        dg[e] -= wv[e] * aw[e];
      }
    }
    // (4) rows x of this block, t in each later block bi: split at 16 bi - 1
    for (int bi = rb + 1; bi < 4; ++bi) {
      const int R = 16 * bi - 1;
      const float gR = sG[R * L::LDG + nn], gRl = glo(R, nn);
      f32x4 aw = zero4();
      if constexpr (sizeof(E) == 2) {
        // one 16-deep step over block bi: A = dAkk and s dAqk columns x (their
        // rows t k-major: transposed reads), B = beta k e^{G[t]-G[R]} and
        // q e^{G[t]-G[R]} from K and Q read the same way
        const s16x4_t a1 = lds_read_kmajor4(sP1r + r0, L::LDC, 16 * bi, lane);
        const s16x4_t a2 = lds_read_kmajor4(sP2 + r0, L::LDC, 16 * bi, lane);
        const s16x4_t kt = lds_read_kmajor4(sK + 16 * ct, L::LD, 16 * bi, lane);
        const s16x4_t qt = lds_read_kmajor4(sQ + 16 * ct, L::LD, 16 * bi, lane);
        float b1[4], b2[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int t = 16 * bi + 4 * (lane >> 4) + jj;
          const float f = exg(sG[t * L::LDG + nn] - gR);
          b1[jj] = sBeta[t] * bf16_to_f32(static_cast<bf16_t>(kt[jj])) * f;  // beta_t on the key, dAkk unscaled
          b2[jj] = bf16_to_f32(static_cast<bf16_t>(qt[jj])) * f;
        }
        mfma16_bf16(aw, a1, pack_bf16x4(b1));
        mfma16_bf16(aw, a2, pack_bf16x4(b2));
      } else for (int k0 = kfloor<E>(16 * bi); k0 < 16 * bi + 16; k0 += Mma<E>::KS) {
        const int kk = k0 + F::off(lane);
        float a1[F::N], a2[F::N], b1[F::N], b2[F::N];
#pragma unroll
        for (int jj = 0; jj < F::N; ++jj) {
          const int t = kk + jj;
          a1[jj] = from_e<E>(sP1r[t * L::LDC + r0 + (lane & 15)]);
          a2[jj] = from_e<E>(sP2[t * L::LDC + r0 + (lane & 15)]);
          const float f = t > R && t <= R + 16 ? exg(gdv(sG[t * L::LDG + nn], glo(t, nn), gR, gRl)) : 0.f;
          b1[jj] = sBeta[t] * from_e<E>(sK[t * L::LD + nn]) * f;  // beta_t on the key, dAkk unscaled
          b2[jj] = from_e<E>(sQ[t * L::LD + nn]) * f;
        }
        F::mfma(aw, a1, b1);
        F::mfma(aw, a2, b2);
      }
      const float gRc = sG[R * L::LDG + c], gRcl = glo(R, c);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float dec = exg(gdv(gRc, gRcl, gr[e], grl[e]));  // e^{G[R]-G[x]}
        dkwj[e] += dec * aw[e];
        dg[e] -= rnd(wv[e] * dec) * aw[e];  // the row side's B operand kw e^{G[R]-G[x]}
      }
    }
    store_acc_global<float>(p.dgcum + row0 * D, gs, dg, r0, 16 * ct, len, lane);
    // this column tile's dq, dk and dkw are final
    st_q.put(dqo, gs, dq[0], r0, 16 * ct, len, lane, j & 1);
    if (p.kw_is_k) {
      st_k.put(dko, gs, dk[0] + dkwj, r0, 16 * ct, len, lane, j & 1);
    } else {
      st_k.put(dko, gs, dk[0], r0, 16 * ct, len, lane, j & 1);
      st_w.put(dkwo, gs, dkwj, r0, 16 * ct, len, lane, j & 1);
    }
    // the next tile's accumulators move into slot 0 (fixed registers: a
    // runtime index into the arrays would go through indexed register moves)
#pragma unroll
    for (int t = 0; t + 1 < HCT; ++t) {
      dq[t] = dq[t + 1];
      dk[t] = dk[t + 1];
      dkws[t] = dkws[t + 1];
    }
  }
  float* sRowB = sRed;          // [2][64] the three-term form
  float* sRowU = sRed + 2 * C;  // [2][64] sum_c dBv U
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float b = group16_sum(db[e]);
    const float bu = group16_sum(dbu[e]);
    if ((lane & 15) == 0) {
      sRowB[ch * C + r0 + acc_row(lane, e)] = b;
      sRowU[ch * C + r0 + acc_row(lane, e)] = bu;
    }
  }
  __syncthreads();
  if (tid < len) {
    const float bt = sBeta[tid];
    p.dbeta[(int64_t)(ci.start + tid) * H + hh] =
        fabsf(bt) >= 1e-20f ? (sRowU[tid] + sRowU[C + tid]) / bt : sRowB[tid] + sRowB[C + tid];
  }
}

template <typename T, int D, typename OT, typename OK>
__global__ __launch_bounds__(kFW) void chunk_fused_bwd_pc_kernel(BwdParams p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const ChunkHead wg = chunk_head<false>(p.H);
  if (wg.cid >= p.geom.num_chunks) return;
  const ChunkInfo ci = chunk_info(p.geom, wg.cid);
  if (ci.len == C) fused_bwd_pc<T, D, OT, OK>(p, ci, C, smem);
  else if (ci.len > 0) fused_bwd_pc<T, D, OT, OK>(p, ci, ci.len, smem);
}

template <typename K>
int set_smem(K kernel, int bytes) {
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) {
    set_error("hipFuncSetAttribute(%d bytes): %s", bytes, hipGetErrorString(e));
    return static_cast<int>(e);
  }
  return 0;
}

// ---------------------------------------------------------------------------
// reverse state pass, BF16 with a per-head gate: register-resident form
//
// The structure of the forward's register-resident pass, chunks in reverse:
// BV/16 compute waves each keep dS [D x 16] in MFMA accumulators and the
// chunk's dU [64 x 16] in registers, and kRrLoaders loader waves stage the
// read-only tiles (Q, KW, K when it is not KW, Aqk, T, the dO slice, G and
// beta) through a double-buffered LDS stage, two groups taking alternate
// chunks.  Per chunk, with W = T diag(beta e^G) K never formed:
//   dU  = Aqk^T dO + diag(e^{G_C - G}) (KW dS)
//   dBv = T^T dU                                          -> du
//   dS <- e^{G_C} dS + Q^T diag(s e^G) dO - K^T diag(beta e^G) dBv
// ---------------------------------------------------------------------------
template <int D, int BV, bool ALIAS>
struct RrBwdLayout {
  static constexpr int LD = D + Pad<bf16_t>::v;
  static constexpr int LDV = BV + Pad<bf16_t>::v;
  static constexpr int LDC = C + Pad<bf16_t>::v;
  static constexpr int off_Q = 0;
  static constexpr int off_KW = off_Q + C * LD * 2;
  static constexpr int off_K = off_KW + C * LD * 2;               // K when it is not KW
  static constexpr int off_A = off_K + (ALIAS ? 0 : C * LD * 2);  // Aqk
  static constexpr int off_T = off_A + C * LDC * 2;
  static constexpr int off_dO = off_T + C * LDC * 2;
  static constexpr int off_G = off_dO + C * LDV * 2;
  static constexpr int off_B = off_G + C * 4;                     // beta (0 past the chunk's end)
  static constexpr int BUF = off_B + C * 4;
  // Output stage (where it fits): the compute waves leave each chunk's dBv
  // rows here, double-buffered, and the loader group that is not staging
  // inputs in that step writes them to global memory.
  static constexpr int OUT = C * LDV * 2;
  static constexpr bool STAGE_OUT = 2 * BUF + 2 * OUT <= 160 * 1024;
  static constexpr int off_Out = 2 * BUF;
  static constexpr int bytes = 2 * BUF + (STAGE_OUT ? 2 * OUT : 0);
  static_assert(BUF % 16 == 0 && (LDV * 2) % 16 == 0, "16-byte aligned stages and rows");
  static_assert(bytes <= 160 * 1024, "LDS of one compute unit");
};

constexpr int kRrLoadersBwd = 4;  // two groups of two waves

template <int D, int BV, bool ALIAS, bool PACK>
__global__ __launch_bounds__(64 * (BV / 16 + kRrLoadersBwd)) void chunk_state_bwd_rr_kernel(BwdParams p) {
  using L = RrBwdLayout<D, BV, ALIAS>;
  using T = bf16_t;
  constexpr int NC = BV / 16;
  constexpr int NKT = D / 16;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const DocSlot ds = doc_slot(p.geom, p.H, D / BV);
  const int n = ds.n, h = ds.h, v0 = ds.z * BV;
  const int H = p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t gs = (int64_t)H * D;
  int first, count, dstart, dlen;
  doc_chunks(p.geom, n, first, count, dstart, dlen);
  const bool loader = wave >= NC;

  // chunks are visited in the order s = 0, 1, ... as jc = count - 1 - s
  if (loader) {
    constexpr int NGT = 64 * kRrLoadersBwd / 2;
    const int lgroup = (tid - 64 * NC) / NGT;  // takes visits s with s % 2 == lgroup
    const int lt = (tid - 64 * NC) % NGT;
    RegTile<NGT, C, D, T> rQ, rKW, rK;
    std::conditional_t<PACK, TriRegTile<NGT>, RegTile<NGT, C, C, T>> rA, rT;
    RegTile<NGT, C, BV, T> rdO;
    float rg = 0.f, rb = 0.f;
    if constexpr (PACK) {  // the stages' blocks above the diagonal: zero once
      const int lt2 = tid - 64 * NC;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        zero_upper_blocks<2 * NGT>(lt2, reinterpret_cast<T*>(smem + b * L::BUF + L::off_A), L::LDC);
        zero_upper_blocks<2 * NGT>(lt2, reinterpret_cast<T*>(smem + b * L::BUF + L::off_T), L::LDC);
      }
    }
    auto load = [&](int s) {
      const int jc = count - 1 - s;
      const int cstart = dstart + jc * C;
      const int clen = min(C, dlen - jc * C);
      const int64_t row0 = (int64_t)cstart * H + h;
      rQ.load_as(lt, static_cast<const T*>(p.q) + row0 * D, gs, clen);
      rKW.load_as(lt, static_cast<const T*>(p.kw) + row0 * D, gs, clen);
      if (!ALIAS) rK.load_as(lt, static_cast<const T*>(p.k) + row0 * D, gs, clen);
      if constexpr (PACK) {
        const int64_t tri0 = ((int64_t)(first + jc) * H + h) * kTriElems;
        rA.load_as(lt, static_cast<const T*>(p.aqk) + tri0);
        rT.load_as(lt, static_cast<const T*>(p.akk) + tri0);
      } else {
        rA.load_as(lt, static_cast<const T*>(p.aqk) + row0 * C, (int64_t)H * C, clen);
        rT.load_as(lt, static_cast<const T*>(p.akk) + row0 * C, (int64_t)H * C, clen);
      }
      rdO.load_as(lt, static_cast<const T*>(p.dO) + row0 * D + v0, gs, clen);
      if (lt < C) {
        const int64_t gi = (int64_t)(cstart + min(lt, clen - 1)) * H + h;
        rg = p.gcum[gi];
        rb = lt < clen ? p.beta[gi] : 0.f;
      }
    };
    auto stash = [&](int b) {
      char* buf = smem + b * L::BUF;
      rQ.store_as(lt, reinterpret_cast<T*>(buf + L::off_Q), L::LD);
      rKW.store_as(lt, reinterpret_cast<T*>(buf + L::off_KW), L::LD);
      if (!ALIAS) rK.store_as(lt, reinterpret_cast<T*>(buf + L::off_K), L::LD);
      rA.store_as(lt, reinterpret_cast<T*>(buf + L::off_A), L::LDC);
      rT.store_as(lt, reinterpret_cast<T*>(buf + L::off_T), L::LDC);
      rdO.store_as(lt, reinterpret_cast<T*>(buf + L::off_dO), L::LDV);
      if (lt < C) {
        reinterpret_cast<float*>(buf + L::off_G)[lt] = rg;
        reinterpret_cast<float*>(buf + L::off_B)[lt] = rb;
      }
    };
    // visit s's dBv rows from the output stage to global memory
    auto flush = [&](int s) {
      constexpr int SEG = BV / 8;  // 16-byte pieces of a row
      static_assert(C * SEG % NGT == 0, "whole passes over the stage");
      const T* so = reinterpret_cast<const T*>(smem + L::off_Out + (s & 1) * L::OUT);
      const int jc = count - 1 - s;
      const int clen = min(C, dlen - jc * C);
      const int64_t row0 = (int64_t)(dstart + jc * C) * H + h;
#pragma unroll
      for (int it = 0; it < C * SEG / NGT; ++it) {
        const int i = lt + it * NGT;
        const int r = i / SEG, sg = i % SEG;
        if (r < clen) {
          const uint4 x = *reinterpret_cast<const uint4*>(so + r * L::LDV + 8 * sg);
          store16_nt(static_cast<T*>(p.dv_handoff ? p.dv : p.du) + (row0 + (int64_t)r * H) * D + v0 + 8 * sg, x);
        }
      }
    };
    if (lgroup < count) load(lgroup);
    if (lgroup == 0 && count > 0) {
      stash(0);
      if (count > 2) load(2);
    }
    for (int s = 0; s < count; ++s) {
      __syncthreads();
      if (((s + 1) & 1) == lgroup) {
        if (s + 1 < count) {
          stash((s + 1) & 1);
          if (s + 3 < count) load(s + 3);
        }
      } else if constexpr (L::STAGE_OUT) {
        if (s > 0) flush(s - 1);
      }
    }
    if constexpr (L::STAGE_OUT) {
      __syncthreads();  // the last visit's outputs
      if ((count & 1) == lgroup && count > 0) flush(count - 1);
    }
    return;
  }

  const int q4 = 4 * (lane >> 4), il = lane & 15;
  const int col0 = v0 + 16 * wave;
  f32x4 dS[NKT];
#pragma unroll
  for (int rt = 0; rt < NKT; ++rt)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      dS[rt][j] = p.dht ? p.dht[(((int64_t)n * H + h) * D + 16 * rt + q4 + j) * D + col0 + il] : 0.f;
  const float scale = p.scale;

  for (int s = 0; s < count; ++s) {
    __syncthreads();
    const int jc = count - 1 - s;
    const char* buf = smem + (s & 1) * L::BUF;
    const T* sQ = reinterpret_cast<const T*>(buf + L::off_Q);
    const T* sKW = reinterpret_cast<const T*>(buf + L::off_KW);
    const T* sK = ALIAS ? sKW : reinterpret_cast<const T*>(buf + L::off_K);
    const T* sA = reinterpret_cast<const T*>(buf + L::off_A);
    const T* sT = reinterpret_cast<const T*>(buf + L::off_T);
    const T* sdO = reinterpret_cast<const T*>(buf + L::off_dO);
    const float* sG = reinterpret_cast<const float*>(buf + L::off_G);
    const float* sB = reinterpret_cast<const float*>(buf + L::off_B);
    const int cid = first + jc;
    const int clen = min(C, dlen - jc * C);
    const int64_t row0 = (int64_t)(dstart + jc * C) * H + h;

    // dS_C as bf16 B operands; checkpoint it (tile-major)
    s16x8_t dSB[NKT / 2];
#pragma unroll
    for (int kk = 0; kk < NKT / 2; ++kk) dSB[kk] = pack_acc_pair(dS[2 * kk], dS[2 * kk + 1]);
    {
      T* hb = static_cast<T*>(p.dh) + ((int64_t)cid * H + h) * D * D;
#pragma unroll
      for (int kk = 0; kk < NKT / 2; ++kk) {
        const uint4 w = __builtin_bit_cast(uint4, dSB[kk]);
        store_packed_tile_nt(hb + tile_offset(D, 2 * kk, col0 / 16), w.x, w.y, lane);
        store_packed_tile_nt(hb + tile_offset(D, 2 * kk + 1, col0 / 16), w.z, w.w, lane);
      }
    }
    // KW dS (eight independent accumulators per k step)
    f32x4 KS[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) KS[rb] = zero4();
#pragma unroll
    for (int kk = 0; kk < NKT / 2; ++kk) {
      s16x8_t ak[4];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) ak[rb] = lds_a_perm(sKW + 16 * rb * L::LD, L::LD, 32 * kk, lane);
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) mfma_bf16(KS[rb], ak[rb], dSB[kk]);
    }
    // dO of this wave's columns as B operands over the tokens
    const s16x8_t dOB[2] = {lds_kmajor_perm(sdO + 16 * wave, L::LDV, 0, lane),
                            lds_kmajor_perm(sdO + 16 * wave, L::LDV, 32, lane)};
    // dU = Aqk^T dO + diag(e^{G_C - G}) KW dS   (Aqk^T row block rb needs k steps kt >= rb / 2)
    const float gC = sG[C - 1];
    f32x4 dU[4];
    {
      s16x8_t aa[6];
      aa[0] = lds_kmajor_perm(sA + 0, L::LDC, 0, lane);
      aa[1] = lds_kmajor_perm(sA + 0, L::LDC, 32, lane);
      aa[2] = lds_kmajor_perm(sA + 16, L::LDC, 0, lane);
      aa[3] = lds_kmajor_perm(sA + 16, L::LDC, 32, lane);
      aa[4] = lds_kmajor_perm(sA + 32, L::LDC, 32, lane);
      aa[5] = lds_kmajor_perm(sA + 48, L::LDC, 32, lane);
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) dU[rb] = zero4();
      mfma_bf16(dU[0], aa[0], dOB[0]);
      mfma_bf16(dU[1], aa[2], dOB[0]);
      mfma_bf16(dU[0], aa[1], dOB[1]);
      mfma_bf16(dU[1], aa[3], dOB[1]);
      mfma_bf16(dU[2], aa[4], dOB[1]);
      mfma_bf16(dU[3], aa[5], dOB[1]);
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int j = 0; j < 4; ++j) dU[rb][j] += exp_fast(gC - sG[16 * rb + q4 + j]) * KS[rb][j];
    // Z = T^T (-dU)   (T^T is upper triangular: row block rb needs k steps kt >= rb / 2)
    s16x8_t dOgB[2], dUnB[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      float f[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = scale * exp_fast(sG[32 * kt + (e < 4 ? 0 : 16) + q4 + (e & 3)]);
      dOgB[kt] = scale_frag(dOB[kt], f);
      dUnB[kt] = pack_acc_pair(-dU[2 * kt], -dU[2 * kt + 1]);
    }
    f32x4 Z[4];
    {
      s16x8_t at[6];
      at[0] = lds_kmajor_perm(sT + 0, L::LDC, 0, lane);
      at[1] = lds_kmajor_perm(sT + 0, L::LDC, 32, lane);
      at[2] = lds_kmajor_perm(sT + 16, L::LDC, 0, lane);
      at[3] = lds_kmajor_perm(sT + 16, L::LDC, 32, lane);
      at[4] = lds_kmajor_perm(sT + 32, L::LDC, 32, lane);
      at[5] = lds_kmajor_perm(sT + 48, L::LDC, 32, lane);
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) Z[rb] = zero4();
      mfma_bf16(Z[0], at[0], dUnB[0]);
      mfma_bf16(Z[1], at[2], dUnB[0]);
      mfma_bf16(Z[0], at[1], dUnB[1]);
      mfma_bf16(Z[1], at[3], dUnB[1]);
      mfma_bf16(Z[2], at[4], dUnB[1]);
      mfma_bf16(Z[3], at[5], dUnB[1]);
    }
    // the per-chunk kernel needs dU only through dBv = T^T dU = -Z: hand it
    // that, or (dv_handoff) dv = beta dBv with dBv itself for the rows whose
    // beta is too small to divide by
    {
      f32x4 hz[4];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) hz[rb] = -Z[rb];
      if (p.dv_handoff) {
        // one test per chunk (lane r looks at row r; the ballot is uniform):
        // rows whose beta is too small to divide by also leave dBv itself
        const float bl = sB[lane];
        if (__builtin_expect(__ballot(lane < clen && !(fabsf(bl) >= 1e-20f)) != 0, 0)) {
          T* du_out = static_cast<T*>(p.du) + row0 * D + col0;
#pragma unroll
          for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int r = 16 * rb + q4 + j;
              if (r < clen && !(fabsf(sB[r]) >= 1e-20f)) du_out[(int64_t)r * gs + il] = to_e<T>(hz[rb][j]);
            }
        }
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
          float b4[4];
          lds4(sB + 16 * rb + q4, b4);
#pragma unroll
          for (int j = 0; j < 4; ++j) hz[rb][j] *= b4[j];
        }
      }
      if constexpr (L::STAGE_OUT) {
        T* so = reinterpret_cast<T*>(smem + L::off_Out + (s & 1) * L::OUT) + 16 * wave;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) store_acc_global<T, true>(so, L::LDV, hz[rb], 16 * rb, 0, C, lane);
      } else {
        T* du_out = static_cast<T*>(p.dv_handoff ? p.dv : p.du) + row0 * D + col0;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) store_acc_global<T>(du_out, gs, hz[rb], 16 * rb, 0, clen, lane);
      }
    }
    // dS <- e^{G_C} dS + Q^T (s e^G dO) + K^T diag(beta e^G) Z
    s16x8_t ZB[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      float fa[4], fb[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int ra = 32 * kt + q4 + j, rb = ra + 16;
        fa[j] = sB[ra] * exp_fast(sG[ra]);
        fb[j] = sB[rb] * exp_fast(sG[rb]);
      }
      ZB[kt] = pack_acc_pair_scaled(Z[2 * kt], fa, Z[2 * kt + 1], fb);
    }
    const float decay = exp_fast(gC);
#pragma unroll
    for (int rt = 0; rt < NKT; ++rt) dS[rt] = dS[rt] * decay;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      s16x8_t aq[NKT], ak[NKT];
#pragma unroll
      for (int rt = 0; rt < NKT; ++rt) {
        aq[rt] = lds_kmajor_perm(sQ + 16 * rt, L::LD, 32 * kt, lane);
        ak[rt] = lds_kmajor_perm(sK + 16 * rt, L::LD, 32 * kt, lane);
      }
#pragma unroll
      for (int rt = 0; rt < NKT; ++rt) {
        mfma_bf16(dS[rt], aq[rt], dOgB[kt]);
        mfma_bf16(dS[rt], ak[rt], ZB[kt]);
      }
    }
  }
  if constexpr (L::STAGE_OUT) __syncthreads();  // the loaders' flush of the last visit
  if (p.dh0) {
    float* db = p.dh0 + ((int64_t)n * H + h) * D * D + col0;
#pragma unroll
    for (int rt = 0; rt < NKT; ++rt) store_acc_global<float>(db, D, dS[rt], 16 * rt, 0, D, lane);
  }
}

template <int D, int BV, bool ALIAS, bool PACK = false>
int launch_state_bwd_rr_as(const BwdParams& p, hipStream_t s) {
  auto kern = chunk_state_bwd_rr_kernel<D, BV, ALIAS, PACK>;
  constexpr int bytes = RrBwdLayout<D, BV, ALIAS>::bytes;
  if (int st = set_smem(kern, bytes)) return st;
  hipLaunchKernelGGL(kern, doc_grid(p.geom.num_seqs, p.H, D / BV), dim3(64 * (BV / 16 + kRrLoadersBwd)), bytes, s, p);
  return launch_status("pkda_chunk_bwd(state)");
}

// Register-resident reverse pass: 64 value columns per workgroup, or 32 when
// that leaves fewer workgroups than compute units.
template <int D>
int launch_state_bwd_rr(const BwdParams& p, hipStream_t s) {
  const int N = p.geom.num_seqs;
  if (N <= 0) return 0;
  const bool narrow = (int64_t)N * p.H * (D / 64) < 256;
  if (p.tri_packed) {  // kw = k (checked at the entry point)
    return narrow ? launch_state_bwd_rr_as<D, 32, true, true>(p, s) : launch_state_bwd_rr_as<D, 64, true, true>(p, s);
  }
  if (narrow) return p.kw_is_k ? launch_state_bwd_rr_as<D, 32, true>(p, s) : launch_state_bwd_rr_as<D, 32, false>(p, s);
  return p.kw_is_k ? launch_state_bwd_rr_as<D, 64, true>(p, s) : launch_state_bwd_rr_as<D, 64, false>(p, s);
}

// ---------------------------------------------------------------------------
// reverse state pass, BF16 with a per-channel gate: register-resident form.
// The structure of chunk_state_bwd_rr_kernel with W, qg and kg as inputs:
//   dU = Aqk^T dO + kg dS_C            (written for the per-chunk kernel)
//   dS <- diag(e^{G_C}) dS + qg^T dO - W^T dU.
// Loader waves stage qg, kg, W, Aqk, the dO slice and e^{G_C}; the compute
// waves leave dU in a double-buffered LDS output stage that the loader group
// not staging inputs writes out.
// ---------------------------------------------------------------------------
template <int D, int BV>
struct RrPcBwdLayout {
  static constexpr int LD = D + Pad<bf16_t>::v;
  static constexpr int LDV = BV + Pad<bf16_t>::v;
  static constexpr int LDC = C + Pad<bf16_t>::v;
  static constexpr int off_Q = 0;                     // qg
  static constexpr int off_KG = off_Q + C * LD * 2;   // kg
  static constexpr int off_W = off_KG + C * LD * 2;
  static constexpr int off_A = off_W + C * LD * 2;    // Aqk
  static constexpr int off_dO = off_A + C * LDC * 2;  // the dO slice
  static constexpr int off_E = off_dO + C * LDV * 2;  // [D] e^{G_C}
  static constexpr int BUF = off_E + D * 4;
  static constexpr int OUT = C * LDV * 2;             // dU rows
  static constexpr bool STAGE_OUT = 2 * BUF + 2 * OUT <= 160 * 1024;
  static constexpr int off_Out = 2 * BUF;
  static constexpr int bytes = 2 * BUF + (STAGE_OUT ? 2 * OUT : 0);
  static_assert(BUF % 16 == 0 && (LDV * 2) % 16 == 0, "16-byte aligned stages and rows");
  static_assert(bytes <= 160 * 1024, "LDS of one compute unit");
};

template <int D, int BV>
__global__ __launch_bounds__(64 * (BV / 16 + kRrLoadersBwd)) void chunk_state_bwd_rr_pc_kernel(BwdParams p) {
  using L = RrPcBwdLayout<D, BV>;
  using T = bf16_t;
  constexpr int NC = BV / 16;
  constexpr int NKT = D / 16;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const DocSlot ds = doc_slot(p.geom, p.H, D / BV);
  const int n = ds.n, h = ds.h, v0 = ds.z * BV;
  const int H = p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t gs = (int64_t)H * D;
  int first, count, dstart, dlen;
  doc_chunks(p.geom, n, first, count, dstart, dlen);
  const bool loader = wave >= NC;

  // chunks are visited in the order s = 0, 1, ... as jc = count - 1 - s
  if (loader) {
    constexpr int NGT = 64 * kRrLoadersBwd / 2;
    static_assert(D <= NGT, "one loader thread per gate channel");
    const int lgroup = (tid - 64 * NC) / NGT;  // takes visits s with s % 2 == lgroup
    const int lt = (tid - 64 * NC) % NGT;
    RegTile<NGT, C, D, T> rQ, rK, rW;
    RegTile<NGT, C, C, T> rA;
    RegTile<NGT, C, BV, T> rdO;
    float re = 0.f;
    auto load = [&](int s) {
      const int jc = count - 1 - s;
      const int cstart = dstart + jc * C;
      const int clen = min(C, dlen - jc * C);
      const int64_t row0 = (int64_t)cstart * H + h;
      rQ.load_as(lt, static_cast<const T*>(p.qg) + row0 * D, gs, clen);
      rK.load_as(lt, static_cast<const T*>(p.kg) + row0 * D, gs, clen);
      rW.load_as(lt, static_cast<const T*>(p.w) + row0 * D, gs, clen);
      rA.load_as(lt, static_cast<const T*>(p.aqk) + row0 * C, (int64_t)H * C, clen);
      rdO.load_as(lt, static_cast<const T*>(p.dO) + row0 * D + v0, gs, clen);
      if (lt < D) re = p.gcum[((int64_t)(cstart + clen - 1) * H + h) * D + lt];
    };
    auto stash = [&](int b) {
      char* buf = smem + b * L::BUF;
      rQ.store_as(lt, reinterpret_cast<T*>(buf + L::off_Q), L::LD);
      rK.store_as(lt, reinterpret_cast<T*>(buf + L::off_KG), L::LD);
      rW.store_as(lt, reinterpret_cast<T*>(buf + L::off_W), L::LD);
      rA.store_as(lt, reinterpret_cast<T*>(buf + L::off_A), L::LDC);
      rdO.store_as(lt, reinterpret_cast<T*>(buf + L::off_dO), L::LDV);
      if (lt < D) reinterpret_cast<float*>(buf + L::off_E)[lt] = exp_fast(re);
    };
    // visit s's dU rows from the output stage to global memory
    auto flush = [&](int s) {
      constexpr int SEG = BV / 8;  // 16-byte pieces of a row
      static_assert(C * SEG % NGT == 0, "whole passes over the stage");
      const T* so = reinterpret_cast<const T*>(smem + L::off_Out + (s & 1) * L::OUT);
      const int jc = count - 1 - s;
      const int clen = min(C, dlen - jc * C);
      const int64_t row0 = (int64_t)(dstart + jc * C) * H + h;
#pragma unroll
      for (int it = 0; it < C * SEG / NGT; ++it) {
        const int i = lt + it * NGT;
        const int r = i / SEG, sg = i % SEG;
        if (r < clen) {
          const uint4 x = *reinterpret_cast<const uint4*>(so + r * L::LDV + 8 * sg);
          store16_nt(static_cast<T*>(p.du) + (row0 + (int64_t)r * H) * D + v0 + 8 * sg, x);
        }
      }
    };
    if (lgroup < count) load(lgroup);
    if (lgroup == 0 && count > 0) {
      stash(0);
      if (count > 2) load(2);
    }
    for (int s = 0; s < count; ++s) {
      __syncthreads();
      if (((s + 1) & 1) == lgroup) {
        if (s + 1 < count) {
          stash((s + 1) & 1);
          if (s + 3 < count) load(s + 3);
        }
      } else if constexpr (L::STAGE_OUT) {
        if (s > 0) flush(s - 1);
      }
    }
    if constexpr (L::STAGE_OUT) {
      __syncthreads();  // the last visit's outputs
      if ((count & 1) == lgroup && count > 0) flush(count - 1);
    }
    return;
  }

  const int q4 = 4 * (lane >> 4), il = lane & 15;
  const int col0 = v0 + 16 * wave;
  f32x4 dS[NKT];
#pragma unroll
  for (int rt = 0; rt < NKT; ++rt)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      dS[rt][j] = p.dht ? p.dht[(((int64_t)n * H + h) * D + 16 * rt + q4 + j) * D + col0 + il] : 0.f;

  for (int s = 0; s < count; ++s) {
    __syncthreads();
    const int jc = count - 1 - s;
    const char* buf = smem + (s & 1) * L::BUF;
    const T* sQ = reinterpret_cast<const T*>(buf + L::off_Q);
    const T* sK = reinterpret_cast<const T*>(buf + L::off_KG);
    const T* sW = reinterpret_cast<const T*>(buf + L::off_W);
    const T* sA = reinterpret_cast<const T*>(buf + L::off_A);
    const T* sdO = reinterpret_cast<const T*>(buf + L::off_dO);
    const float* sE = reinterpret_cast<const float*>(buf + L::off_E);
    const int cid = first + jc;
    const int clen = min(C, dlen - jc * C);
    const int64_t row0 = (int64_t)(dstart + jc * C) * H + h;

    // dS_C as bf16 B operands; checkpoint it (tile-major)
    s16x8_t dSB[NKT / 2];
#pragma unroll
    for (int kk = 0; kk < NKT / 2; ++kk) dSB[kk] = pack_acc_pair(dS[2 * kk], dS[2 * kk + 1]);
    {
      T* hb = static_cast<T*>(p.dh) + ((int64_t)cid * H + h) * D * D;
#pragma unroll
      for (int kk = 0; kk < NKT / 2; ++kk) {
        const uint4 w = __builtin_bit_cast(uint4, dSB[kk]);
        store_packed_tile_nt(hb + tile_offset(D, 2 * kk, col0 / 16), w.x, w.y, lane);
        store_packed_tile_nt(hb + tile_offset(D, 2 * kk + 1, col0 / 16), w.z, w.w, lane);
      }
    }
    // kg dS (eight independent accumulators per k step)
    f32x4 dU[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) dU[rb] = zero4();
#pragma unroll
    for (int kk = 0; kk < NKT / 2; ++kk) {
      s16x8_t ak[4];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) ak[rb] = lds_a_perm(sK + 16 * rb * L::LD, L::LD, 32 * kk, lane);
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) mfma_bf16(dU[rb], ak[rb], dSB[kk]);
    }
    // dO of this wave's columns as B operands over the tokens
    const s16x8_t dOB[2] = {lds_kmajor_perm(sdO + 16 * wave, L::LDV, 0, lane),
                            lds_kmajor_perm(sdO + 16 * wave, L::LDV, 32, lane)};
    // dU += Aqk^T dO   (Aqk^T row block rb needs k steps kt >= rb / 2)
    {
      s16x8_t aa[6];
      aa[0] = lds_kmajor_perm(sA + 0, L::LDC, 0, lane);
      aa[1] = lds_kmajor_perm(sA + 0, L::LDC, 32, lane);
      aa[2] = lds_kmajor_perm(sA + 16, L::LDC, 0, lane);
      aa[3] = lds_kmajor_perm(sA + 16, L::LDC, 32, lane);
      aa[4] = lds_kmajor_perm(sA + 32, L::LDC, 32, lane);
      aa[5] = lds_kmajor_perm(sA + 48, L::LDC, 32, lane);
      mfma_bf16(dU[0], aa[0], dOB[0]);
      mfma_bf16(dU[1], aa[2], dOB[0]);
      mfma_bf16(dU[0], aa[1], dOB[1]);
      mfma_bf16(dU[1], aa[3], dOB[1]);
      mfma_bf16(dU[2], aa[4], dOB[1]);
      mfma_bf16(dU[3], aa[5], dOB[1]);
    }
    if constexpr (L::STAGE_OUT) {
      T* so = reinterpret_cast<T*>(smem + L::off_Out + (s & 1) * L::OUT) + 16 * wave;
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) store_acc_global<T, true>(so, L::LDV, dU[rb], 16 * rb, 0, C, lane);
    } else {
      T* du_out = static_cast<T*>(p.du) + row0 * D + col0;
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) store_acc_global<T>(du_out, gs, dU[rb], 16 * rb, 0, clen, lane);
    }
    // dS <- diag(e^{G_C}) dS + qg^T dO - W^T dU
    const s16x8_t dUnB[2] = {pack_acc_pair(-dU[0], -dU[1]), pack_acc_pair(-dU[2], -dU[3])};
#pragma unroll
    for (int rt = 0; rt < NKT; ++rt)
#pragma unroll
      for (int j = 0; j < 4; ++j) dS[rt][j] *= sE[16 * rt + q4 + j];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      s16x8_t aq[NKT], aw[NKT];
#pragma unroll
      for (int rt = 0; rt < NKT; ++rt) {
        aq[rt] = lds_kmajor_perm(sQ + 16 * rt, L::LD, 32 * kt, lane);
        aw[rt] = lds_kmajor_perm(sW + 16 * rt, L::LD, 32 * kt, lane);
      }
#pragma unroll
      for (int rt = 0; rt < NKT; ++rt) {
        mfma_bf16(dS[rt], aq[rt], dOB[kt]);
        mfma_bf16(dS[rt], aw[rt], dUnB[kt]);
      }
    }
  }
  if constexpr (L::STAGE_OUT) __syncthreads();  // the loaders' flush of the last visit
  if (p.dh0) {
    float* db = p.dh0 + ((int64_t)n * H + h) * D * D + col0;
#pragma unroll
    for (int rt = 0; rt < NKT; ++rt) store_acc_global<float>(db, D, dS[rt], 16 * rt, 0, D, lane);
  }
}

template <int D, int BV>
int launch_state_bwd_rr_pc_as(const BwdParams& p, hipStream_t s) {
  auto kern = chunk_state_bwd_rr_pc_kernel<D, BV>;
  constexpr int bytes = RrPcBwdLayout<D, BV>::bytes;
  if (int st = set_smem(kern, bytes)) return st;
  hipLaunchKernelGGL(kern, doc_grid(p.geom.num_seqs, p.H, D / BV), dim3(64 * (BV / 16 + kRrLoadersBwd)), bytes, s, p);
  return launch_status("pkda_chunk_bwd(state)");
}

template <int D>
int launch_state_bwd_rr_pc(const BwdParams& p, hipStream_t s) {
  const int N = p.geom.num_seqs;
  if (N <= 0) return 0;
  const bool narrow = (int64_t)N * p.H * (D / 64) < 256;
  return narrow ? launch_state_bwd_rr_pc_as<D, 32>(p, s) : launch_state_bwd_rr_pc_as<D, 64>(p, s);
}

template <typename T, int D, int BV, typename OT, typename OK>
int launch_bwd(const BwdParams& p_in, int num_chunks, int stages, hipStream_t s) {
  BwdParams p = p_in;
  // the four-wave per-chunk kernel runs: the reverse pass hands it dv
  p.dv_handoff = implicit_w<T>() && std::is_same<OT, bf16_t>::value && std::is_same<OK, bf16_t>::value && !p.qg &&
                 p.kw_is_k;
  const int N = p.geom.num_seqs;
  const bool all = stages == 0;
  if (all || (stages & PKDA_STAGE_BWD_STATE)) {
    bool done = false;
    if constexpr (std::is_same<T, bf16_t>::value) {
      if (!p.qg) {  // BF16, per-head gate: the register-resident pass
        if (int st = launch_state_bwd_rr<D>(p, s)) return st;
      } else {      // BF16, per-channel gate: its register-resident pass
        if (int st = launch_state_bwd_rr_pc<D>(p, s)) return st;
      }
      done = true;
    }
    if (!done) {
      auto kern = p.qg ? chunk_state_bwd_kernel<T, D, BV, true> : chunk_state_bwd_kernel<T, D, BV, false>;
      const int bytes = StateBwdLayout<T, D, BV>::bytes;
      if (int st = set_smem(kern, bytes)) return st;
      if (N > 0) hipLaunchKernelGGL(kern, doc_grid(N, p.H, D / BV), dim3(state_threads(D, BV)), bytes, s, p);
      if (int st = launch_status("pkda_chunk_bwd(state)")) return st;
    }
  }
  if (num_chunks == 0) return 0;
  if (all || (stages & PKDA_STAGE_BWD_CHUNK)) {
    if constexpr (implicit_w<T>() && std::is_same<OT, bf16_t>::value && std::is_same<OK, bf16_t>::value) {
      if (!p.qg && p.kw_is_k) {  // BF16, per-head gate, kw = k: the four-wave form
        auto kern = chunk_fused_bwd_w4_kernel<D>;
        constexpr int bytes = FusedW4Layout<D>::bytes;
        if (int st = set_smem(kern, bytes)) return st;
        hipLaunchKernelGGL(kern, dim3(chunk_grid<true>(num_chunks, p.H)), dim3(kW4), bytes, s, p);
        return launch_status("pkda_chunk_bwd(chunk)");
      }
    }
    auto kern = p.qg ? chunk_fused_bwd_pc_kernel<T, D, OT, OK>
                     : (p.kw_is_k ? chunk_fused_bwd_kernel<T, D, OT, OK, true>
                                  : chunk_fused_bwd_kernel<T, D, OT, OK, false>);
    const int bytes = p.qg ? FusedBwdPcLayout<T, D>::bytes : FusedBwdLayout<T, D>::bytes;
    if (int st = set_smem(kern, bytes)) return st;
    hipLaunchKernelGGL(kern, p.qg ? dim3(chunk_grid<false>(num_chunks, p.H)) : dim3(chunk_grid<true>(num_chunks, p.H)), dim3(kFW), bytes, s, p);
    if (int st = launch_status("pkda_chunk_bwd(chunk)")) return st;
  }
  return 0;
}

}  // namespace
}  // namespace pkda

using namespace pkda;

extern "C" int pkda_chunk_bwd(const pkda_chunk_bwd_args* a, void* stream) {
  PKDA_REQUIRE(a != nullptr, PKDA_EINVAL, "null args");
  PKDA_REQUIRE(a->struct_size == (int32_t)sizeof(pkda_chunk_bwd_args), PKDA_EINVAL, "pkda_chunk_bwd_args size mismatch");
  PKDA_REQUIRE(a->dtype == PKDA_F32 || a->dtype == PKDA_BF16, PKDA_EUNSUPPORTED, "dtype %d", a->dtype);
  PKDA_REQUIRE(a->head_dim == 64 || a->head_dim == 128, PKDA_EUNSUPPORTED, "chunked head_dim %d (64, 128)", a->head_dim);
  PKDA_REQUIRE(!(a->dtype == PKDA_F32 && a->head_dim == 128), PKDA_EUNSUPPORTED,
               "the FP32 chunked backward is built for head_dim 64 only");
  PKDA_REQUIRE(a->heads > 0, PKDA_EINVAL, "heads");
  PKDA_REQUIRE(!a->gate_per_channel || (a->qg && a->kg), PKDA_EINVAL, "per-channel gates need the forward's qg and kg");
  PKDA_REQUIRE(a->grad_dtype == PKDA_F32 || a->grad_dtype == a->dtype, PKDA_EUNSUPPORTED,
               "grad_dtype %d (FP32 or the activation dtype)", a->grad_dtype);
  PKDA_REQUIRE(a->key_grad_dtype == a->grad_dtype || (a->key_grad_dtype == PKDA_F32 && a->grad_dtype == a->dtype),
               PKDA_EUNSUPPORTED, "key_grad_dtype %d with grad_dtype %d (equal, or FP32 key gradients)",
               a->key_grad_dtype, a->grad_dtype);
  BwdParams p;
  if (int st = chunk_geom_from(a->cu_seqlens, a->num_seqs, a->seqlen, a->num_chunks, a->table, p.geom)) return st;
  if (a->num_seqs == 0) return 0;
  PKDA_REQUIRE(a->q && a->k && a->v && a->gcum && a->beta && a->u && a->aqk && a->akk && a->h && a->do_ &&
                   a->dh && a->du && a->dq && a->dk && a->dv && a->dbeta && a->dgcum,
               PKDA_EINVAL, "null tensor");
  PKDA_REQUIRE(a->w || (a->dtype == PKDA_BF16 && !a->gate_per_channel), PKDA_EINVAL,
               "this dtype / gate needs the forward's w");
  const bool kw_is_k = a->kw == nullptr || a->kw == a->k;
  PKDA_REQUIRE(kw_is_k || a->dkw, PKDA_EINVAL, "a separate write key needs dkw");
  const int st = a->stages;
  PKDA_REQUIRE(st >= 0 && st <= (PKDA_STAGE_BWD_STATE | PKDA_STAGE_BWD_CHUNK), PKDA_EINVAL, "stages %d", st);
  p.H = a->heads;
  p.q = a->q; p.k = a->k; p.kw = kw_is_k ? a->k : a->kw; p.v = a->v;
  p.gcum = a->gcum; p.beta = a->beta; p.scale = a->scale;
  p.gcum_lo = a->gate_per_channel && a->dtype == PKDA_F32 ? a->gcum_lo : nullptr;
  p.w = a->w; p.u = a->u; p.aqk = a->aqk; p.akk = a->akk; p.h = a->h;
  p.dO = a->do_; p.dht = a->dht; p.dh = a->dh; p.du = a->du;
  p.dq = a->dq; p.dk = a->dk; p.dkw = a->dkw; p.dv = a->dv; p.dbeta = a->dbeta; p.dgcum = a->dgcum; p.dh0 = a->dh0;
  p.kw_is_k = kw_is_k;
  p.qg = a->gate_per_channel ? a->qg : nullptr;
  p.kg = a->gate_per_channel ? a->kg : nullptr;
  p.kw32 = a->gate_per_channel && !kw_is_k && a->dtype == PKDA_BF16 ? a->kw32 : nullptr;
  p.tri_packed = a->tri_packed != 0;
  PKDA_REQUIRE(!p.tri_packed || (a->dtype == PKDA_BF16 && !a->gate_per_channel && kw_is_k), PKDA_EUNSUPPORTED,
               "packed aqk / akk (tri_packed) are built for BF16 with a per-head gate and kw == k");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nc = a->num_chunks;
  if (a->dtype == PKDA_BF16) {
    if (a->grad_dtype == PKDA_BF16 && a->key_grad_dtype == PKDA_BF16) {
      return a->head_dim == 128 ? launch_bwd<bf16_t, 128, 64, bf16_t, bf16_t>(p, nc, st, s)
                                : launch_bwd<bf16_t, 64, 64, bf16_t, bf16_t>(p, nc, st, s);
    }
    if (a->grad_dtype == PKDA_BF16) {
      return a->head_dim == 128 ? launch_bwd<bf16_t, 128, 64, bf16_t, float>(p, nc, st, s)
                                : launch_bwd<bf16_t, 64, 64, bf16_t, float>(p, nc, st, s);
    }
    return a->head_dim == 128 ? launch_bwd<bf16_t, 128, 64, float, float>(p, nc, st, s)
                              : launch_bwd<bf16_t, 64, 64, float, float>(p, nc, st, s);
  }
  return launch_bwd<float, 64, 64, float, float>(p, nc, st, s);
}
