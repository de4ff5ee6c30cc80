// Chunked PKDA backward for gfx950 (per-head gate).
//
// With the forward's chunk quantities (T = (I+Akk)^-1, W, U, Aqk, the
// entering state S0 = h of every chunk) and the upstream dO, the backward of
// one chunk, given the gradient dS_C of the state leaving it, is
//
//   dU   = Aqk^T dO + Kg dS_C                    (Kg = diag(e^{G_C-G}) KW)
//   dS0  = e^{G_C} dS_C + Qg^T dO - W^T dU        (Qg = diag(scale e^G) Q)
//   dQg  = dO S0^T,  dW = -dU S0^T,  dKg = U dS_C^T,  dAqk = dO U^T
//   dBw  = T^T dW,   dBv = T^T dU                (Bw = diag(beta e^G) K, Bv = diag(beta) V)
//   dT   = dW Bw^T + dU Bv^T,   dAkk = -T^T dT T^T   (strictly lower part)
//
// and the pairwise terms Akk[t,s] = beta_t E_ts (k_t . kw_s),
// Aqk[t,s] = scale E_ts (q_t . kw_s), E_ts = e^{G_t - G_s}, give the rest of
// dq, dk (read key), dkw (write key), dbeta and the gradient of the
// chunk-local cumulative gate.  Four kernels:
//   state_bwd  -- per (document, head, BV columns), reverse over chunks:
//                 dS carried in MFMA accumulators; writes dh (= dS_C per
//                 chunk), dU, and dS0 of the first chunk.
//   dqkw       -- per (chunk, head): dQg, dW, dKg, dAqk and their gate terms.
//   wy_bwd     -- per (chunk, head): dBw, dBv, dT, dAkk.
//   intra_bwd  -- per (chunk, head): pairwise terms; final dq, dk, dkw.
// Every reduction has a fixed order: results are bitwise reproducible.
#include "pkda_chunk_common.h"

namespace pkda {
namespace {

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
  const void* u;
  const void* aqk;
  const void* akk;
  const void* h;
  const void* dO;
  const float* dht;
  void* dh;
  float* du;
  float* dw;
  float* daqk;
  float* da;
  float* dq;
  float* dk;
  float* dkw;
  float* dv;
  float* dbeta;
  float* dgcum;
  float* dh0;
  bool kw_is_k;
};

__device__ __forceinline__ void load_gam(float* s_gam, const float* gcum, int start, int len, int H, int h) {
  const int t = threadIdx.x;
  if (t < C) {
    const int tt = t < len ? t : len - 1;
    s_gam[t] = gcum[(int64_t)(start + tt) * H + h];
  }
}

__device__ __forceinline__ void load_beta(float* s_beta, const float* beta, int start, int len, int H, int h) {
  const int t = threadIdx.x;
  if (t < C) s_beta[t] = t < len ? beta[(int64_t)(start + t) * H + h] : 0.f;
}

// Sum over the 16 lanes of a lane group (same lane >> 4), fixed order.
__device__ __forceinline__ float group16_sum(float x) {
  x += __shfl_xor(x, 1);
  x += __shfl_xor(x, 2);
  x += __shfl_xor(x, 4);
  x += __shfl_xor(x, 8);
  return x;
}

// Deterministic sum of one value per thread over the workgroup.
__device__ __forceinline__ float block_sum(float x, float* s_red) {
  s_red[threadIdx.x] = x;
  __syncthreads();
  for (int off = kWG / 2; off > 0; off >>= 1) {
    if (threadIdx.x < off) s_red[threadIdx.x] += s_red[threadIdx.x + off];
    __syncthreads();
  }
  const float r = s_red[0];
  __syncthreads();
  return r;
}

// ---------------------------------------------------------------------------
// reverse state pass
// ---------------------------------------------------------------------------
template <typename T, int D, int BV>
struct StateBwdLayout {
  static constexpr int LD = D + Pad<T>::v;
  static constexpr int LDC = C + Pad<T>::v;
  static constexpr int off_dST = 0;                                        // [BV][LD]  dS^T
  static constexpr int off_Kg = off_dST + BV * LD * (int)sizeof(T);        // [64][LD]
  static constexpr int off_AqkT = off_Kg + C * LD * (int)sizeof(T);        // [64][LDC]
  static constexpr int off_dOT = off_AqkT + C * LDC * (int)sizeof(T);      // [BV][LDC]
  static constexpr int off_dUT = off_dOT + BV * LDC * (int)sizeof(T);      // [BV][LDC]
  static constexpr int off_QgT = off_dUT + BV * LDC * (int)sizeof(T);      // [D][LDC]
  static constexpr int off_WT = off_QgT + D * LDC * (int)sizeof(T);        // [D][LDC] (negated)
  static constexpr int off_gam = off_WT + D * LDC * (int)sizeof(T);
  static constexpr int bytes = off_gam + C * 4;
};

template <typename T, int D, int BV>
__global__ __launch_bounds__(kWG) void chunk_state_bwd_kernel(BwdParams p) {
  using L = StateBwdLayout<T, D, BV>;
  using E = T;
  constexpr int NCT = BV / 16;
  constexpr int NS = (D / 16) * NCT / 4;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  E* sdST = reinterpret_cast<E*>(smem + L::off_dST);
  E* sKg = reinterpret_cast<E*>(smem + L::off_Kg);
  E* sAqkT = reinterpret_cast<E*>(smem + L::off_AqkT);
  E* sdOT = reinterpret_cast<E*>(smem + L::off_dOT);
  E* sdUT = reinterpret_cast<E*>(smem + L::off_dUT);
  E* sQgT = reinterpret_cast<E*>(smem + L::off_QgT);
  E* sWT = reinterpret_cast<E*>(smem + L::off_WT);
  float* sGam = reinterpret_cast<float*>(smem + L::off_gam);

  const int n = blockIdx.x, h = blockIdx.y, v0 = blockIdx.z * BV;
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
  const float scale = p.scale;
  for (int jc = count - 1; jc >= 0; --jc) {
    const int cid = first + jc;
    const int cstart = dstart + jc * C;
    const int clen = min(C, dlen - jc * C);
    const int64_t row0 = (int64_t)cstart * H + h;
    // (a) checkpoint dS_C, publish it as the B operand
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int ti = wave * NS + i;
      const int rt = ti / NCT, ct = ti % NCT;
      store_acc_lds_t(sdST, L::LD, dS[i], 16 * rt, 16 * ct, lane);
      T* hb = static_cast<T*>(p.dh) + ((int64_t)cid * H + h) * D * D + v0;
      store_acc_global<T>(hb, D, dS[i], 16 * rt, 16 * ct, D, lane);
    }
    load_gam(sGam, p.gcum, cstart, clen, H, h);
    __syncthreads();
    const float gC = sGam[C - 1];
    load_rows<T, E, D>(sKg, L::LD, static_cast<const T*>(p.kw) + row0 * D, gs, C, clen,
                       [&](int r, int, float x) { return expf(gC - sGam[r]) * x; });
    load_rows_t<T, E, C>(sAqkT, L::LDC, static_cast<const T*>(p.aqk) + row0 * C, (int64_t)H * C, C, clen, Ident());
    load_rows_t<T, E, BV>(sdOT, L::LDC, static_cast<const T*>(p.dO) + row0 * D + v0, gs, C, clen, Ident());
    load_rows_t<T, E, D>(sQgT, L::LDC, static_cast<const T*>(p.q) + row0 * D, gs, C, clen,
                         [&](int r, int, float x) { return scale * expf(sGam[r]) * x; });
    load_rows_t<T, E, D>(sWT, L::LDC, static_cast<const T*>(p.w) + row0 * D, gs, C, clen,
                         [&](int, int, float x) { return -x; });
    __syncthreads();
    // (b) dU = Aqk^T dO + Kg dS_C     wave w: row tile w
    float* du_out = p.du + row0 * D + v0;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      f32x4 acc = zero4();
      mma_tile<E, ROW, COL>(acc, sAqkT, L::LDC, 16 * wave, sdOT, L::LDC, 16 * ct, C, lane);
      mma_tile<E, ROW, COL>(acc, sKg, L::LD, 16 * wave, sdST, L::LD, 16 * ct, D, lane);
      store_acc_global<float>(du_out, gs, acc, 16 * wave, 16 * ct, clen, lane);
      store_acc_lds_t(sdUT, L::LDC, acc, 16 * wave, 16 * ct, lane);
    }
    __syncthreads();
    // (c) dS <- e^{G_C} dS + Qg^T dO - W^T dU
    const float decay = expf(gC);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int ti = wave * NS + i;
      const int rt = ti / NCT, ct = ti % NCT;
      dS[i] = dS[i] * decay;
      mma_tile<E, ROW, COL>(dS[i], sQgT, L::LDC, 16 * rt, sdOT, L::LDC, 16 * ct, C, lane);
      mma_tile<E, ROW, COL>(dS[i], sWT, L::LDC, 16 * rt, sdUT, L::LDC, 16 * ct, C, lane);
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
// dQg, dW, dKg, dAqk per chunk
// ---------------------------------------------------------------------------
template <typename T, int D>
struct DqkwLayout {
  static constexpr int LD = D + Pad<T>::v;
  static constexpr int off_dO = 0;
  static constexpr int off_dU = off_dO + C * LD * (int)sizeof(T);
  static constexpr int off_U = off_dU + C * LD * (int)sizeof(T);
  static constexpr int off_H = off_U + C * LD * (int)sizeof(T);    // [D][LD] h, then dh
  static constexpr int off_gam = off_H + D * LD * (int)sizeof(T);
  static constexpr int off_red = off_gam + C * 4;
  static constexpr int off_dg = off_red + kWG * 4;
  static constexpr int bytes = off_dg + C * 4;
};

template <typename T, int D>
__global__ __launch_bounds__(kWG) void chunk_dqkw_kernel(BwdParams p) {
  using L = DqkwLayout<T, D>;
  using E = T;
  constexpr int NCT = D / 16;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const ChunkInfo ci = chunk_info(p.geom, blockIdx.x);
  if (ci.len <= 0) return;
  const int cid = blockIdx.x;
  const int h = blockIdx.y;
  const int H = p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t gs = (int64_t)H * D;
  const int64_t row0 = (int64_t)ci.start * H + h;
  E* sdO = reinterpret_cast<E*>(smem + L::off_dO);
  E* sdU = reinterpret_cast<E*>(smem + L::off_dU);
  E* sU = reinterpret_cast<E*>(smem + L::off_U);
  E* sH = reinterpret_cast<E*>(smem + L::off_H);
  float* sGam = reinterpret_cast<float*>(smem + L::off_gam);
  float* sRed = reinterpret_cast<float*>(smem + L::off_red);
  float* sDg = reinterpret_cast<float*>(smem + L::off_dg);
  const T* hsrc = static_cast<const T*>(p.h) + ((int64_t)cid * H + h) * D * D;
  const T* dhsrc = static_cast<const T*>(p.dh) + ((int64_t)cid * H + h) * D * D;

  load_gam(sGam, p.gcum, ci.start, ci.len, H, h);
  load_rows<T, E, D>(sdO, L::LD, static_cast<const T*>(p.dO) + row0 * D, gs, C, ci.len, Ident());
  load_rows<float, E, D>(sdU, L::LD, p.du + row0 * D, gs, C, ci.len, Ident());
  load_rows<T, E, D>(sU, L::LD, static_cast<const T*>(p.u) + row0 * D, gs, C, ci.len, Ident());
  load_rows<T, E, D>(sH, L::LD, hsrc, D, D, D, Ident());
  // e^{G_C} sum(dh * h): the decay term of the gate at the chunk's last row
  float hd = 0.f;
  for (int i = tid; i < D * D; i += kWG) hd += from_e<T>(hsrc[i]) * from_e<T>(dhsrc[i]);
  __syncthreads();
  const float gC = sGam[C - 1];
  const float hd_sum = block_sum(hd, sRed);

  const int t0 = 16 * wave;
  float dg_row[4] = {0.f, 0.f, 0.f, 0.f};
  // dQg = dO h^T  -> dq (partial), gate term sum_c dQg * Qg
  {
    float part[4] = {0.f, 0.f, 0.f, 0.f};
    const T* qrow = static_cast<const T*>(p.q) + row0 * D;
    float* dq = p.dq + row0 * D;
    for (int ct = 0; ct < NCT; ++ct) {
      f32x4 acc = zero4();
      mma_tile<E, ROW, COL>(acc, sdO, L::LD, t0, sH, L::LD, 16 * ct, D, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = t0 + acc_row(lane, j), c = 16 * ct + acc_col(lane);
        if (t < ci.len) {
          const float g = p.scale * expf(sGam[t]) * acc[j];
          dq[t * gs + c] = g;
          part[j] += g * io<T>::load(qrow + t * gs + c);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) dg_row[j] += group16_sum(part[j]);
  }
  // dW = -dU h^T
  {
    float* dw = p.dw + row0 * D;
    for (int ct = 0; ct < NCT; ++ct) {
      f32x4 acc = zero4();
      mma_tile<E, ROW, COL>(acc, sdU, L::LD, t0, sH, L::LD, 16 * ct, D, lane);
      store_acc_global<float>(dw, gs, -acc, t0, 16 * ct, ci.len, lane);
    }
  }
  // dAqk = dO U^T  (s <= t)
  {
    float* da = p.daqk + row0 * C;
    for (int ct = 0; ct < 4; ++ct) {
      f32x4 acc = zero4();
      if (ct <= wave) mma_tile<E, ROW, COL>(acc, sdO, L::LD, t0, sU, L::LD, 16 * ct, D, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = t0 + acc_row(lane, j), s = 16 * ct + acc_col(lane);
        if (t < ci.len) da[(int64_t)t * H * C + s] = (s <= t) ? acc[j] : 0.f;
      }
    }
  }
  __syncthreads();
  load_rows<T, E, D>(sH, L::LD, dhsrc, D, D, D, Ident());
  __syncthreads();
  // dKg = U dh^T -> dkw (partial) and gate terms
  float kg_total = 0.f;
  {
    float part[4] = {0.f, 0.f, 0.f, 0.f};
    const T* kwrow = static_cast<const T*>(p.kw) + row0 * D;
    float* dkw = (p.kw_is_k ? p.dk : p.dkw) + row0 * D;
    for (int ct = 0; ct < NCT; ++ct) {
      f32x4 acc = zero4();
      mma_tile<E, ROW, COL>(acc, sU, L::LD, t0, sH, L::LD, 16 * ct, D, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int s = t0 + acc_row(lane, j), c = 16 * ct + acc_col(lane);
        if (s < ci.len) {
          const float g = expf(gC - sGam[s]) * acc[j];
          dkw[s * gs + c] = g;
          part[j] += g * io<T>::load(kwrow + s * gs + c);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float r = group16_sum(part[j]);
      dg_row[j] -= r;
      kg_total += (lane & 15) == 0 ? r : 0.f;
    }
  }
  // rows' gate terms to LDS; the last row also collects the G_C terms
  if ((lane & 15) == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) sDg[t0 + acc_row(lane, j)] = dg_row[j];
  }
  const float kg_sum = block_sum(kg_total, sRed);
  if (tid < ci.len) {
    float g = sDg[tid];
    if (tid == ci.len - 1) g += kg_sum + expf(gC) * hd_sum;
    p.dgcum[(int64_t)(ci.start + tid) * H + h] = g;
  }
}

// ---------------------------------------------------------------------------
// WY backward: dBw, dBv -> dk (partial), dv, dbeta, gate; dT -> dAkk
// ---------------------------------------------------------------------------
template <typename T, int D>
struct WyLayout {
  static constexpr int LD = D + Pad<T>::v;
  static constexpr int LDC = C + Pad<T>::v;
  static constexpr int off_TT = 0;                                  // [64][LDC] T^T
  static constexpr int off_R = off_TT + C * LDC * (int)sizeof(T);   // phase region
  // phase 1: dW^T, dU^T [D][LDC]
  static constexpr int P1 = 2 * D * LDC * (int)sizeof(T);
  // phase 2: dW, dU, Bw, Bv [64][LD]; dT^T, X, T [64][LDC]
  static constexpr int P2 = 4 * C * LD * (int)sizeof(T) + 3 * C * LDC * (int)sizeof(T);
  static constexpr int off_beta = off_R + (P1 > P2 ? P1 : P2);
  static constexpr int off_gam = off_beta + C * 4;
  static constexpr int off_db = off_gam + C * 4;
  static constexpr int off_dg = off_db + C * 4;
  static constexpr int bytes = off_dg + C * 4;
};

template <typename T, int D>
__global__ __launch_bounds__(kWG) void chunk_wy_bwd_kernel(BwdParams p) {
  using L = WyLayout<T, D>;
  using E = T;
  constexpr int NCT = D / 16;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const ChunkInfo ci = chunk_info(p.geom, blockIdx.x);
  if (ci.len <= 0) return;
  const int h = blockIdx.y;
  const int H = p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t gs = (int64_t)H * D;
  const int64_t row0 = (int64_t)ci.start * H + h;
  E* sTT = reinterpret_cast<E*>(smem + L::off_TT);
  E* sdWT = reinterpret_cast<E*>(smem + L::off_R);
  E* sdUT = sdWT + D * L::LDC;
  float* sBeta = reinterpret_cast<float*>(smem + L::off_beta);
  float* sGam = reinterpret_cast<float*>(smem + L::off_gam);
  float* sDb = reinterpret_cast<float*>(smem + L::off_db);
  float* sDg = reinterpret_cast<float*>(smem + L::off_dg);
  const T* krow = static_cast<const T*>(p.k) + row0 * D;
  const T* vrow = static_cast<const T*>(p.v) + row0 * D;

  load_gam(sGam, p.gcum, ci.start, ci.len, H, h);
  load_beta(sBeta, p.beta, ci.start, ci.len, H, h);
  load_rows_t<T, E, C>(sTT, L::LDC, static_cast<const T*>(p.akk) + row0 * C, (int64_t)H * C, C, ci.len, Ident());
  load_rows_t<float, E, D>(sdWT, L::LDC, p.dw + row0 * D, gs, C, ci.len, Ident());
  load_rows_t<float, E, D>(sdUT, L::LDC, p.du + row0 * D, gs, C, ci.len, Ident());
  __syncthreads();
  const int s0 = 16 * wave;
  // dBw = T^T dW: dk (read key, partial) = beta e^G dBw; R1 = sum_c dBw k
  {
    float r1[4] = {0.f, 0.f, 0.f, 0.f};
    float* dk = p.dk + row0 * D;
    for (int ct = 0; ct < NCT; ++ct) {
      f32x4 acc = zero4();
      mma_tile<E, ROW, COL>(acc, sTT, L::LDC, s0, sdWT, L::LDC, 16 * ct, C, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int s = s0 + acc_row(lane, j), c = 16 * ct + acc_col(lane);
        if (s < ci.len) {
          const float x = acc[j];
          const float kv = io<T>::load(krow + s * gs + c);
          const float contrib = sBeta[s] * expf(sGam[s]) * x;
          if (p.kw_is_k) dk[s * gs + c] += contrib;  // dqkw wrote dkw here
          else dk[s * gs + c] = contrib;
          r1[j] += x * kv;
        }
      }
    }
    // dBv = T^T dU: dv = beta dBv; R2 = sum_c dBv v
    float r2[4] = {0.f, 0.f, 0.f, 0.f};
    float* dv = p.dv + row0 * D;
    for (int ct = 0; ct < NCT; ++ct) {
      f32x4 acc = zero4();
      mma_tile<E, ROW, COL>(acc, sTT, L::LDC, s0, sdUT, L::LDC, 16 * ct, C, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int s = s0 + acc_row(lane, j), c = 16 * ct + acc_col(lane);
        if (s < ci.len) {
          dv[s * gs + c] = sBeta[s] * acc[j];
          r2[j] += acc[j] * io<T>::load(vrow + s * gs + c);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = group16_sum(r1[j]);
      const float b = group16_sum(r2[j]);
      const int s = s0 + acc_row(lane, j);
      if ((lane & 15) == 0) {
        const float eg = expf(sGam[s]);
        sDb[s] = eg * a + b;
        sDg[s] = sBeta[s] * eg * a;
      }
    }
  }
  __syncthreads();
  // phase 2: dT = dW Bw^T + dU Bv^T;  X = T^T dT;  dAkk = -X T^T
  E* sdW = reinterpret_cast<E*>(smem + L::off_R);
  E* sdU = sdW + C * L::LD;
  E* sBw = sdU + C * L::LD;
  E* sBv = sBw + C * L::LD;
  E* sdTT = sBv + C * L::LD;
  E* sX = sdTT + C * L::LDC;
  E* sT = sX + C * L::LDC;
  load_rows<float, E, D>(sdW, L::LD, p.dw + row0 * D, gs, C, ci.len, Ident());
  load_rows<float, E, D>(sdU, L::LD, p.du + row0 * D, gs, C, ci.len, Ident());
  load_rows<T, E, D>(sBw, L::LD, krow, gs, C, ci.len,
                     [&](int r, int, float x) { return sBeta[r] * expf(sGam[r]) * x; });
  load_rows<T, E, D>(sBv, L::LD, vrow, gs, C, ci.len, [&](int r, int, float x) { return sBeta[r] * x; });
  load_rows<T, E, C>(sT, L::LDC, static_cast<const T*>(p.akk) + row0 * C, (int64_t)H * C, C, ci.len, Ident());
  __syncthreads();
  for (int ct = 0; ct < 4; ++ct) {
    f32x4 acc = zero4();
    mma_tile<E, ROW, COL>(acc, sdW, L::LD, s0, sBw, L::LD, 16 * ct, D, lane);
    mma_tile<E, ROW, COL>(acc, sdU, L::LD, s0, sBv, L::LD, 16 * ct, D, lane);
    store_acc_lds_t(sdTT, L::LDC, acc, s0, 16 * ct, lane);
  }
  __syncthreads();
  for (int ct = 0; ct < 4; ++ct) {
    f32x4 acc = zero4();
    mma_tile<E, ROW, COL>(acc, sTT, L::LDC, s0, sdTT, L::LDC, 16 * ct, C, lane);
    store_acc_lds(sX, L::LDC, acc, s0, 16 * ct, lane);
  }
  __syncthreads();
  float* da = p.da + row0 * C;
  for (int ct = 0; ct < 4; ++ct) {
    f32x4 acc = zero4();
    mma_tile<E, ROW, COL>(acc, sX, L::LDC, s0, sT, L::LDC, 16 * ct, C, lane);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = s0 + acc_row(lane, j), s = 16 * ct + acc_col(lane);
      if (t < ci.len) da[(int64_t)t * H * C + s] = (s < t) ? -acc[j] : 0.f;
    }
  }
  if (tid < ci.len) {
    const int64_t idx = (int64_t)(ci.start + tid) * H + h;
    p.dbeta[idx] = sDb[tid];
    p.dgcum[idx] += sDg[tid];
  }
}

// ---------------------------------------------------------------------------
// intra-chunk pairwise backward
// ---------------------------------------------------------------------------
template <typename T, int D>
struct IntraBwdLayout {
  static constexpr int LDC = C + Pad<T>::v;
  static constexpr int LDF = C + 4;
  static constexpr int off_KT = 0;                                      // [D][LDC]
  static constexpr int off_KWT = off_KT + D * LDC * (int)sizeof(T);
  static constexpr int off_QT = off_KWT + D * LDC * (int)sizeof(T);
  static constexpr int off_P1 = off_QT + D * LDC * (int)sizeof(T);      // [64][LDC] x4
  static constexpr int off_P2 = off_P1 + C * LDC * (int)sizeof(T);
  static constexpr int off_P1T = off_P2 + C * LDC * (int)sizeof(T);
  static constexpr int off_P2T = off_P1T + C * LDC * (int)sizeof(T);
  static constexpr int off_M = off_P2T + C * LDC * (int)sizeof(T);     // [64][LDF] fp32
  static constexpr int off_beta = off_M + C * LDF * 4;
  static constexpr int off_gam = off_beta + C * 4;
  static constexpr int off_db = off_gam + C * 4;
  static constexpr int bytes = off_db + C * 4;
};

template <typename T, int D>
__global__ __launch_bounds__(kWG) void chunk_intra_bwd_kernel(BwdParams p) {
  using L = IntraBwdLayout<T, D>;
  using E = T;
  constexpr int NCT = D / 16;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const ChunkInfo ci = chunk_info(p.geom, blockIdx.x);
  if (ci.len <= 0) return;
  const int h = blockIdx.y;
  const int H = p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t gs = (int64_t)H * D;
  const int64_t row0 = (int64_t)ci.start * H + h;
  E* sKT = reinterpret_cast<E*>(smem + L::off_KT);
  E* sKWT = reinterpret_cast<E*>(smem + L::off_KWT);
  E* sQT = reinterpret_cast<E*>(smem + L::off_QT);
  E* sP1 = reinterpret_cast<E*>(smem + L::off_P1);
  E* sP2 = reinterpret_cast<E*>(smem + L::off_P2);
  E* sP1T = reinterpret_cast<E*>(smem + L::off_P1T);
  E* sP2T = reinterpret_cast<E*>(smem + L::off_P2T);
  float* sM = reinterpret_cast<float*>(smem + L::off_M);
  float* sBeta = reinterpret_cast<float*>(smem + L::off_beta);
  float* sGam = reinterpret_cast<float*>(smem + L::off_gam);
  float* sDb = reinterpret_cast<float*>(smem + L::off_db);

  load_gam(sGam, p.gcum, ci.start, ci.len, H, h);
  load_beta(sBeta, p.beta, ci.start, ci.len, H, h);
  load_rows_t<T, E, D>(sKT, L::LDC, static_cast<const T*>(p.k) + row0 * D, gs, C, ci.len, Ident());
  load_rows_t<T, E, D>(sKWT, L::LDC, static_cast<const T*>(p.kw) + row0 * D, gs, C, ci.len, Ident());
  load_rows_t<T, E, D>(sQT, L::LDC, static_cast<const T*>(p.q) + row0 * D, gs, C, ci.len, Ident());
  __syncthreads();
  const int t0 = 16 * wave;
  const float* dA = p.da + row0 * C;
  const float* dAqk = p.daqk + row0 * C;
  float db[4] = {0.f, 0.f, 0.f, 0.f};
  for (int ct = 0; ct < 4; ++ct) {
    f32x4 rk = zero4(), rq = zero4();
    if (ct <= wave) {
      // raw k_t . kw_s and q_t . kw_s (A read from K^T / Q^T, B from KW^T)
      mma_tile<E, COL, ROW>(rk, sKT, L::LDC, t0, sKWT, L::LDC, 16 * ct, D, lane);
      mma_tile<E, COL, ROW>(rq, sQT, L::LDC, t0, sKWT, L::LDC, 16 * ct, D, lane);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = t0 + acc_row(lane, j), s = 16 * ct + acc_col(lane);
      float p1 = 0.f, p2 = 0.f, m = 0.f;
      if (t < ci.len && s <= t) {
        const float e = expf(sGam[t] - sGam[s]);
        const float dak = dA[(int64_t)t * H * C + s];
        const float daq = dAqk[(int64_t)t * H * C + s];
        if (s < t) {
          p1 = dak * sBeta[t] * e;
          db[j] += dak * e * rk[j];
          m += p1 * rk[j];
        }
        p2 = daq * p.scale * e;
        m += p2 * rq[j];
      }
      sP1[t * L::LDC + s] = to_e<E>(p1);
      sP2[t * L::LDC + s] = to_e<E>(p2);
      sP1T[s * L::LDC + t] = to_e<E>(p1);
      sP2T[s * L::LDC + t] = to_e<E>(p2);
      sM[t * L::LDF + s] = m;
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float r = group16_sum(db[j]);
    if ((lane & 15) == 0) sDb[t0 + acc_row(lane, j)] = r;
  }
  __syncthreads();
  // gate: dG_t += sum_s M[t,s] - sum_s M[s,t]; beta
  if (tid < ci.len) {
    float row = 0.f, col = 0.f;
    for (int s = 0; s < C; ++s) {
      row += sM[tid * L::LDF + s];
      col += sM[s * L::LDF + tid];
    }
    const int64_t idx = (int64_t)(ci.start + tid) * H + h;
    p.dgcum[idx] += row - col;
    p.dbeta[idx] += sDb[tid];
  }
  // dk += P1 KW, dq += P2 KW, dkw += P1^T K + P2^T Q
  float* dk = p.dk + row0 * D;
  float* dq = p.dq + row0 * D;
  float* dkw = (p.kw_is_k ? p.dk : p.dkw) + row0 * D;
  for (int ct = 0; ct < NCT; ++ct) {
    f32x4 ak = zero4(), aq = zero4(), aw = zero4();
    mma_tile<E, ROW, COL>(ak, sP1, L::LDC, t0, sKWT, L::LDC, 16 * ct, C, lane);
    mma_tile<E, ROW, COL>(aq, sP2, L::LDC, t0, sKWT, L::LDC, 16 * ct, C, lane);
    mma_tile<E, ROW, COL>(aw, sP1T, L::LDC, t0, sKT, L::LDC, 16 * ct, C, lane);
    mma_tile<E, ROW, COL>(aw, sP2T, L::LDC, t0, sQT, L::LDC, 16 * ct, C, lane);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = t0 + acc_row(lane, j), c = 16 * ct + acc_col(lane);
      if (t < ci.len) {
        const int64_t o = t * gs + c;
        dq[o] += aq[j];
        if (p.kw_is_k) {
          dk[o] += ak[j] + aw[j];
        } else {
          dk[o] += ak[j];
          dkw[o] += aw[j];
        }
      }
    }
  }
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

template <typename T, int D, int BV>
int launch_bwd(const BwdParams& p, int num_chunks, int stages, hipStream_t s) {
  const int N = p.geom.num_seqs;
  const bool all = stages == 0;
  if (all || (stages & PKDA_STAGE_BWD_STATE)) {
    auto kern = chunk_state_bwd_kernel<T, D, BV>;
    const int bytes = StateBwdLayout<T, D, BV>::bytes;
    if (int st = set_smem(kern, bytes)) return st;
    if (N > 0) hipLaunchKernelGGL(kern, dim3(N, p.H, D / BV), dim3(kWG), bytes, s, p);
    if (int st = launch_status("pkda_chunk_bwd(state)")) return st;
  }
  if (num_chunks == 0) return 0;
  if (all || (stages & PKDA_STAGE_BWD_DQKW)) {
    auto kern = chunk_dqkw_kernel<T, D>;
    const int bytes = DqkwLayout<T, D>::bytes;
    if (int st = set_smem(kern, bytes)) return st;
    hipLaunchKernelGGL(kern, dim3(num_chunks, p.H), dim3(kWG), bytes, s, p);
    if (int st = launch_status("pkda_chunk_bwd(dqkw)")) return st;
  }
  if (all || (stages & PKDA_STAGE_BWD_WY)) {
    auto kern = chunk_wy_bwd_kernel<T, D>;
    const int bytes = WyLayout<T, D>::bytes;
    if (int st = set_smem(kern, bytes)) return st;
    hipLaunchKernelGGL(kern, dim3(num_chunks, p.H), dim3(kWG), bytes, s, p);
    if (int st = launch_status("pkda_chunk_bwd(wy)")) return st;
  }
  if (all || (stages & PKDA_STAGE_BWD_INTRA)) {
    auto kern = chunk_intra_bwd_kernel<T, D>;
    const int bytes = IntraBwdLayout<T, D>::bytes;
    if (int st = set_smem(kern, bytes)) return st;
    hipLaunchKernelGGL(kern, dim3(num_chunks, p.H), dim3(kWG), bytes, s, p);
    if (int st = launch_status("pkda_chunk_bwd(intra)")) return st;
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
  PKDA_REQUIRE(!a->gate_per_channel, PKDA_EUNSUPPORTED, "per-channel gates are not in this chunked build");
  BwdParams p;
  if (int st = chunk_geom_from(a->cu_seqlens, a->num_seqs, a->seqlen, a->num_chunks, a->table, p.geom)) return st;
  if (a->num_seqs == 0) return 0;
  PKDA_REQUIRE(a->q && a->k && a->v && a->gcum && a->beta && a->w && a->u && a->aqk && a->akk && a->h && a->do_ &&
                   a->dh && a->du && a->dw && a->daqk && a->da && a->dq && a->dk && a->dv && a->dbeta && a->dgcum,
               PKDA_EINVAL, "null tensor");
  const bool kw_is_k = a->kw == nullptr || a->kw == a->k;
  PKDA_REQUIRE(kw_is_k || a->dkw, PKDA_EINVAL, "a separate write key needs dkw");
  p.H = a->heads;
  p.q = a->q; p.k = a->k; p.kw = kw_is_k ? a->k : a->kw; p.v = a->v;
  p.gcum = a->gcum; p.beta = a->beta; p.scale = a->scale;
  p.w = a->w; p.u = a->u; p.aqk = a->aqk; p.akk = a->akk; p.h = a->h;
  p.dO = a->do_; p.dht = a->dht; p.dh = a->dh;
  p.du = a->du; p.dw = a->dw; p.daqk = a->daqk; p.da = a->da;
  p.dq = a->dq; p.dk = a->dk; p.dkw = a->dkw; p.dv = a->dv; p.dbeta = a->dbeta; p.dgcum = a->dgcum; p.dh0 = a->dh0;
  p.kw_is_k = kw_is_k;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nc = a->num_chunks;
  const int st = a->stages;
  PKDA_REQUIRE(st >= 0 && st <= 15, PKDA_EINVAL, "stages %d", st);
  if (a->dtype == PKDA_BF16) {
    return a->head_dim == 128 ? launch_bwd<bf16_t, 128, 64>(p, nc, st, s) : launch_bwd<bf16_t, 64, 64>(p, nc, st, s);
  }
  return launch_bwd<float, 64, 64>(p, nc, st, s);
}
