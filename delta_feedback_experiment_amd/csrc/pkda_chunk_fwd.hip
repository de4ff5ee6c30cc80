// Chunked PKDA forward for gfx950: an intra-chunk pass over all chunks in
// parallel, then a per-document pass that carries the FP32 state across
// chunks.  Chunk algebra, per chunk of C = 64 tokens with entering state S0
// and chunk-local cumulative log-decay G (per head here):
//
//   Akk[t,s] = beta_t exp(G_t - G_s) (k_t . kw_s)          s <  t
//   T        = (I + Akk)^-1
//   W        = T diag(beta exp(G)) K,   Uu = T diag(beta) V
//   Aqk[t,s] = scale exp(G_t - G_s) (q_t . kw_s)           s <= t
//   U        = Uu - W S0
//   O        = diag(scale exp(G)) Q S0 + Aqk U
//   S_C      = exp(G_last) S0 + (diag(exp(G_last - G)) KW)^T U
//
// which is the token recurrence of delta_feedback_experiment/pkda.py:399-406
// with the prediction read by k and the write by the preconditioned kw.
//
// intra kernel: one workgroup per (chunk, head).  Akk/Aqk on MFMA; T by a
//   blocked solve: each 16x16 diagonal block (I + N) is inverted as
//   (I - N)(I + N^2)(I + N^4)(I + N^8) (N is strictly lower, N^16 = 0) and
//   the off-diagonal blocks follow by block forward substitution, all on
//   FP32 MFMA; W and Uu on MFMA.
// state kernel: one workgroup per (document, head, BV value columns).  The
//   FP32 state slice lives in MFMA accumulators for the whole document; each
//   chunk it is published to LDS (as the B operand), U, O and the update are
//   MFMA products.
#include "pkda_chunk_common.h"

namespace pkda {
namespace {

struct FwdParams {
  ChunkGeom geom;
  int H;
  const void* q;
  const void* k;
  const void* kw;
  const void* v;
  const float* gcum;
  const float* beta;
  float scale;
  const float* s0;
  float* sT;
  void* o;
  void* w;
  void* u;
  void* aqk;
  void* akk;
  void* h;
};

__device__ __forceinline__ float clamp_gate(const float* s_gam, int t) { return s_gam[t]; }

// Load per-row beta and cumulative gate of a chunk into LDS.  Rows past the
// chunk's end repeat the last cumulative gate (so exp(G_t - G_s) stays finite
// where masks zero it) and get beta = 0.
__device__ __forceinline__ void load_chunk_scalars(float* s_beta, float* s_gam, const float* beta, const float* gcum,
                                                   int start, int len, int H, int h) {
  const int t = threadIdx.x;
  if (t < C) {
    const int tt = t < len ? t : len - 1;
    const int64_t idx = (int64_t)(start + tt) * H + h;
    s_gam[t] = gcum[idx];
    if (s_beta) s_beta[t] = t < len ? beta[idx] : 0.f;
  }
}

// ---------------------------------------------------------------------------
// Blocked inverse of (I + A), A strictly lower 64x64 FP32 in LDS (ld = ldf).
// Result into s_t (same ld).  scratch: 4 waves x 3 x 16 x 17 floats.
// ---------------------------------------------------------------------------
constexpr int SLD = 17;

__device__ __forceinline__ void solve_unit_lower_64(const float* s_a, float* s_t, int ldf, float* scratch) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  for (int i = tid; i < C * C; i += kWG) s_t[(i / C) * ldf + (i % C)] = 0.f;
  float* M = scratch + wave * 3 * 16 * SLD;
  float* P = M + 16 * SLD;
  float* X = P + 16 * SLD;
  const int b = wave;  // diagonal block of this wave
  const float* N = s_a + (16 * b) * ldf + 16 * b;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = acc_row(lane, j), c = acc_col(lane);
    const float n = N[r * ldf + c];
    M[r * SLD + c] = n;
    P[r * SLD + c] = (r == c ? 1.f : 0.f) - n;
  }
  __syncthreads();
  for (int step = 0; step < 3; ++step) {
    f32x4 acc = zero4();
    mma_tile<float, ROW, ROW>(acc, M, SLD, 0, M, SLD, 0, 16, lane);  // M <- M^2
    __syncthreads();
    store_acc_lds(M, SLD, acc, 0, 0, lane);
    __syncthreads();
    f32x4 pacc;
#pragma unroll
    for (int j = 0; j < 4; ++j) pacc[j] = P[acc_row(lane, j) * SLD + acc_col(lane)];
    mma_tile<float, ROW, ROW>(pacc, P, SLD, 0, M, SLD, 0, 16, lane);  // P <- P (I + M)
    __syncthreads();
    store_acc_lds(P, SLD, pacc, 0, 0, lane);
    __syncthreads();
  }
  // diagonal block inverse -> s_t
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = acc_row(lane, j), c = acc_col(lane);
    s_t[(16 * b + r) * ldf + 16 * b + c] = P[r * SLD + c];
  }
  __syncthreads();
  // off-diagonal blocks, block row by block row: T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj
  for (int i = 1; i < 4; ++i) {
    const int j = wave;
    const bool active = j < i;
    f32x4 x = zero4();
    if (active) {
      for (int k = j; k < i; ++k)
        mma_tile<float, ROW, ROW>(x, s_a + (16 * i) * ldf + 16 * k, ldf, 0, s_t + (16 * k) * ldf + 16 * j, ldf, 0, 16,
                                  lane);
      store_acc_lds(X, SLD, x, 0, 0, lane);
    }
    __syncthreads();
    if (active) {
      f32x4 y = zero4();
      mma_tile<float, ROW, ROW>(y, s_t + (16 * i) * ldf + 16 * i, ldf, 0, X, SLD, 0, 16, lane);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
        s_t[(16 * i + acc_row(lane, jj)) * ldf + 16 * j + acc_col(lane)] = -y[jj];
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// intra-chunk forward
// ---------------------------------------------------------------------------
template <typename T, int D>
struct IntraLayout {
  static constexpr int LD = D + Pad<T>::v;
  static constexpr int LDC = C + Pad<T>::v;
  static constexpr int LDF = C + 4;
  static constexpr int X12 = 3 * C * LD * (int)sizeof(T);
  static constexpr int X4 = 2 * D * LDC * (int)sizeof(T);
  static constexpr int XS = 4 * 3 * 16 * SLD * (int)sizeof(float);
  static constexpr int XB = (X12 > X4 ? (X12 > XS ? X12 : XS) : (X4 > XS ? X4 : XS));
  static constexpr int off_A = (XB + 15) / 16 * 16;
  static constexpr int off_T = off_A + C * LDF * 4;
  static constexpr int off_Te = off_T + C * LDF * 4;
  static constexpr int off_beta = off_Te + C * LDC * (int)sizeof(T) + 16;
  static constexpr int off_gam = off_beta + C * 4;
  static constexpr int bytes = off_gam + C * 4;
};

template <typename T, int D>
__global__ __launch_bounds__(kWG) void chunk_intra_fwd_kernel(FwdParams p) {
  using L = IntraLayout<T, D>;
  using E = T;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const ChunkInfo ci = chunk_info(p.geom, blockIdx.x);
  if (ci.len <= 0) return;
  const int h = blockIdx.y;
  const int H = p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t row0 = (int64_t)ci.start * H + h;  // token-row index of the chunk's first token
  const int64_t gs = (int64_t)H * D;               // token stride in elements

  E* sK = reinterpret_cast<E*>(smem);
  E* sKW = sK + C * L::LD;
  E* sQ = sKW + C * L::LD;
  float* sA = reinterpret_cast<float*>(smem + L::off_A);
  float* sTf = reinterpret_cast<float*>(smem + L::off_T);
  E* sTe = reinterpret_cast<E*>(smem + L::off_Te);
  float* sBeta = reinterpret_cast<float*>(smem + L::off_beta);
  float* sGam = reinterpret_cast<float*>(smem + L::off_gam);

  const T* q = static_cast<const T*>(p.q) + row0 * D;
  const T* k = static_cast<const T*>(p.k) + row0 * D;
  const T* kw = static_cast<const T*>(p.kw) + row0 * D;
  const T* v = static_cast<const T*>(p.v) + row0 * D;
  const bool alias = p.kw == p.k;

  load_chunk_scalars(sBeta, sGam, p.beta, p.gcum, ci.start, ci.len, H, h);
  load_rows<T, E, D>(sK, L::LD, k, gs, C, ci.len, Ident());
  if (!alias) load_rows<T, E, D>(sKW, L::LD, kw, gs, C, ci.len, Ident());
  load_rows<T, E, D>(sQ, L::LD, q, gs, C, ci.len, Ident());
  __syncthreads();
  const E* sKWr = alias ? sK : sKW;

  // ---- Akk, Aqk: wave w owns row tile w ------------------------------------
  T* aqk_out = static_cast<T*>(p.aqk) + row0 * C;
  for (int ct = 0; ct < 4; ++ct) {
    f32x4 akk = zero4(), aqk = zero4();
    if (ct <= wave) {
      mma_tile<E, ROW, COL>(akk, sK, L::LD, 16 * wave, sKWr, L::LD, 16 * ct, D, lane);
      mma_tile<E, ROW, COL>(aqk, sQ, L::LD, 16 * wave, sKWr, L::LD, 16 * ct, D, lane);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * wave + acc_row(lane, j);
      const int s = 16 * ct + acc_col(lane);
      const bool valid_t = t < ci.len;
      const float dec = (s <= t && valid_t) ? expf(sGam[t] - sGam[s]) : 0.f;
      sA[t * L::LDF + s] = (s < t) ? sBeta[t] * dec * akk[j] : 0.f;
      if (valid_t) io<T>::store(aqk_out + (int64_t)t * H * C + s, p.scale * dec * aqk[j]);
    }
  }
  __syncthreads();

  // ---- T = (I + Akk)^-1 ------------------------------------------------------
  solve_unit_lower_64(sA, sTf, L::LDF, reinterpret_cast<float*>(smem));
  T* akk_out = static_cast<T*>(p.akk) + row0 * C;
  for (int i = tid; i < C * C; i += kWG) {
    const int r = i / C, c = i % C;
    const float x = sTf[r * L::LDF + c];
    sTe[r * L::LDC + c] = to_e<E>(x);
    if (r < ci.len) io<T>::store(akk_out + (int64_t)r * H * C + c, x);
  }
  // ---- W = T diag(beta e^G) K,  Uu = T diag(beta) V ---------------------------
  E* sBw = reinterpret_cast<E*>(smem);
  E* sBv = sBw + C * L::LD;
  load_rows<T, E, D>(sBw, L::LD, k, gs, C, ci.len,
                     [&](int r, int, float x) { return sBeta[r] * expf(sGam[r]) * x; });
  load_rows<T, E, D>(sBv, L::LD, v, gs, C, ci.len, [&](int r, int, float x) { return sBeta[r] * x; });
  __syncthreads();
  const int kdim = ((16 * (wave + 1) + Mma<E>::KS - 1) / Mma<E>::KS) * Mma<E>::KS;  // T is lower triangular
  T* w_out = static_cast<T*>(p.w) + row0 * D;
  T* u_out = static_cast<T*>(p.u) + row0 * D;
  for (int ct = 0; ct < D / 16; ++ct) {
    f32x4 aw = zero4(), au = zero4();
    mma_tile<E, ROW, ROW>(aw, sTe, L::LDC, 16 * wave, sBw, L::LD, 16 * ct, kdim, lane);
    mma_tile<E, ROW, ROW>(au, sTe, L::LDC, 16 * wave, sBv, L::LD, 16 * ct, kdim, lane);
    store_acc_global<T>(w_out, gs, aw, 16 * wave, 16 * ct, ci.len, lane);
    store_acc_global<T>(u_out, gs, au, 16 * wave, 16 * ct, ci.len, lane);
  }
}

// ---------------------------------------------------------------------------
// per-document state pass
//
// One workgroup per (document, head, BV value columns).  The FP32 state slice
// S [D x BV] lives in MFMA accumulators; each chunk it is published to LDS
// (bf16/fp32, natural [c][v] layout) as the B operand of W S and Q S.  The
// next chunk's tiles (W, Q, KW, Aqk, u, G) are loaded into registers while the
// current chunk computes, so the chain of chunks is not serialised on HBM
// latency.  Per chunk:
//   U = u - W S                     (written back over u: the backward's U)
//   O = diag(s e^G) (Q S) + Aqk U
//   S <- e^{G_C} S + KW^T diag(e^{G_C - G}) U
// with the decays applied to accumulator rows or to U, never to the loaded
// tiles.
// ---------------------------------------------------------------------------
template <typename T, int D, int BV>
struct StateLayout {
  static constexpr int LD = D + Pad<T>::v;
  static constexpr int LDV = BV + Pad<T>::v;
  static constexpr int LDC = C + Pad<T>::v;
  static constexpr int off_S = 0;                                     // [D][LDV]
  static constexpr int off_W = off_S + D * LDV * (int)sizeof(T);      // [64][LD]
  static constexpr int off_Q = off_W + C * LD * (int)sizeof(T);       // [64][LD]
  static constexpr int off_KW = off_Q + C * LD * (int)sizeof(T);      // [64][LD]
  static constexpr int off_Aqk = off_KW + C * LD * (int)sizeof(T);    // [64][LDC]
  static constexpr int off_Uin = off_Aqk + C * LDC * (int)sizeof(T);  // [64][LDV]  u
  static constexpr int off_U = off_Uin + C * LDV * (int)sizeof(T);    // [64][LDV]  U
  static constexpr int off_Ug = off_U + C * LDV * (int)sizeof(T);     // [64][LDV]  e^{G_C-G} U
  static constexpr int off_gam = off_Ug + C * LDV * (int)sizeof(T);
  static constexpr int bytes = off_gam + C * 4;
};

template <typename T, int D, int BV>
__global__ __launch_bounds__(kWG) void chunk_state_fwd_kernel(FwdParams p) {
  using L = StateLayout<T, D, BV>;
  using E = T;
  constexpr int NCT = BV / 16;              // column tiles of the slice
  constexpr int NS = (D / 16) * NCT / 4;    // state tiles per wave
  extern __shared__ __attribute__((aligned(16))) char smem[];
  E* sS = reinterpret_cast<E*>(smem + L::off_S);
  E* sW = reinterpret_cast<E*>(smem + L::off_W);
  E* sQ = reinterpret_cast<E*>(smem + L::off_Q);
  E* sKW = reinterpret_cast<E*>(smem + L::off_KW);
  E* sAqk = reinterpret_cast<E*>(smem + L::off_Aqk);
  E* sUin = reinterpret_cast<E*>(smem + L::off_Uin);
  E* sU = reinterpret_cast<E*>(smem + L::off_U);
  E* sUg = reinterpret_cast<E*>(smem + L::off_Ug);
  float* sGam = reinterpret_cast<float*>(smem + L::off_gam);

  const int n = blockIdx.x, h = blockIdx.y, v0 = blockIdx.z * BV;
  const int H = p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t gs = (int64_t)H * D;
  int first, count, dstart, dlen;
  doc_chunks(p.geom, n, first, count, dstart, dlen);

  f32x4 S[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const int ti = wave * NS + i;
    const int rt = ti / NCT, ct = ti % NCT;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = 16 * rt + acc_row(lane, j), c = v0 + 16 * ct + acc_col(lane);
      S[i][j] = p.s0 ? p.s0[((int64_t)n * H + h) * D * D + r * D + c] : 0.f;
    }
  }

  RegTile<kWG, C, D, T> rW, rQ, rKW;
  RegTile<kWG, C, C, T> rA;
  RegTile<kWG, C, BV, T> rU;
  float rg = 0.f;
  auto prefetch = [&](int jc) {
    const int cstart = dstart + jc * C;
    const int clen = min(C, dlen - jc * C);
    const int64_t row0 = (int64_t)cstart * H + h;
    rW.load(static_cast<const T*>(p.w) + row0 * D, gs, clen);
    rQ.load(static_cast<const T*>(p.q) + row0 * D, gs, clen);
    rKW.load(static_cast<const T*>(p.kw) + row0 * D, gs, clen);
    rA.load(static_cast<const T*>(p.aqk) + row0 * C, (int64_t)H * C, clen);
    rU.load(static_cast<const T*>(p.u) + row0 * D + v0, gs, clen);
    if (tid < C) rg = p.gcum[(int64_t)(cstart + min(tid, clen - 1)) * H + h];
  };
  if (count > 0) prefetch(0);
  const float scale = p.scale;
  const int r0 = 16 * wave;

  for (int jc = 0; jc < count; ++jc) {
    const int cid = first + jc;
    const int cstart = dstart + jc * C;
    const int clen = min(C, dlen - jc * C);
    const int64_t row0 = (int64_t)cstart * H + h;
    // publish this chunk's operands and the entering state; checkpoint it
    rW.store(sW, L::LD);
    rQ.store(sQ, L::LD);
    rKW.store(sKW, L::LD);
    rA.store(sAqk, L::LDC);
    rU.store(sUin, L::LDV);
    if (tid < C) sGam[tid] = rg;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int ti = wave * NS + i;
      const int rt = ti / NCT, ct = ti % NCT;
      store_acc_lds(sS, L::LDV, S[i], 16 * rt, 16 * ct, lane);
      if (p.h) {
        T* hb = static_cast<T*>(p.h) + ((int64_t)cid * H + h) * D * D + v0;
        store_acc_global<T>(hb, D, S[i], 16 * rt, 16 * ct, D, lane);
      }
    }
    __syncthreads();
    if (jc + 1 < count) prefetch(jc + 1);
    const float gC = sGam[C - 1];  // padded rows repeat the last valid gate
    float eg[4], egc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float g = sGam[r0 + acc_row(lane, e)];
      eg[e] = scale * expf(g);
      egc[e] = expf(gC - g);
    }
    // U = u - W S
    T* u_io = static_cast<T*>(p.u) + row0 * D + v0;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      f32x4 acc = zero4();
      mma_tile<E, ROW, ROW>(acc, sW, L::LD, r0, sS, L::LDV, 16 * ct, D, lane);
      f32x4 U;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = r0 + acc_row(lane, e), c = 16 * ct + acc_col(lane);
        U[e] = from_e<E>(sUin[r * L::LDV + c]) - acc[e];
        sU[r * L::LDV + c] = to_e<E>(U[e]);
        sUg[r * L::LDV + c] = to_e<E>(egc[e] * U[e]);
      }
      store_acc_global<T>(u_io, gs, U, r0, 16 * ct, clen, lane);
    }
    __syncthreads();
    // O = diag(s e^G) Q S + Aqk U
    T* o_out = static_cast<T*>(p.o) + row0 * D + v0;
    const int kend = kceil<E>(r0 + 16);  // Aqk is lower triangular
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      f32x4 a1 = zero4(), a2 = zero4();
      mma_tile<E, ROW, ROW>(a1, sQ, L::LD, r0, sS, L::LDV, 16 * ct, D, lane);
      mma_tile_range<E, ROW, ROW>(a2, sAqk, L::LDC, r0, sU, L::LDV, 16 * ct, 0, kend, lane);
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = eg[e] * a1[e] + a2[e];
      store_acc_global<T>(o_out, gs, o, r0, 16 * ct, clen, lane);
    }
    // S <- e^{G_C} S + KW^T Ug
    const float decay = expf(gC);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int ti = wave * NS + i;
      const int rt = ti / NCT, ct = ti % NCT;
      S[i] = S[i] * decay;
      mma_tile<E, COL, ROW>(S[i], sKW, L::LD, 16 * rt, sUg, L::LDV, 16 * ct, C, lane);
    }
    __syncthreads();
  }
  if (p.sT) {
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int ti = wave * NS + i;
      const int rt = ti / NCT, ct = ti % NCT;
      float* sb = p.sT + ((int64_t)n * H + h) * D * D + v0;
      store_acc_global<float>(sb, D, S[i], 16 * rt, 16 * ct, D, lane);
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
int launch_fwd(const FwdParams& p, int num_chunks, int stages, hipStream_t s) {
  const bool all = stages == 0;
  if (all || (stages & PKDA_STAGE_FWD_INTRA)) {
    auto kern = chunk_intra_fwd_kernel<T, D>;
    const int bytes = IntraLayout<T, D>::bytes;
    if (int st = set_smem(kern, bytes)) return st;
    if (num_chunks > 0) hipLaunchKernelGGL(kern, dim3(num_chunks, p.H), dim3(kWG), bytes, s, p);
    if (int st = launch_status("pkda_chunk_fwd(intra)")) return st;
  }
  if (all || (stages & PKDA_STAGE_FWD_STATE)) {
    auto kern = chunk_state_fwd_kernel<T, D, BV>;
    const int bytes = StateLayout<T, D, BV>::bytes;
    if (int st = set_smem(kern, bytes)) return st;
    if (p.geom.num_seqs > 0) hipLaunchKernelGGL(kern, dim3(p.geom.num_seqs, p.H, D / BV), dim3(kWG), bytes, s, p);
    if (int st = launch_status("pkda_chunk_fwd(state)")) return st;
  }
  return 0;
}

}  // namespace

int chunk_geom_from(const int32_t* cu, int num_seqs, int seqlen, int num_chunks, const int32_t* table, ChunkGeom& g) {
  PKDA_REQUIRE(num_seqs >= 0 && num_chunks >= 0, PKDA_EINVAL, "sizes");
  g.num_seqs = num_seqs;
  g.seqlen = seqlen;
  g.cu = cu;
  g.nt = cu ? 0 : (seqlen + C - 1) / C;
  g.table = reinterpret_cast<const int4*>(table);
  g.offsets = table ? table + 4 * num_chunks : nullptr;
  g.num_chunks = num_chunks;
  PKDA_REQUIRE(!cu || table, PKDA_EINVAL, "packed documents need the chunk table (pkda_chunk_table)");
  PKDA_REQUIRE(cu || num_chunks == num_seqs * g.nt, PKDA_EINVAL, "num_chunks %d != num_seqs * ceil(seqlen / 64) = %d",
               num_chunks, num_seqs * g.nt);
  return 0;
}

}  // namespace pkda

using namespace pkda;

extern "C" int pkda_chunk_fwd(const pkda_chunk_fwd_args* a, void* stream) {
  PKDA_REQUIRE(a != nullptr, PKDA_EINVAL, "null args");
  PKDA_REQUIRE(a->struct_size == (int32_t)sizeof(pkda_chunk_fwd_args), PKDA_EINVAL, "pkda_chunk_fwd_args size mismatch");
  PKDA_REQUIRE(a->dtype == PKDA_F32 || a->dtype == PKDA_BF16, PKDA_EUNSUPPORTED, "dtype %d", a->dtype);
  PKDA_REQUIRE(a->head_dim == 64 || a->head_dim == 128, PKDA_EUNSUPPORTED, "chunked head_dim %d (64, 128)", a->head_dim);
  PKDA_REQUIRE(a->heads > 0, PKDA_EINVAL, "heads");
  PKDA_REQUIRE(!a->gate_per_channel, PKDA_EUNSUPPORTED, "per-channel gates are not in this chunked build");
  FwdParams p;
  if (int st = chunk_geom_from(a->cu_seqlens, a->num_seqs, a->seqlen, a->num_chunks, a->table, p.geom)) return st;
  if (a->num_seqs == 0) return 0;
  PKDA_REQUIRE(a->q && a->k && a->v && a->gcum && a->beta && a->o && a->w && a->u && a->aqk && a->akk, PKDA_EINVAL,
               "null tensor");
  p.H = a->heads;
  p.q = a->q; p.k = a->k; p.kw = a->kw ? a->kw : a->k; p.v = a->v;
  p.gcum = a->gcum; p.beta = a->beta; p.scale = a->scale;
  p.s0 = a->initial_state; p.sT = a->final_state; p.o = a->o;
  p.w = a->w; p.u = a->u; p.aqk = a->aqk; p.akk = a->akk; p.h = a->h;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nc = a->num_chunks;
  const int st = a->stages;
  PKDA_REQUIRE(st >= 0 && st <= (PKDA_STAGE_FWD_INTRA | PKDA_STAGE_FWD_STATE), PKDA_EINVAL, "stages %d", st);
  if (a->dtype == PKDA_BF16) {
    return a->head_dim == 128 ? launch_fwd<bf16_t, 128, 64>(p, nc, st, s) : launch_fwd<bf16_t, 64, 64>(p, nc, st, s);
  }
  return a->head_dim == 128 ? launch_fwd<float, 128, 16>(p, nc, st, s) : launch_fwd<float, 64, 64>(p, nc, st, s);
}
