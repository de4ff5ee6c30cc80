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
#include <type_traits>

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
  void* qg;   // per-channel gates: s e^G q
  void* kg;   // per-channel gates: e^{G_last - G} kw
  const int32_t* slot;  // document -> state row (slot-indexed pools), or null
  const float* gcum_lo;  // FP32 per-channel gates, optional: gcum's FP64 remainder
  bool tri_packed;       // BF16, per-head gate, kw = k: Aqk and T as their ten lower blocks
};

// Row of the initial/final state of document n.
__device__ __forceinline__ int64_t state_row(const FwdParams& p, int n) { return p.slot ? p.slot[n] : n; }

// ---------------------------------------------------------------------------
// Blocked inverse of (I + A) in place, A strictly lower 64x64 FP32 in LDS
// (ld = ldf) whose blocks above the diagonal are zero.  Each 16x16 diagonal
// block (I + N) is inverted as (I - N)(I + N^2)(I + N^4)(I + N^8) (N^16 = 0)
// in three squarings, then the blocks below the diagonal follow by block
// forward substitution T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj, one block row at
// a time; all products on FP32 MFMA.  Waves 0..3 work, every wave of the
// workgroup reaches every barrier.  scratch: 4 x 3 x 16 x SLD floats.
// ---------------------------------------------------------------------------
constexpr int SLD = 17;

// Orders this wave's LDS accesses (its stores before its later loads): the
// diagonal-block phase of the solve touches only wave-private scratch, so a
// wavefront fence stands in for a workgroup barrier there.
__device__ __forceinline__ void wave_lds_fence() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); }

__device__ __forceinline__ void solve_unit_lower_64(float* s, int ldf, float* scratch) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const bool active = wave < 4;
  const int b = wave & 3;  // diagonal block of this wave
  float* M = scratch + b * 3 * 16 * SLD;
  float* P = M + 16 * SLD;
  float* X = P + 16 * SLD;
  float* N = s + (16 * b) * ldf + 16 * b;
  if (active) {  // wave-private: M, P and this wave's diagonal block
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = acc_row(lane, j), c = acc_col(lane);
      const float n = N[r * ldf + c];
      M[r * SLD + c] = n;
      P[r * SLD + c] = (r == c ? 1.f : 0.f) - n;
    }
    for (int step = 0; step < 3; ++step) {
      wave_lds_fence();
      f32x4 acc = zero4(), pacc;
      mma_tile<float, ROW, ROW>(acc, M, SLD, 0, M, SLD, 0, 16, lane);  // M <- M^2
#pragma unroll
      for (int j = 0; j < 4; ++j) pacc[j] = P[acc_row(lane, j) * SLD + acc_col(lane)];
      wave_lds_fence();
      store_acc_lds(M, SLD, acc, 0, 0, lane);
      wave_lds_fence();
      mma_tile<float, ROW, ROW>(pacc, P, SLD, 0, M, SLD, 0, 16, lane);  // P <- P (I + M)
      wave_lds_fence();
      store_acc_lds(P, SLD, pacc, 0, 0, lane);
    }
    wave_lds_fence();
#pragma unroll
    for (int j = 0; j < 4; ++j) N[acc_row(lane, j) * ldf + acc_col(lane)] = P[acc_row(lane, j) * SLD + acc_col(lane)];
  }
  __syncthreads();
  for (int i = 1; i < 4; ++i) {
    const int j = b;
    const bool on = active && j < i;
    f32x4 y = zero4();
    if (on) {  // X is this wave's own
      f32x4 x = zero4();
      for (int k = j; k < i; ++k)
        mma_tile<float, ROW, ROW>(x, s + (16 * i) * ldf + 16 * k, ldf, 0, s + (16 * k) * ldf + 16 * j, ldf, 0, 16,
                                  lane);
      store_acc_lds(X, SLD, x, 0, 0, lane);
      wave_lds_fence();
      mma_tile<float, ROW, ROW>(y, s + (16 * i) * ldf + 16 * i, ldf, 0, X, SLD, 0, 16, lane);
    }
    __syncthreads();  // every wave has read row i's A blocks before T_ij replaces them
    if (on) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) s[(16 * i + acc_row(lane, jj)) * ldf + 16 * j + acc_col(lane)] = -y[jj];
    }
    __syncthreads();  // row i of T is complete before row i + 1 reads it
  }
}


// ---------------------------------------------------------------------------
// intra-chunk forward: one 8-wave workgroup per (chunk, head).
//   Akk, Aqk   the ten 16x16 blocks on or below the diagonal (raw k.kw and
//              q.kw products, then the pairwise decay): Akk into LDS (FP32)
//              for the solve, Aqk straight from the accumulators to global
//              memory; the six blocks above the diagonal are written as zeros;
//   T          in place over Akk (waves 0..3), then to global memory;
//   W, u       (WU only) (T diag(beta e^G)) K, (T diag(beta)) V: wave w owns
//              row block w % 4 and column half w / 4; they leave from the
//              accumulators.  Without WU the state passes form W S and W^T dU
//              from T and K themselves, and V is not read here.
// LDS is three [64 x D] regions, reused as the work moves on (52 KB at
// D = 128 BF16, three workgroups per compute unit):
//   region K:  K
//   region Q:  Q, then the solve's scratch, then T diag(beta e^G) and
//              T diag(beta) in the operand type (the row scalings of K and V
//              folded into T's columns)
//   region A:  Akk / T in FP32, then V (which waits in registers)
// ---------------------------------------------------------------------------
constexpr int kIW = 512;

template <typename T, int D, bool ALIAS>
struct IntraLayout {
  static constexpr int LD = D + Pad<T>::v;
  static constexpr int LDC = C + Pad<T>::v;
  static constexpr int LDF = C + 4;
  static constexpr int RT = C * LD * (int)sizeof(T);
  static constexpr int SCR = 4 * 3 * 16 * SLD * 4;       // solve scratch
  static constexpr int TE = C * LDC * (int)sizeof(T);    // T in the operand type
  static constexpr int max3(int a, int b, int c) { return a > b ? (a > c ? a : c) : (b > c ? b : c); }
  static constexpr int QR = max3(RT, SCR, 2 * TE);
  static constexpr int AR = C * LDF * 4 > RT ? C * LDF * 4 : RT;
  static constexpr int off_K = 0;                         // K, then Bw
  static constexpr int off_Q = off_K + RT;                // Q, then solve scratch, then Tw | Tu
  static constexpr int off_KW = off_Q + QR;               // KW (when not aliased to K)
  static constexpr int off_A = off_KW + (ALIAS ? 0 : RT); // fp32 [64][LDF]: Akk, then T; then V
  static constexpr int off_beta = off_A + AR;
  static constexpr int off_gam = off_beta + C * 4;
  static constexpr int bytes = off_gam + C * 4;
  // Without W and u (the state passes form them from T) and where it fits:
  // Akk waits in the accumulators until every wave is done with K, then takes
  // K's region, so the workgroup needs no region of its own for it (four per
  // compute unit at D = 128 BF16 instead of three).
  static constexpr bool lean_fits = C * LDF * 4 <= RT && SCR <= RT;
  static constexpr int off_A_lean = off_K;
  static constexpr int off_beta_lean = off_KW + (ALIAS ? 0 : RT);
  static constexpr int off_gam_lean = off_beta_lean + C * 4;
  static constexpr int bytes_lean = off_gam_lean + C * 4;
};

// The body for one chunk; `len` is a literal C for whole chunks (every row
// test folds away, so no branch holds a load back).
template <typename T, int D, bool ALIAS, bool WU>
__device__ __forceinline__ void intra_fwd_chunk(const FwdParams& p, const ChunkInfo ci, const int len, char* smem) {
  using L = IntraLayout<T, D, ALIAS>;
  constexpr bool LEAN = !WU && L::lean_fits;  // Akk over K's region
  using E = T;
  constexpr int HCT = D / 32;  // column tiles per wave of W / u
  const int H = p.H;
  const ChunkHead wg = chunk_head<true>(H);
  const int h = wg.h;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t row0 = (int64_t)ci.start * H + h;  // token-row index of the chunk's first token
  const int64_t gs = (int64_t)H * D;               // token stride in elements

  E* sK = reinterpret_cast<E*>(smem + L::off_K);
  E* sQ = reinterpret_cast<E*>(smem + L::off_Q);
  E* sTw = sQ;                 // T diag(beta e^G)
  E* sTu = sQ + C * L::LDC;    // T diag(beta)
  E* sKW = ALIAS ? sK : reinterpret_cast<E*>(smem + L::off_KW);
  float* sA = reinterpret_cast<float*>(smem + (LEAN ? L::off_A_lean : L::off_A));
  E* sV = reinterpret_cast<E*>(smem + L::off_A);
  float* sBeta = reinterpret_cast<float*>(smem + (LEAN ? L::off_beta_lean : L::off_beta));
  float* sGam = reinterpret_cast<float*>(smem + (LEAN ? L::off_gam_lean : L::off_gam));

  const T* q = static_cast<const T*>(p.q) + row0 * D;
  const T* k = static_cast<const T*>(p.k) + row0 * D;
  const T* kw = static_cast<const T*>(p.kw) + row0 * D;
  const T* v = static_cast<const T*>(p.v) + row0 * D;

  // all tiles in one memory round trip (the gate and beta loads go out first,
  // so that their LDS stores wait for those loads only); V waits in
  // registers until region A frees
  RegTile<kIW, C, D, T> rV;
  {
    const int64_t gidx = (int64_t)(ci.start + min(tid & (C - 1), len - 1)) * H + h;
    const float gval = p.gcum[gidx];  // rows past the end repeat the last gate: e^{G_t-G_s} stays finite
    const float bval = p.beta[gidx];
    RegTile<kIW, C, D, T> rK, rQ, rKW;
    rK.load(k, gs, len);
    rQ.load(q, gs, len);
    if (!ALIAS) rKW.load(kw, gs, len);
    if (WU) rV.load(v, gs, len);
    // every thread writes (the C rows' values, repeated): no branch
    sGam[tid & (C - 1)] = gval;
    sBeta[tid & (C - 1)] = (tid & (C - 1)) < len ? bval : 0.f;
    rK.store(sK, L::LD);
    rQ.store(sQ, L::LD);
    if (!ALIAS) rKW.store(sKW, L::LD);
  }
  __syncthreads();

  // ---- Akk, Aqk: lower blocks 0..9 on MFMA, upper blocks 10..15 zero ----------
  // (block blk = wave + 8 u of this wave; without W and u the Akk values wait
  // in registers until every wave is done with K, whose region they take)
  T* aqk_out = static_cast<T*>(p.aqk) + row0 * C;
  // packed (BF16, per-head gate, kw = k): the chunk's ten lower blocks, rows
  // past its end zero
  constexpr bool TRI_OK = std::is_same<T, bf16_t>::value && !WU;
  const bool tri = TRI_OK && p.tri_packed;
  T* aqk_tri = static_cast<T*>(p.aqk) + ((int64_t)wg.cid * H + h) * kTriElems;
  f32x4 akk_keep[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int blk = wave + 8 * u;
    if (blk < 10) {
      const int tb = blk < 1 ? 0 : blk < 3 ? 1 : blk < 6 ? 2 : 3;
      const int sb = blk - tb * (tb + 1) / 2;
      f32x4 akk = zero4(), aqk = zero4();
      mma_tile<E, ROW, COL>(akk, sK, L::LD, 16 * tb, sKW, L::LD, 16 * sb, D, lane);
      mma_tile<E, ROW, COL>(aqk, sQ, L::LD, 16 * tb, sKW, L::LD, 16 * sb, D, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * tb + acc_row(lane, j);
        const int s = 16 * sb + acc_col(lane);
        const float dec = (s <= t && t < len) ? exp_fast(sGam[t] - sGam[s]) : 0.f;
        akk[j] = (s < t) ? sBeta[t] * dec * akk[j] : 0.f;
        aqk[j] = p.scale * dec * aqk[j];
      }
      if (tri) {
        f32x4 a = aqk;
#pragma unroll
        for (int j = 0; j < 4; ++j) a[j] = 16 * tb + acc_row(lane, j) < len ? a[j] : 0.f;
        store_acc_global<T, true>(aqk_tri + blk * 256, 16, a, 0, 0, 16, lane);
      } else {
        store_acc_global<T>(aqk_out, (int64_t)H * C, aqk, 16 * tb, 16 * sb, len, lane);
      }
      akk_keep[u] = akk;
    } else {  // (tb, sb) above the diagonal
      const int v = blk - 10;  // 0..5: (0,1) (0,2) (0,3) (1,2) (1,3) (2,3)
      const int tb = v < 3 ? 0 : v < 5 ? 1 : 2;
      const int sb = v < 3 ? v + 1 : v < 5 ? v - 1 : 3;
      if (!tri) store_acc_global<T>(aqk_out, (int64_t)H * C, zero4(), 16 * tb, 16 * sb, len, lane);
      akk_keep[u] = zero4();
    }
    if (!LEAN) {  // Akk has a region of its own
      const int b = blk;
      int tb, sb;
      if (b < 10) {
        tb = b < 1 ? 0 : b < 3 ? 1 : b < 6 ? 2 : 3;
        sb = b - tb * (tb + 1) / 2;
      } else {
        const int v = b - 10;
        tb = v < 3 ? 0 : v < 5 ? 1 : 2;
        sb = v < 3 ? v + 1 : v < 5 ? v - 1 : 3;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) sA[(16 * tb + acc_row(lane, j)) * L::LDF + 16 * sb + acc_col(lane)] = akk_keep[u][j];
    }
  }
  if (LEAN) {
    __syncthreads();  // every wave is done with K
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int b = wave + 8 * u;
      int tb, sb;
      if (b < 10) {
        tb = b < 1 ? 0 : b < 3 ? 1 : b < 6 ? 2 : 3;
        sb = b - tb * (tb + 1) / 2;
      } else {
        const int v = b - 10;
        tb = v < 3 ? 0 : v < 5 ? 1 : 2;
        sb = v < 3 ? v + 1 : v < 5 ? v - 1 : 3;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) sA[(16 * tb + acc_row(lane, j)) * L::LDF + 16 * sb + acc_col(lane)] = akk_keep[u][j];
    }
  }
  __syncthreads();

  // ---- T = (I + Akk)^-1 in place (scratch over Q, dead since Aqk) -------------
  solve_unit_lower_64(sA, L::LDF, reinterpret_cast<float*>(sQ));
  if (!WU) {
    if constexpr (TRI_OK) {
      if (tri) {
        store_tri_from_f32<kIW>(static_cast<bf16_t*>(p.akk) + ((int64_t)wg.cid * H + h) * kTriElems, sA, L::LDF,
                                len);
        return;
      }
    }
    store_tile_from_f32<kIW, C, C>(static_cast<T*>(p.akk) + row0 * C, (int64_t)H * C, sA, L::LDF, len);
    return;
  }
  // T's two column-scaled copies over the scratch, and T itself to global
  for (int i = tid; i < C * C; i += kIW) {
    const int r = i / C, c = i - r * C;
    const float t = sA[r * L::LDF + c];
    sTw[r * L::LDC + c] = to_e<E>(t * (sBeta[c] * exp_fast(sGam[c])));
    sTu[r * L::LDC + c] = to_e<E>(t * sBeta[c]);
  }
  store_tile_from_f32<kIW, C, C>(static_cast<T*>(p.akk) + row0 * C, (int64_t)H * C, sA, L::LDF, len);
  __syncthreads();
  rV.store(sV, L::LD);  // over T's FP32 copy, read above
  __syncthreads();

  // ---- W = T Bw, u = T Bv, from the accumulators -------------------------------
  const int rb = wave & 3, ch = wave >> 2;
  const int kend = kceil<E>(16 * rb + 16);  // T is lower triangular
#pragma unroll
  for (int j = 0; j < HCT; ++j) {
    const int ct = ch * HCT + j;
    f32x4 aw = zero4(), au = zero4();
    mma_tile_range<E, ROW, ROW>(aw, sTw, L::LDC, 16 * rb, sK, L::LD, 16 * ct, 0, kend, lane);
    mma_tile_range<E, ROW, ROW>(au, sTu, L::LDC, 16 * rb, sV, L::LD, 16 * ct, 0, kend, lane);
    store_acc_global<T>(static_cast<T*>(p.w) + row0 * D, gs, aw, 16 * rb, 16 * ct, len, lane);
    store_acc_global<T>(static_cast<T*>(p.u) + row0 * D, gs, au, 16 * rb, 16 * ct, len, lane);
  }
}


template <typename T, int D, bool ALIAS, bool WU>
__global__ __launch_bounds__(kIW) void chunk_intra_fwd_kernel(FwdParams p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const ChunkHead wg = chunk_head<true>(p.H);
  if (wg.cid >= p.geom.num_chunks) return;
  const ChunkInfo ci = chunk_info(p.geom, wg.cid);
  if (ci.len == C) intra_fwd_chunk<T, D, ALIAS, WU>(p, ci, C, smem);
  else if (ci.len > 0) intra_fwd_chunk<T, D, ALIAS, WU>(p, ci, ci.len, smem);
}

// ---------------------------------------------------------------------------
// intra-chunk forward, per-channel gate (G [64][D] per chunk).
//   Akk[t,s] = beta_t sum_c k[t,c] kw[s,c] e^{G[t,c]-G[s,c]},  Aqk likewise
//   with s q.  For a block of rows tb and columns sb < tb the decay is split
//   at r = 16 tb - 1, the last row before the row block:
//     e^{G[t]-G[s]} = e^{G[t]-G[r]} e^{G[r]-G[s]},  both factors <= 1,
//   applied to the MFMA operands as they are read (no overflow for any gate).
//   The four diagonal blocks are summed exactly, one (t, s) pair per lane.
//   Also writes qg = s e^G q and kg = e^{G_last - G} kw for the state pass.
// ---------------------------------------------------------------------------
template <typename T, int D, bool ALIAS>
struct IntraPcLayout {
  static constexpr int LD = D + Pad<T>::v;
  static constexpr int LDC = C + Pad<T>::v;
  static constexpr int LDF = C + 4;
  static constexpr int LDG = D + 4;
  static constexpr int RT = C * LD * (int)sizeof(T);
  static constexpr int SCR = 4 * 3 * 16 * SLD * 4;
  static constexpr int QR = RT > SCR ? RT : SCR;
  static constexpr int off_K = 0;                          // K, then Bw, then W
  static constexpr int off_Q = off_K + RT;                 // Q, then solve scratch, then Bv, then u
  static constexpr int off_KW = off_Q + QR;                // KW (when not aliased to K)
  static constexpr int off_G = off_KW + (ALIAS ? 0 : RT);  // fp32 [64][LDG]
  static constexpr int off_A = off_G + C * LDG * 4;        // fp32 [64][LDF]: Akk, then T
  static constexpr int off_Te = off_A + C * LDF * 4;
  static constexpr int off_Aqk = off_Te + C * LDC * (int)sizeof(T);
  static constexpr int off_beta = off_Aqk + C * LDC * (int)sizeof(T);
  // FP32: the gate's FP64 remainder, [64][LDG] (pair decays from hi and lo)
  static constexpr bool GLO = sizeof(T) == 4;
  static constexpr int off_Glo = off_beta + C * 4;
  static constexpr int bytes = off_Glo + (GLO ? C * LDG * 4 : 0);
};

// One chunk's input tiles in registers.  `len` is a literal C for whole
// chunks: the row tests of the loads fold away, so no branch (and no register
// copy inside one) makes a load wait before the next goes out.
template <typename T, int D, bool ALIAS>
struct IntraPcTiles {
  RegTile<kIW, C, D, T> K, Q, KW, V;
  RegTile<kIW, C, D, float> G, Glo;  // Glo: FP32 only, zero without gcum_lo
  float beta;  // of row threadIdx.x % C (clamped into the chunk)
  __device__ __forceinline__ void load(const FwdParams& p, const ChunkInfo& ci, int h, const int len) {
    const int64_t row0 = (int64_t)ci.start * p.H + h;
    const int64_t gs = (int64_t)p.H * D;
    // beta first: its LDS store then waits for this load only
    beta = p.beta[(int64_t)(ci.start + min((int)threadIdx.x & (C - 1), len - 1)) * p.H + h];
    K.load(static_cast<const T*>(p.k) + row0 * D, gs, len);
    Q.load(static_cast<const T*>(p.q) + row0 * D, gs, len);
    if (!ALIAS) KW.load(static_cast<const T*>(p.kw) + row0 * D, gs, len);
    // G rows past the end repeat the last row (G is non-increasing in t, so
    // every split factor stays <= 1 there too)
    G.load_clamped(p.gcum + row0 * D, gs, len);
    if constexpr (sizeof(T) == 4) {
      if (p.gcum_lo) Glo.load_clamped(p.gcum_lo + row0 * D, gs, len);
      else Glo.load(p.gcum + row0 * D, gs, 0);  // zeros
    }
    V.load(static_cast<const T*>(p.v) + row0 * D, gs, len);
  }
};

// The body for one chunk (its tiles' loads already issued).
template <typename T, int D, bool ALIAS>
__device__ __forceinline__ void intra_pc_chunk(const FwdParams& p, const ChunkInfo ci, const int h, const int len,
                                               const IntraPcTiles<T, D, ALIAS>& tiles, char* smem) {
  using L = IntraPcLayout<T, D, ALIAS>;
  using E = T;
  using F = FragK<E>;
  constexpr int HCT = D / 32;
  constexpr int V = Vec16<T>::N;
  const int H = p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t row0 = (int64_t)ci.start * H + h;
  const int64_t gs = (int64_t)H * D;

  E* sK = reinterpret_cast<E*>(smem + L::off_K);
  E* sQ = reinterpret_cast<E*>(smem + L::off_Q);
  E* sKW = ALIAS ? sK : reinterpret_cast<E*>(smem + L::off_KW);
  float* sG = reinterpret_cast<float*>(smem + L::off_G);
  float* sA = reinterpret_cast<float*>(smem + L::off_A);
  E* sTe = reinterpret_cast<E*>(smem + L::off_Te);
  E* sAqk = reinterpret_cast<E*>(smem + L::off_Aqk);
  float* sBeta = reinterpret_cast<float*>(smem + L::off_beta);

  sBeta[tid & (C - 1)] = (tid & (C - 1)) < len ? tiles.beta : 0.f;  // every thread: no branch
  // V waits in registers until Q's slot frees
  tiles.K.store(sK, L::LD);
  tiles.Q.store(sQ, L::LD);
  if (!ALIAS) tiles.KW.store(sKW, L::LD);
  tiles.G.store(sG, L::LDG);
  float* sGlo = reinterpret_cast<float*>(smem + L::off_Glo);
  if constexpr (L::GLO) tiles.Glo.store(sGlo, L::LDG);
  // G[a] - G[b] at column c; FP32 adds the remainders' difference, so a
  // difference of two large cumsums carries only its own rounding
  auto gd = [&](int a, int b, int c) {
    float d = sG[a * L::LDG + c] - sG[b * L::LDG + c];
    if constexpr (L::GLO) d += sGlo[a * L::LDG + c] - sGlo[b * L::LDG + c];
    return d;
  };
  const RegTile<kIW, C, D, T>& rV = tiles.V;
  for (int i = tid; i < C * C; i += kIW) {
    const int r = i / C, c = i - r * C;
    sA[r * L::LDF + c] = 0.f;
    sAqk[r * L::LDC + c] = to_e<E>(0.f);
  }
  __syncthreads();

  // ---- diagonal blocks, exactly: one (t, s) pair, s <= t, per lane -----------
  // The 4 x 136 pairs are numbered block by block.  Every wave takes pairs
  // lane + 64 wave (0..511); waves 2-7 then take one off-diagonal block each
  // and wave 0 the last 32 pairs, each split over two lanes (channels 0-63
  // and 64-127, summed by a lane exchange), so no wave carries more than one
  // pair pass and one block's worth of work.
  auto pair_of = [&](int pg, int& t, int& s) {
    const int tb = pg / 136;
    int tl = 0, rest = pg - tb * 136;
    while (rest > tl) {
      rest -= tl + 1;
      ++tl;
    }
    t = 16 * tb + tl;
    s = 16 * tb + rest;
  };
  auto pair_sums = [&](int t, int s, int c0, int c1, float& akk, float& aqk) {
    akk = 0.f;
    aqk = 0.f;
    for (int c = c0; c < c1; c += V) {
      float kx[V], qx[V], wx[V];
      lds_vec<V>(sK + t * L::LD + c, kx);
      lds_vec<V>(sQ + t * L::LD + c, qx);
      lds_vec<V>(sKW + s * L::LD + c, wx);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float e = exp_fast(gd(t, s, c + j));
        akk += kx[j] * wx[j] * e;
        aqk += qx[j] * wx[j] * e;
      }
    }
  };
  auto pair_store = [&](int t, int s, float akk, float aqk) {
    sA[t * L::LDF + s] = (s < t && t < len) ? sBeta[t] * akk : 0.f;
    sAqk[t * L::LDC + s] = to_e<E>(t < len ? p.scale * aqk : 0.f);
  };
  {
    int t, s;
    float akk, aqk;
    pair_of(lane + 64 * wave, t, s);
    pair_sums(t, s, 0, D, akk, aqk);
    pair_store(t, s, akk, aqk);
  }
  if (wave == 0) {
    int t, s;
    float akk, aqk;
    pair_of(512 + (lane & 31), t, s);
    const int half = lane >> 5;
    pair_sums(t, s, half * (D / 2), (half + 1) * (D / 2), akk, aqk);
    akk += __shfl_xor(akk, 32);
    aqk += __shfl_xor(aqk, 32);
    if (half == 0) pair_store(t, s, akk, aqk);
  } else if (wave >= 2) {
    // ---- off-diagonal blocks (tb > sb) with the split decay --------------------
    const int blk = wave - 2;
    const int tb = blk < 1 ? 1 : blk < 3 ? 2 : 3;
    const int sb = blk - (tb - 1) * tb / 2;
    const int r = 16 * tb - 1;
    const int t = 16 * tb + (lane & 15), s = 16 * sb + (lane & 15);
    f32x4 akk = zero4(), aqk = zero4();
    for (int k0 = 0; k0 < D; k0 += Mma<E>::KS) {
      const int kk = k0 + F::off(lane);
      float ak[F::N], aq[F::N], bw[F::N];
#pragma unroll
      for (int j = 0; j < F::N; ++j) {
        const float fa = exp_fast(gd(t, r, kk + j));
        const float fb = exp_fast(gd(r, s, kk + j));
        ak[j] = from_e<E>(sK[t * L::LD + kk + j]) * fa;
        aq[j] = from_e<E>(sQ[t * L::LD + kk + j]) * fa;
        bw[j] = from_e<E>(sKW[s * L::LD + kk + j]) * fb;
      }
      F::mfma(akk, ak, bw);
      F::mfma(aqk, aq, bw);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int tt = 16 * tb + acc_row(lane, e), ss = 16 * sb + acc_col(lane);
      sA[tt * L::LDF + ss] = tt < len ? sBeta[tt] * akk[e] : 0.f;
      sAqk[tt * L::LDC + ss] = to_e<E>(tt < len ? p.scale * aqk[e] : 0.f);
    }
  }
  // ---- qg = s e^G q and kg = e^{G_last - G} kw, straight to global -----------
  T* qg_out = static_cast<T*>(p.qg) + row0 * D;
  T* kg_out = static_cast<T*>(p.kg) + row0 * D;
  for (int i = tid; i < C * (D / V); i += kIW) {
    const int r = i / (D / V), c = (i - r * (D / V)) * V;
    if (r < len) {
      float qx[V], wx[V];
      lds_vec<V>(sQ + r * L::LD + c, qx);
      lds_vec<V>(sKW + r * L::LD + c, wx);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        qx[j] *= p.scale * exp_fast(sG[r * L::LDG + c + j]);
        wx[j] *= exp_fast(gd(C - 1, r, c + j));
      }
      store_vec<V>(qg_out + r * gs + c, qx);
      store_vec<V>(kg_out + r * gs + c, wx);
    }
  }
  __syncthreads();

  // ---- T = (I + Akk)^-1 in place; Aqk leaves meanwhile ------------------------
  store_tile<kIW, C, C>(static_cast<T*>(p.aqk) + row0 * C, (int64_t)H * C, sAqk, L::LDC, len);
  solve_unit_lower_64(sA, L::LDF, reinterpret_cast<float*>(sQ));
  for (int i = tid; i < C * C; i += kIW) {
    const int r = i / C, c = i - r * C;
    sTe[r * L::LDC + c] = to_e<E>(sA[r * L::LDF + c]);
  }
  // Bw = diag(beta) (e^G * K) in place over K; Bv = diag(beta) V over Q
  for (int i = tid; i < C * D; i += kIW) {
    const int r = i / D, c = i - r * D;
    sK[r * L::LD + c] = to_e<E>(sBeta[r] * exp_fast(sG[r * L::LDG + c]) * from_e<E>(sK[r * L::LD + c]));
  }
  rV.store(sQ, L::LD, RowScale{sBeta});
  __syncthreads();
  store_tile<kIW, C, C>(static_cast<T*>(p.akk) + row0 * C, (int64_t)H * C, sTe, L::LDC, len);

  const int rb = wave & 3, ch = wave >> 2;
  const int kend = kceil<E>(16 * rb + 16);
  f32x4 aw[HCT], au[HCT];
#pragma unroll
  for (int j = 0; j < HCT; ++j) {
    const int ct = ch * HCT + j;
    aw[j] = zero4();
    au[j] = zero4();
    mma_tile_range<E, ROW, ROW>(aw[j], sTe, L::LDC, 16 * rb, sK, L::LD, 16 * ct, 0, kend, lane);
    mma_tile_range<E, ROW, ROW>(au[j], sTe, L::LDC, 16 * rb, sQ, L::LD, 16 * ct, 0, kend, lane);
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < HCT; ++j) {
    const int ct = ch * HCT + j;
    store_acc_lds(sK, L::LD, aw[j], 16 * rb, 16 * ct, lane);
    store_acc_lds(sQ, L::LD, au[j], 16 * rb, 16 * ct, lane);
  }
  __syncthreads();
  store_tile<kIW, C, D>(static_cast<T*>(p.w) + row0 * D, gs, sK, L::LD, len);
  store_tile<kIW, C, D>(static_cast<T*>(p.u) + row0 * D, gs, sQ, L::LD, len);
}

template <typename T, int D, bool ALIAS>
__device__ __forceinline__ void intra_pc_run(const FwdParams& p, const ChunkInfo& ci, const int h, const int len,
                                             char* smem) {
  IntraPcTiles<T, D, ALIAS> tiles;
  tiles.load(p, ci, h, len);
  intra_pc_chunk<T, D, ALIAS>(p, ci, h, len, tiles, smem);
}

template <typename T, int D, bool ALIAS>
__global__ __launch_bounds__(kIW) void chunk_intra_fwd_pc_kernel(FwdParams p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const ChunkHead wg = chunk_head<false>(p.H);
  if (wg.cid >= p.geom.num_chunks) return;
  const ChunkInfo ci = chunk_info(p.geom, wg.cid);
  if (ci.len == C) intra_pc_run<T, D, ALIAS>(p, ci, wg.h, C, smem);
  else if (ci.len > 0) intra_pc_run<T, D, ALIAS>(p, ci, wg.h, ci.len, smem);
}

// ---------------------------------------------------------------------------
// The same, BF16 at head_dim 128, with the channels in two halves of 64 so
// that a workgroup needs ~72 KB of LDS and two share a compute unit (one
// workgroup's loads then overlap the other's products).  Every contraction
// over the channels (the pair sums of Akk and Aqk) accumulates in registers
// across the halves; qg, kg and the column blocks of W = T Bw and u = T Bv
// are per half.  The second half's tiles are loaded while the first half
// computes, and W's first column block takes Bw = diag(beta) (e^G * K) of
// the first half, formed while that half's K and G are in LDS and kept in a
// region of its own (not loaded a second time).
// ---------------------------------------------------------------------------
template <bool ALIAS>
struct IntraPc2Layout {
  static constexpr int DH = 64;                 // channels per half
  static constexpr int LD = DH + Pad<bf16_t>::v;
  static constexpr int LDG = DH + 4;
  static constexpr int LDC = C + Pad<bf16_t>::v;
  static constexpr int LDF = C + 4;
  static constexpr int RT = C * LD * 2;         // a bf16 half tile
  static constexpr int SCR = 4 * 3 * 16 * SLD * 4;
  static constexpr int QR = ALIAS ? (RT > SCR ? RT : SCR) : RT;
  static constexpr int off_K = 0;                          // K half, then Bw half
  static constexpr int off_Q = off_K + RT;                 // Q half, then solve scratch (with KW), then Bv half
  static constexpr int off_KW = off_Q + QR;                // KW half (when not aliased to K)
  static constexpr int off_G = off_KW + (ALIAS ? 0 : RT);  // fp32 [64][LDG] half of G, times log2 e
  static constexpr int off_A = off_G + C * LDG * 4;        // fp32 [64][LDF]: Akk, then T
  static constexpr int off_Aqk = off_A + C * LDF * 4;      // bf16 Aqk, then T
  static constexpr int off_beta = off_Aqk + C * LDC * 2;
  static constexpr int off_Bw0 = off_beta + C * 4;         // bf16 Bw of the first half (W's first block)
  static constexpr int bytes = off_Bw0 + RT;
  static_assert(ALIAS || QR + RT >= SCR, "the solve's scratch fits the Q and KW regions");
  static_assert(2 * bytes <= 160 * 1024, "two workgroups per compute unit");
};

template <bool ALIAS>
__device__ __forceinline__ void intra_pc2_chunk(const FwdParams& p, const ChunkInfo ci, const int h, const int len,
                                                char* smem) {
  using L = IntraPc2Layout<ALIAS>;
  using T = bf16_t;
  using E = T;
  using F = FragK<E>;
  constexpr int D = 128, DH = L::DH;
  constexpr int V = Vec16<T>::N;
  const int H = p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t row0 = (int64_t)ci.start * H + h;
  const int64_t gs = (int64_t)H * D;

  E* sK = reinterpret_cast<E*>(smem + L::off_K);
  E* sQ = reinterpret_cast<E*>(smem + L::off_Q);
  E* sKW = ALIAS ? sK : reinterpret_cast<E*>(smem + L::off_KW);
  float* sG = reinterpret_cast<float*>(smem + L::off_G);
  float* sA = reinterpret_cast<float*>(smem + L::off_A);
  E* sAqk = reinterpret_cast<E*>(smem + L::off_Aqk);
  E* sTe = sAqk;
  float* sBeta = reinterpret_cast<float*>(smem + L::off_beta);
  E* sBw0 = reinterpret_cast<E*>(smem + L::off_Bw0);

  const T* k = static_cast<const T*>(p.k) + row0 * D;
  const T* q = static_cast<const T*>(p.q) + row0 * D;
  const T* kw = static_cast<const T*>(p.kw) + row0 * D;
  const float* g = p.gcum + row0 * D;

  // the first half's tiles (beta first: its LDS store waits for it only); G
  // rows past the end repeat the last row, so every split factor stays <= 1.
  // Each later tile set is loaded one phase ahead of its use: with two
  // workgroups per compute unit the other one covers the wait, and the
  // registers stay within the 128 of four waves per SIMD.
  const float bval = p.beta[(int64_t)(ci.start + min(tid & (C - 1), len - 1)) * H + h];
  {
    RegTile<kIW, C, DH, T> K0, Q0, KW0;
    RegTile<kIW, C, DH, float> G0;
    K0.load(k, gs, len);
    Q0.load(q, gs, len);
    if (!ALIAS) KW0.load(kw, gs, len);
    G0.load_clamped(g, gs, len);
    sBeta[tid & (C - 1)] = (tid & (C - 1)) < len ? bval : 0.f;  // every thread: no branch
    K0.store(sK, L::LD);
    Q0.store(sQ, L::LD);
    if (!ALIAS) KW0.store(sKW, L::LD);
    G0.scale(kLog2e);
    G0.store(sG, L::LDG);
  }
#pragma unroll 1
  for (int i = tid; i < C * C; i += kIW) {
    const int r = i / C, c = i - r * C;
    sA[r * L::LDF + c] = 0.f;
    sAqk[r * L::LDC + c] = to_e<E>(0.f);
  }

  // the pair sums over one half's channels, accumulated in registers:
  // diagonal blocks exactly (one (t, s) pair, s <= t, per lane: the 4 x 136
  // pairs numbered block by block, every wave taking pairs lane + 64 wave and
  // wave 0 also the last 32, split over two lanes), the off-diagonal blocks
  // (tb > sb, waves 2-7, one each) on MFMA with the decay split at the row
  // before the row block
  auto pair_of = [&](int pg, int& t, int& s) {
    const int tb = pg / 136;
    int tl = 0, rest = pg - tb * 136;
    while (rest > tl) {
      rest -= tl + 1;
      ++tl;
    }
    t = 16 * tb + tl;
    s = 16 * tb + rest;
  };
  // (eight VALU operations per pair and channel: three widenings, the
  // difference, exp2 of it (G is staged times log2 e), w e^(G_t - G_s) once for
  // both sums, two FMAs; unrolled four pieces deep: fully unrolled, the loads
  // hoisted ahead take every register and spill)
  auto pair_sums = [&](int t, int s, int c0, int c1, float& akk, float& aqk) {
#pragma unroll 4
    for (int c = c0; c < c1; c += V) {
      float kx[V], qx[V], wx[V];
      lds_vec<V>(sK + t * L::LD + c, kx);
      lds_vec<V>(sQ + t * L::LD + c, qx);
      lds_vec<V>(sKW + s * L::LD + c, wx);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float we = wx[j] * exp2_fast(sG[t * L::LDG + c + j] - sG[s * L::LDG + c + j]);
        akk = __builtin_fmaf(kx[j], we, akk);
        aqk = __builtin_fmaf(qx[j], we, aqk);
      }
    }
  };
  const int xh = lane >> 5;  // wave 0's extra pairs: this lane's 32 channels of each half
  float akk1 = 0.f, aqk1 = 0.f, akk2 = 0.f, aqk2 = 0.f;
  const int blk = wave - 2;
  const int tb = blk < 1 ? 1 : blk < 3 ? 2 : 3;
  const int sb = blk - (tb - 1) * tb / 2;
  f32x4 akk4 = zero4(), aqk4 = zero4();
  T* qg_out = static_cast<T*>(p.qg) + row0 * D;
  T* kg_out = static_cast<T*>(p.kg) + row0 * D;

  auto half_pass = [&](int hc) {  // the half of channels [hc, hc + DH) is in LDS
    {  // (pair indices recomputed where used: nothing held across the passes)
      int t1, s1;
      pair_of(lane + 64 * wave, t1, s1);
      pair_sums(t1, s1, 0, DH, akk1, aqk1);
    }
    if (wave == 0) {
      int t2, s2;
      pair_of(512 + (lane & 31), t2, s2);
      pair_sums(t2, s2, xh * (DH / 2), (xh + 1) * (DH / 2), akk2, aqk2);
    } else if (wave >= 2) {
      const int r = 16 * tb - 1;
      const int t = 16 * tb + (lane & 15), s = 16 * sb + (lane & 15);
#pragma unroll
      for (int k0 = 0; k0 < DH; k0 += Mma<E>::KS) {
        const int kk = k0 + F::off(lane);
        float ak[F::N], aq[F::N], bw[F::N];
#pragma unroll
        for (int j = 0; j < F::N; ++j) {
          const float gr = sG[r * L::LDG + kk + j];
          const float fa = exp2_fast(sG[t * L::LDG + kk + j] - gr);
          const float fb = exp2_fast(gr - sG[s * L::LDG + kk + j]);
          ak[j] = from_e<E>(sK[t * L::LD + kk + j]) * fa;
          aq[j] = from_e<E>(sQ[t * L::LD + kk + j]) * fa;
          bw[j] = from_e<E>(sKW[s * L::LD + kk + j]) * fb;
        }
        F::mfma(akk4, ak, bw);
        F::mfma(aqk4, aq, bw);
      }
    }
    // qg = s e^G q and kg = e^{G_last - G} kw of this half, straight to global
    {
      const int r = tid / (DH / V), c = (tid % (DH / V)) * V;  // C x DH / V = kIW pieces: one per thread
      if (r < len) {
        float qx[V], wx[V];
        lds_vec<V>(sQ + r * L::LD + c, qx);
        lds_vec<V>(sKW + r * L::LD + c, wx);
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const float gv = sG[r * L::LDG + c + j];
          qx[j] *= p.scale * exp2_fast(gv);
          wx[j] *= exp2_fast(sG[(C - 1) * L::LDG + c + j] - gv);
        }
        store_vec<V>(qg_out + r * gs + hc + c, qx);
        store_vec<V>(kg_out + r * gs + hc + c, wx);
      }
    }
  };
  static_assert(C * (DH / V) == kIW, "one qg / kg piece per thread and half");

  // ---- first half (the second half's loads go out first) -------------------------
  {
    RegTile<kIW, C, DH, T> K1, Q1, KW1;
    RegTile<kIW, C, DH, float> G1;
    __syncthreads();
    half_pass(0);
    K1.load(k + DH, gs, len);
    Q1.load(q + DH, gs, len);
    if (!ALIAS) KW1.load(kw + DH, gs, len);
    G1.load_clamped(g + DH, gs, len);
    // W's first column block takes Bw = beta e^G K of this half: formed while
    // its K and G are in LDS (the second half's tiles replace them next)
#pragma unroll 1
    for (int i = tid; i < C * DH; i += kIW) {
      const int r = i / DH, c = i - r * DH;
      sBw0[r * L::LD + c] = to_e<E>(sBeta[r] * exp2_fast(sG[r * L::LDG + c]) * from_e<E>(sK[r * L::LD + c]));
    }
    __syncthreads();
    // ---- second half -----------------------------------------------------------
    K1.store(sK, L::LD);
    Q1.store(sQ, L::LD);
    if (!ALIAS) KW1.store(sKW, L::LD);
    G1.scale(kLog2e);
    G1.store(sG, L::LDG);
  }
  __syncthreads();
  half_pass(DH);
  // ---- Akk and Aqk from the registers --------------------------------------------
  {
    auto pair_store = [&](int t, int s, float akk, float aqk) {
      sA[t * L::LDF + s] = (s < t && t < len) ? sBeta[t] * akk : 0.f;
      sAqk[t * L::LDC + s] = to_e<E>(t < len ? p.scale * aqk : 0.f);
    };
    int t1, s1;
    pair_of(lane + 64 * wave, t1, s1);
    pair_store(t1, s1, akk1, aqk1);
    if (wave == 0) {
      akk2 += __shfl_xor(akk2, 32);
      aqk2 += __shfl_xor(aqk2, 32);
      int t2, s2;
      pair_of(512 + (lane & 31), t2, s2);
      if (xh == 0) pair_store(t2, s2, akk2, aqk2);
    } else if (wave >= 2) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int tt = 16 * tb + acc_row(lane, e), ss = 16 * sb + acc_col(lane);
        sA[tt * L::LDF + ss] = tt < len ? sBeta[tt] * akk4[e] : 0.f;
        sAqk[tt * L::LDC + ss] = to_e<E>(tt < len ? p.scale * aqk4[e] : 0.f);
      }
    }
  }
  __syncthreads();
  // ---- T = (I + Akk)^-1 in place (scratch over Q and KW); Aqk leaves first ------
  store_tile<kIW, C, C>(static_cast<T*>(p.aqk) + row0 * C, (int64_t)H * C, sAqk, L::LDC, len);
  solve_unit_lower_64(sA, L::LDF, reinterpret_cast<float*>(sQ));
  // u's operand V (both halves)
  RegTile<kIW, C, D, T> rV;
  rV.load(static_cast<const T*>(p.v) + row0 * D, gs, len);
  // (loops over the tile not unrolled: hoisted addresses would be held, and
  // spilled, across the phases)
#pragma unroll 1
  for (int i = tid; i < C * C; i += kIW) {  // T in bf16 over Aqk (its reads ended before the solve's barriers)
    const int r = i / C, c = i - r * C;
    sTe[r * L::LDC + c] = to_e<E>(sA[r * L::LDF + c]);
  }
  // ---- W = T Bw and u = T Bv, column half by column half -------------------------
  // Bw = diag(beta) (e^G * K), Bv = diag(beta) V; the second half's Bw is
  // formed in place over its K (still in LDS), the first half's is sBw0
  const int rb = wave & 3, ch = wave >> 2;
  const int kend = kceil<E>(16 * rb + 16);
  T* w_out = static_cast<T*>(p.w) + row0 * D;
  T* u_out = static_cast<T*>(p.u) + row0 * D;
  auto wu_half = [&](int hc, E* sBw) {
    if (hc == DH) {
#pragma unroll 1
      for (int i = tid; i < C * DH; i += kIW) {
        const int r = i / DH, c = i - r * DH;
        sK[r * L::LD + c] = to_e<E>(sBeta[r] * exp2_fast(sG[r * L::LDG + c]) * from_e<E>(sK[r * L::LD + c]));
      }
    }
    // this half's V columns from the register tile (pieces of 8 columns)
#pragma unroll
    for (int i = 0; i < RegTile<kIW, C, D, T>::ITER; ++i) {
      const int idx = tid + i * kIW;
      const int r = idx / (D / V), c = (idx % (D / V)) * V;
      if (c >= hc && c < hc + DH) {
        float x[V];
        Vec16<T>::unpack(rV.r[i], x);
#pragma unroll
        for (int j = 0; j < V; ++j) x[j] *= sBeta[r];
        store_vec<V>(sQ + r * L::LD + c - hc, x);
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < DH / 32; ++j) {
      const int ct = ch * (DH / 32) + j;  // column tile within the half
      f32x4 aw = zero4(), au = zero4();
      mma_tile_range<E, ROW, ROW>(aw, sTe, L::LDC, 16 * rb, sBw, L::LD, 16 * ct, 0, kend, lane);
      mma_tile_range<E, ROW, ROW>(au, sTe, L::LDC, 16 * rb, sQ, L::LD, 16 * ct, 0, kend, lane);
      store_acc_global<T>(w_out, gs, aw, 16 * rb, hc + 16 * ct, len, lane);
      store_acc_global<T>(u_out, gs, au, 16 * rb, hc + 16 * ct, len, lane);
    }
  };
  wu_half(DH, sK);
  __syncthreads();  // every wave is done with the second half's Bv
  wu_half(0, sBw0);
  store_tile<kIW, C, C>(static_cast<T*>(p.akk) + row0 * C, (int64_t)H * C, sTe, L::LDC, len);
}

template <bool ALIAS>
__global__ __launch_bounds__(kIW, 4) void chunk_intra_fwd_pc2_kernel(FwdParams p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const ChunkHead wg = chunk_head<false>(p.H);
  if (wg.cid >= p.geom.num_chunks) return;
  const ChunkInfo ci = chunk_info(p.geom, wg.cid);
  if (ci.len == C) intra_pc2_chunk<ALIAS>(p, ci, wg.h, C, smem);
  else if (ci.len > 0) intra_pc2_chunk<ALIAS>(p, ci, wg.h, ci.len, smem);
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
  static constexpr int off_gc = off_gam + C * 4;                      // [D] last-row G (per channel)
  static constexpr int bytes = off_gc + D * 4;
};

// PC: per-channel gate.  The forward intra kernel wrote qg = s e^G q and
// kg = e^{G_last - G} kw, so no row scaling applies and S decays row by row.
template <typename T, int D, int BV, bool PC>
__global__ __launch_bounds__(state_threads(D, BV)) void chunk_state_fwd_kernel(FwdParams p) {
  using L = StateLayout<T, D, BV>;
  using E = T;
  constexpr int kSW = state_threads(D, BV);
  constexpr int NW = kSW / 64;
  constexpr int NCT = BV / 16;              // column tiles of the slice
  constexpr int NS = (D / 16) * NCT / NW;   // state tiles per wave
  constexpr int NRT = 4 * NCT;              // 16x16 tiles of a [64 x BV] chunk operand
  static_assert(NS * NW == (D / 16) * NCT, "state tiles split evenly over the waves");
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
  float* sGC = reinterpret_cast<float*>(smem + L::off_gc);

  const DocSlot ds = doc_slot(p.geom, p.H, D / BV);
  const int n = ds.n, h = ds.h, v0 = ds.z * BV;
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
      S[i][j] = p.s0 ? p.s0[(state_row(p, n) * H + h) * D * D + r * D + c] : 0.f;
    }
  }

  RegTile<kSW, C, D, T> rW, rQ, rKW;
  RegTile<kSW, C, C, T> rA;
  RegTile<kSW, C, BV, T> rU;
  float rg = 0.f;
  auto prefetch = [&](int jc) {
    const int cstart = dstart + jc * C;
    const int clen = min(C, dlen - jc * C);
    const int64_t row0 = (int64_t)cstart * H + h;
    rW.load(static_cast<const T*>(p.w) + row0 * D, gs, clen);
    rQ.load(static_cast<const T*>(PC ? p.qg : p.q) + row0 * D, gs, clen);
    rKW.load(static_cast<const T*>(PC ? p.kg : p.kw) + row0 * D, gs, clen);
    rA.load(static_cast<const T*>(p.aqk) + row0 * C, (int64_t)H * C, clen);
    rU.load(static_cast<const T*>(p.u) + row0 * D + v0, gs, clen);
    if (PC) {
      if (tid < D) rg = p.gcum[((int64_t)(cstart + clen - 1) * H + h) * D + tid];
    } else if (tid < C) {
      rg = p.gcum[(int64_t)(cstart + min(tid, clen - 1)) * H + h];
    }
  };
  if (count > 0) prefetch(0);
  const float scale = p.scale;

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
    if (PC) {
      if (tid < D) sGC[tid] = rg;
    } else if (tid < C) {
      sGam[tid] = rg;
    }
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int ti = wave * NS + i;
      const int rt = ti / NCT, ct = ti % NCT;
      store_acc_lds(sS, L::LDV, S[i], 16 * rt, 16 * ct, lane);
      if (p.h) {
        T* hb = static_cast<T*>(p.h) + ((int64_t)cid * H + h) * D * D;
        store_acc_tile(hb + tile_offset(D, rt, v0 / 16 + ct), S[i], lane);
      }
    }
    __syncthreads();
    if (jc + 1 < count) prefetch(jc + 1);
    const float gC = PC ? 0.f : sGam[C - 1];  // padded rows repeat the last valid gate
    // U = u - W S      (tile ti: row block ti % 4, column tile ti / 4)
    T* u_io = static_cast<T*>(p.u) + row0 * D + v0;
#pragma unroll
    for (int ti = wave; ti < NRT; ti += NW) {
      const int r0 = 16 * (ti & 3), ct = ti >> 2;
      f32x4 acc = zero4();
      mma_tile<E, ROW, ROW>(acc, sW, L::LD, r0, sS, L::LDV, 16 * ct, D, lane);
      f32x4 U;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = r0 + acc_row(lane, e), c = 16 * ct + acc_col(lane);
        U[e] = from_e<E>(sUin[r * L::LDV + c]) - acc[e];
        sU[r * L::LDV + c] = to_e<E>(U[e]);
        if (!PC) sUg[r * L::LDV + c] = to_e<E>(exp_fast(gC - sGam[r]) * U[e]);
      }
      store_acc_global<T>(u_io, gs, U, r0, 16 * ct, clen, lane);
    }
    __syncthreads();
    // O = diag(s e^G) Q S + Aqk U
    T* o_out = static_cast<T*>(p.o) + row0 * D + v0;
#pragma unroll
    for (int ti = wave; ti < NRT; ti += NW) {
      const int r0 = 16 * (ti & 3), ct = ti >> 2;
      const int kend = kceil<E>(r0 + 16);  // Aqk is lower triangular
      f32x4 a1 = zero4(), a2 = zero4();
      mma_tile<E, ROW, ROW>(a1, sQ, L::LD, r0, sS, L::LDV, 16 * ct, D, lane);
      mma_tile_range<E, ROW, ROW>(a2, sAqk, L::LDC, r0, sU, L::LDV, 16 * ct, 0, kend, lane);
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (PC ? 1.f : scale * exp_fast(sGam[r0 + acc_row(lane, e)])) * a1[e] + a2[e];
      store_acc_global<T>(o_out, gs, o, r0, 16 * ct, clen, lane);
    }
    // S <- e^{G_C} S + KW^T Ug   (per-channel: diag(e^{G_C}) S + kg^T U)
    const float decay = exp_fast(gC);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int ti = wave * NS + i;
      const int rt = ti / NCT, ct = ti % NCT;
      if (PC) {
#pragma unroll
        for (int j = 0; j < 4; ++j) S[i][j] *= exp_fast(sGC[16 * rt + acc_row(lane, j)]);
      } else {
        S[i] = S[i] * decay;
      }
      mma_tile<E, COL, ROW>(S[i], sKW, L::LD, 16 * rt, PC ? sU : sUg, L::LDV, 16 * ct, C, lane);
    }
    __syncthreads();
  }
  if (p.sT) {
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int ti = wave * NS + i;
      const int rt = ti / NCT, ct = ti % NCT;
      float* sb = p.sT + (state_row(p, n) * H + h) * D * D + v0;
      store_acc_global<float>(sb, D, S[i], 16 * rt, 16 * ct, D, lane);
    }
  }
}

// ---------------------------------------------------------------------------
// per-document state pass, BF16 with a per-head gate: register-resident form
//
// One workgroup per (document, head, BV value columns): BV/16 compute waves,
// each owning 16 value columns, and kRrLoaders loader waves.  A compute wave
// keeps its S [D x 16] slice in MFMA accumulators and the chunk's U [64 x 16]
// in registers; both feed the next products directly as B operands (the k
// order of pack_acc_pair), so a chunk has no LDS round trip of S or U and no
// barrier between its products.  W = T diag(beta e^G) K and u = T diag(beta) V
// are never formed; with Y the prediction error of the chunk,
//   Y = diag(beta) (V - diag(e^G) (K S)),   U = T Y   (= u - W S),
//   O = diag(s e^G)(Q S) + Aqk U,
//   S <- e^{G_C} S + KW^T diag(e^{G_C - G}) U.
// Reading T (64 x 64) and the V slice costs fewer bytes than W (64 x D) and
// the u slice, and the intra pass writes neither.
// The loader waves move each chunk's read-only tiles (Q, KW, K when it is not
// KW, Aqk, T, the V slice, G and beta) from global memory into a
// double-buffered LDS stage one chunk ahead.  They form two groups that take
// alternate chunks, each holding one chunk in registers, so two chunks' loads
// are in flight while one chunk computes and each wave only ever waits for its
// own loads (never for a compute wave's stores).  One barrier per chunk.
// ---------------------------------------------------------------------------
constexpr int kRrLoaders = 4;  // two groups of two waves

template <int D, int BV, bool ALIAS>
struct RrFwdLayout {  // (PACK kernels: Aqk and T come packed, see TriRegTile)
  static constexpr int LD = D + Pad<bf16_t>::v;
  static constexpr int LDV = BV + Pad<bf16_t>::v;
  static constexpr int LDC = C + Pad<bf16_t>::v;
  static constexpr int off_Q = 0;
  static constexpr int off_KW = off_Q + C * LD * 2;
  static constexpr int off_K = off_KW + C * LD * 2;               // K when it is not KW
  static constexpr int off_A = off_K + (ALIAS ? 0 : C * LD * 2);  // Aqk
  static constexpr int off_T = off_A + C * LDC * 2;
  static constexpr int off_V = off_T + C * LDC * 2;
  static constexpr int off_G = off_V + C * LDV * 2;
  static constexpr int off_B = off_G + C * 4;                     // beta (0 past the chunk's end)
  static constexpr int BUF = off_B + C * 4;
  // Output stage (where it fits): the compute waves leave each chunk's U and
  // O rows here, double-buffered, and the loader group that is not staging
  // inputs in that step writes them to global memory, so the compute waves
  // issue no global stores for them.
  static constexpr int OUT = 2 * C * LDV * 2;  // U, then O
  static constexpr bool STAGE_OUT = 2 * BUF + 2 * OUT <= 160 * 1024;
  static constexpr int off_Out = 2 * BUF;
  static constexpr int bytes = 2 * BUF + (STAGE_OUT ? 2 * OUT : 0);
  static_assert(BUF % 16 == 0 && (LDV * 2) % 16 == 0, "16-byte aligned stages and rows");
  static_assert(bytes <= 160 * 1024, "LDS of one compute unit");
};

template <int D, int BV, bool ALIAS, bool PACK>
__global__ __launch_bounds__(64 * (BV / 16 + kRrLoaders)) void chunk_state_fwd_rr_kernel(FwdParams p) {
  using L = RrFwdLayout<D, BV, ALIAS>;
  using T = bf16_t;
  constexpr int NC = BV / 16;           // compute waves
  constexpr int NKT = D / 16;           // 16-row tiles of the state slice
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const DocSlot ds = doc_slot(p.geom, p.H, D / BV);
  const int n = ds.n, h = ds.h, v0 = ds.z * BV;
  const int H = p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t gs = (int64_t)H * D;
  int first, count, dstart, dlen;
  doc_chunks(p.geom, n, first, count, dstart, dlen);
  const bool loader = wave >= NC;
  constexpr int NGT = 64 * kRrLoaders / 2;         // threads of one loader group
  const int lgroup = (tid - 64 * NC) / NGT;        // loader group: chunks jc with jc % 2 == lgroup
  const int lt = (tid - 64 * NC) % NGT;

  if (loader) {
    // The two roles run separate loops with the same barriers, so neither
    // keeps the other's registers live.
    RegTile<NGT, C, D, T> rQ, rKW, rK;
    std::conditional_t<PACK, TriRegTile<NGT>, RegTile<NGT, C, C, T>> rA, rT;
    RegTile<NGT, C, BV, T> rV;
    float rg = 0.f, rb = 0.f;
    if constexpr (PACK) {  // the stages' blocks above the diagonal: zero once
      const int lt2 = tid - 64 * NC;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        zero_upper_blocks<2 * NGT>(lt2, reinterpret_cast<T*>(smem + b * L::BUF + L::off_A), L::LDC);
        zero_upper_blocks<2 * NGT>(lt2, reinterpret_cast<T*>(smem + b * L::BUF + L::off_T), L::LDC);
      }
    }
    auto load = [&](int jc) {
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
      rV.load_as(lt, static_cast<const T*>(p.v) + row0 * D + v0, gs, clen);
      if (lt < C) {
        const int64_t gi = (int64_t)(cstart + min(lt, clen - 1)) * H + h;
        rg = p.gcum[gi];  // padded rows repeat the last gate
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
      rV.store_as(lt, reinterpret_cast<T*>(buf + L::off_V), L::LDV);
      if (lt < C) {
        reinterpret_cast<float*>(buf + L::off_G)[lt] = rg;
        reinterpret_cast<float*>(buf + L::off_B)[lt] = rb;
      }
    };
    // chunk jc's U and O rows from the output stage to global memory
    auto flush = [&](int jc) {
      constexpr int SEG = BV / 8;  // 16-byte pieces of a row
      const T* so = reinterpret_cast<const T*>(smem + L::off_Out + (jc & 1) * L::OUT);
      const int clen = min(C, dlen - jc * C);
      const int64_t row0 = (int64_t)(dstart + jc * C) * H + h;
      static_assert(2 * C * SEG % NGT == 0, "whole passes over the stage");
#pragma unroll
      for (int it = 0; it < 2 * C * SEG / NGT; ++it) {
        const int i = lt + it * NGT;
        const int which = i / (C * SEG);
        const int r = (i - which * C * SEG) / SEG, sg = i % SEG;
        if (r < clen) {
          const uint4 x = *reinterpret_cast<const uint4*>(so + (which * C + r) * L::LDV + 8 * sg);
          T* dst = static_cast<T*>(which ? p.o : p.u) + (row0 + (int64_t)r * H) * D + v0 + 8 * sg;
          *reinterpret_cast<uint4*>(dst) = x;
        }
      }
    };
    // group g holds chunks g, g + 2, ...; chunk 0 is staged before the loop
    if (lgroup < count) load(lgroup);
    if (lgroup == 0 && count > 0) {
      stash(0);
      if (count > 2) load(2);
    }
    for (int jc = 0; jc < count; ++jc) {
      __syncthreads();
      if (((jc + 1) & 1) == lgroup) {
        if (jc + 1 < count) {
          stash((jc + 1) & 1);
          if (jc + 3 < count) load(jc + 3);
        }
      } else if constexpr (L::STAGE_OUT) {
        if (jc > 0) flush(jc - 1);
      }
    }
    if constexpr (L::STAGE_OUT) {
      __syncthreads();  // the last chunk's outputs
      if ((count & 1) == lgroup && count > 0) flush(count - 1);
    }
    return;
  }

  const int q4 = 4 * (lane >> 4), il = lane & 15;
  const int cl = 16 * wave + il;  // this lane's column within the slice (compute waves)
  const int col0 = v0 + 16 * wave;  // first column of this wave's block
  const int col = col0 + il;
  f32x4 S[NKT];
#pragma unroll
  for (int rt = 0; rt < NKT; ++rt)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      S[rt][j] = p.s0 ? p.s0[((state_row(p, n) * H + h) * D + 16 * rt + q4 + j) * D + col] : 0.f;
  const float scale = p.scale;

  // A whole chunk (every one of a document's but its last) stores without
  // row tests: no branches split the step's code, so the scheduler
  // interleaves its products, LDS reads and stores.
  auto step = [&](int jc, auto full_t) {
    constexpr bool FULL = decltype(full_t)::value;
      const char* buf = smem + (jc & 1) * L::BUF;
      const T* sQ = reinterpret_cast<const T*>(buf + L::off_Q);
      const T* sKW = reinterpret_cast<const T*>(buf + L::off_KW);
      const T* sK = ALIAS ? sKW : reinterpret_cast<const T*>(buf + L::off_K);
      const T* sA = reinterpret_cast<const T*>(buf + L::off_A);
      const T* sT = reinterpret_cast<const T*>(buf + L::off_T);
      const T* sV = reinterpret_cast<const T*>(buf + L::off_V);
      const float* sG = reinterpret_cast<const float*>(buf + L::off_G);
      const float* sB = reinterpret_cast<const float*>(buf + L::off_B);
      const int cid = first + jc;
      const int clen = min(C, dlen - jc * C);
      const int64_t row0 = (int64_t)(dstart + jc * C) * H + h;

      // S as bf16 B operands; checkpoint the entering state
      s16x8_t SB[NKT / 2];
#pragma unroll
      for (int kk = 0; kk < NKT / 2; ++kk) SB[kk] = pack_acc_pair(S[2 * kk], S[2 * kk + 1]);
      if (p.h) {
        T* hb = static_cast<T*>(p.h) + ((int64_t)cid * H + h) * D * D;
#pragma unroll
        for (int kk = 0; kk < NKT / 2; ++kk) {
          const uint4 w = __builtin_bit_cast(uint4, SB[kk]);
          store_packed_tile_nt(hb + tile_offset(D, 2 * kk, col0 / 16), w.x, w.y, lane);
          store_packed_tile_nt(hb + tile_offset(D, 2 * kk + 1, col0 / 16), w.z, w.w, lane);
        }
      }
      // K S and Q S: for each k step the eight tiles are independent accumulators
      f32x4 KS[4], QS[4];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) KS[rb] = QS[rb] = zero4();
#pragma unroll
      for (int kk = 0; kk < NKT / 2; ++kk) {
        s16x8_t ak[4], aq[4];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
          ak[rb] = lds_a_perm(sK + 16 * rb * L::LD, L::LD, 32 * kk, lane);
          aq[rb] = lds_a_perm(sQ + 16 * rb * L::LD, L::LD, 32 * kk, lane);
        }
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
          mfma_bf16(KS[rb], ak[rb], SB[kk]);
          mfma_bf16(QS[rb], aq[rb], SB[kk]);
        }
      }
      // Y = diag(beta) (V - diag(e^G) K S) as B operands over the tokens
      s16x8_t YB[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        f32x4 y[2];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r = 32 * kt + 16 * hf + q4 + j;
            y[hf][j] = sB[r] * (bf16_to_f32(sV[r * L::LDV + cl]) - exp_fast(sG[r]) * KS[2 * kt + hf][j]);
          }
        }
        YB[kt] = pack_acc_pair(y[0], y[1]);
      }
      // U = T Y   (T is lower triangular: row block rb needs k steps kt <= rb / 2)
      f32x4 U[4];
      {
        s16x8_t at[6];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) at[rb] = lds_a_perm(sT + 16 * rb * L::LDC, L::LDC, 0, lane);
        at[4] = lds_a_perm(sT + 32 * L::LDC, L::LDC, 32, lane);
        at[5] = lds_a_perm(sT + 48 * L::LDC, L::LDC, 32, lane);
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
          U[rb] = zero4();
          mfma_bf16(U[rb], at[rb], YB[0]);
        }
        mfma_bf16(U[2], at[4], YB[1]);
        mfma_bf16(U[3], at[5], YB[1]);
      }
      T* so = reinterpret_cast<T*>(smem + L::off_Out + (jc & 1) * L::OUT) + 16 * wave;
      if constexpr (L::STAGE_OUT) {
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) store_acc_global<T, true>(so, L::LDV, U[rb], 16 * rb, 0, C, lane);
      } else {
        T* u_out = static_cast<T*>(p.u) + row0 * D + col0;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) store_acc_global<T, FULL>(u_out, gs, U[rb], 16 * rb, 0, clen, lane);
      }
      const s16x8_t UB[2] = {pack_acc_pair(U[0], U[1]), pack_acc_pair(U[2], U[3])};
      // O = diag(s e^G) Q S + Aqk U   (Aqk is lower triangular: row block rb needs k steps kt <= rb / 2)
      f32x4 AU[4];
      {
        s16x8_t aa[6];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) aa[rb] = lds_a_perm(sA + 16 * rb * L::LDC, L::LDC, 0, lane);
        aa[4] = lds_a_perm(sA + 32 * L::LDC, L::LDC, 32, lane);
        aa[5] = lds_a_perm(sA + 48 * L::LDC, L::LDC, 32, lane);
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
          AU[rb] = zero4();
          mfma_bf16(AU[rb], aa[rb], UB[0]);
        }
        mfma_bf16(AU[2], aa[4], UB[1]);
        mfma_bf16(AU[3], aa[5], UB[1]);
      }
      T* o_out = static_cast<T*>(p.o) + row0 * D + col0;
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        f32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = scale * exp_fast(sG[16 * rb + q4 + j]) * QS[rb][j] + AU[rb][j];
        if constexpr (L::STAGE_OUT) store_acc_global<T, true>(so + C * L::LDV, L::LDV, o, 16 * rb, 0, C, lane);
        else store_acc_global<T, FULL>(o_out, gs, o, 16 * rb, 0, clen, lane);
      }
      // S <- e^{G_C} S + KW^T diag(e^{G_C - G}) U
      const float gC = sG[C - 1];
      s16x8_t UgB[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        float fa[4], fb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          fa[j] = exp_fast(gC - sG[32 * kt + q4 + j]);
          fb[j] = exp_fast(gC - sG[32 * kt + 16 + q4 + j]);
        }
        UgB[kt] = pack_acc_pair_scaled(U[2 * kt], fa, U[2 * kt + 1], fb);
      }
      const float decay = exp_fast(gC);
#pragma unroll
      for (int rt = 0; rt < NKT; ++rt) S[rt] = S[rt] * decay;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        s16x8_t ak[NKT];
#pragma unroll
        for (int rt = 0; rt < NKT; ++rt) ak[rt] = lds_kmajor_perm(sKW + 16 * rt, L::LD, 32 * kt, lane);
#pragma unroll
        for (int rt = 0; rt < NKT; ++rt) mfma_bf16(S[rt], ak[rt], UgB[kt]);
      }
  };
  for (int jc = 0; jc + 1 < count; ++jc) {
    __syncthreads();
    step(jc, std::true_type{});
  }
  if (count > 0) {
    __syncthreads();
    if (dlen - (count - 1) * C == C) step(count - 1, std::true_type{});
    else step(count - 1, std::false_type{});
  }
  if constexpr (L::STAGE_OUT) __syncthreads();  // the loaders' flush of the last chunk
  if (p.sT) {
    float* sb = p.sT + (state_row(p, n) * H + h) * D * D + col0;
#pragma unroll
    for (int rt = 0; rt < NKT; ++rt) store_acc_global<float>(sb, D, S[rt], 16 * rt, 0, D, lane);
  }
}

// ---------------------------------------------------------------------------
// per-document state pass, BF16 with a per-channel gate: register-resident
// form.  The structure of chunk_state_fwd_rr_kernel with the intra kernel's
// W, u, qg = s e^G q and kg = e^{G_last - G} kw as inputs:
//   U = u - W S,   O = qg S + Aqk U,   S <- diag(e^{G_C}) S + kg^T U.
// BV/16 compute waves each keep the S [D x 16] slice in MFMA accumulators and
// the chunk's U [64 x 16] in registers; kRrLoaders loader waves stage qg, W,
// kg, Aqk, the u slice and e^{G_C} (the chunk's last gate row, exponentiated
// by the loader) one chunk ahead in a double-buffered LDS stage.
// ---------------------------------------------------------------------------
template <int D, int BV>
struct RrPcFwdLayout {
  static constexpr int LD = D + Pad<bf16_t>::v;
  static constexpr int LDV = BV + Pad<bf16_t>::v;
  static constexpr int LDC = C + Pad<bf16_t>::v;
  static constexpr int off_Q = 0;                   // qg
  static constexpr int off_W = off_Q + C * LD * 2;
  static constexpr int off_KG = off_W + C * LD * 2;  // kg
  static constexpr int off_A = off_KG + C * LD * 2;  // Aqk
  static constexpr int off_U = off_A + C * LDC * 2;  // the u slice
  static constexpr int off_E = off_U + C * LDV * 2;  // [D] e^{G_C}
  static constexpr int BUF = off_E + D * 4;
  // output stage (where it fits): O rows, double-buffered, written out by the
  // loader group that is not staging inputs in that step
  static constexpr int OUT = C * LDV * 2;
  static constexpr bool STAGE_OUT = 2 * BUF + 2 * OUT <= 160 * 1024;
  static constexpr int off_Out = 2 * BUF;
  static constexpr int bytes = 2 * BUF + (STAGE_OUT ? 2 * OUT : 0);
  static_assert(BUF % 16 == 0 && (LDV * 2) % 16 == 0, "16-byte aligned stages and rows");
  static_assert(bytes <= 160 * 1024, "LDS of one compute unit");
};

template <int D, int BV>
__global__ __launch_bounds__(64 * (BV / 16 + kRrLoaders)) void chunk_state_fwd_rr_pc_kernel(FwdParams p) {
  using L = RrPcFwdLayout<D, BV>;
  using T = bf16_t;
  constexpr int NC = BV / 16;   // compute waves
  constexpr int NKT = D / 16;   // 16-row tiles of the state slice
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const DocSlot ds = doc_slot(p.geom, p.H, D / BV);
  const int n = ds.n, h = ds.h, v0 = ds.z * BV;
  const int H = p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t gs = (int64_t)H * D;
  int first, count, dstart, dlen;
  doc_chunks(p.geom, n, first, count, dstart, dlen);
  const bool loader = wave >= NC;
  constexpr int NGT = 64 * kRrLoaders / 2;   // threads of one loader group
  const int lgroup = (tid - 64 * NC) / NGT;  // loader group: chunks jc with jc % 2 == lgroup
  const int lt = (tid - 64 * NC) % NGT;

  if (loader) {
    RegTile<NGT, C, D, T> rQ, rW, rK;
    RegTile<NGT, C, C, T> rA;
    RegTile<NGT, C, BV, T> rU;
    float re = 0.f;
    auto load = [&](int jc) {
      const int cstart = dstart + jc * C;
      const int clen = min(C, dlen - jc * C);
      const int64_t row0 = (int64_t)cstart * H + h;
      rQ.load_as(lt, static_cast<const T*>(p.qg) + row0 * D, gs, clen);
      rW.load_as(lt, static_cast<const T*>(p.w) + row0 * D, gs, clen);
      rK.load_as(lt, static_cast<const T*>(p.kg) + row0 * D, gs, clen);
      rA.load_as(lt, static_cast<const T*>(p.aqk) + row0 * C, (int64_t)H * C, clen);
      rU.load_as(lt, static_cast<const T*>(p.u) + row0 * D + v0, gs, clen);
      if (lt < D) re = p.gcum[((int64_t)(cstart + clen - 1) * H + h) * D + lt];
    };
    auto stash = [&](int b) {
      char* buf = smem + b * L::BUF;
      rQ.store_as(lt, reinterpret_cast<T*>(buf + L::off_Q), L::LD);
      rW.store_as(lt, reinterpret_cast<T*>(buf + L::off_W), L::LD);
      rK.store_as(lt, reinterpret_cast<T*>(buf + L::off_KG), L::LD);
      rA.store_as(lt, reinterpret_cast<T*>(buf + L::off_A), L::LDC);
      rU.store_as(lt, reinterpret_cast<T*>(buf + L::off_U), L::LDV);
      if (lt < D) reinterpret_cast<float*>(buf + L::off_E)[lt] = exp_fast(re);
    };
    static_assert(D <= NGT, "one loader thread per gate channel");
    // chunk jc's O rows from the output stage to global memory
    auto flush = [&](int jc) {
      constexpr int SEG = BV / 8;  // 16-byte pieces of a row
      static_assert(C * SEG % NGT == 0, "whole passes over the stage");
      const T* so = reinterpret_cast<const T*>(smem + L::off_Out + (jc & 1) * L::OUT);
      const int clen = min(C, dlen - jc * C);
      const int64_t row0 = (int64_t)(dstart + jc * C) * H + h;
#pragma unroll
      for (int it = 0; it < C * SEG / NGT; ++it) {
        const int i = lt + it * NGT;
        const int r = i / SEG, sg = i % SEG;
        if (r < clen) {
          const uint4 x = *reinterpret_cast<const uint4*>(so + r * L::LDV + 8 * sg);
          *reinterpret_cast<uint4*>(static_cast<T*>(p.o) + (row0 + (int64_t)r * H) * D + v0 + 8 * sg) = x;
        }
      }
    };
    if (lgroup < count) load(lgroup);
    if (lgroup == 0 && count > 0) {
      stash(0);
      if (count > 2) load(2);
    }
    for (int jc = 0; jc < count; ++jc) {
      __syncthreads();
      if (((jc + 1) & 1) == lgroup) {
        if (jc + 1 < count) {
          stash((jc + 1) & 1);
          if (jc + 3 < count) load(jc + 3);
        }
      } else if constexpr (L::STAGE_OUT) {
        if (jc > 0) flush(jc - 1);
      }
    }
    if constexpr (L::STAGE_OUT) {
      __syncthreads();  // the last chunk's outputs
      if ((count & 1) == lgroup && count > 0) flush(count - 1);
    }
    return;
  }

  const int q4 = 4 * (lane >> 4), il = lane & 15;
  const int cl = 16 * wave + il;    // this lane's column within the slice
  const int col0 = v0 + 16 * wave;  // first column of this wave's block
  const int col = col0 + il;
  f32x4 S[NKT];
#pragma unroll
  for (int rt = 0; rt < NKT; ++rt)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      S[rt][j] = p.s0 ? p.s0[((state_row(p, n) * H + h) * D + 16 * rt + q4 + j) * D + col] : 0.f;

  auto step = [&](int jc, auto full_t) {
    constexpr bool FULL = decltype(full_t)::value;
    const char* buf = smem + (jc & 1) * L::BUF;
    const T* sQ = reinterpret_cast<const T*>(buf + L::off_Q);
    const T* sW = reinterpret_cast<const T*>(buf + L::off_W);
    const T* sK = reinterpret_cast<const T*>(buf + L::off_KG);
    const T* sA = reinterpret_cast<const T*>(buf + L::off_A);
    const T* sU = reinterpret_cast<const T*>(buf + L::off_U);
    const float* sE = reinterpret_cast<const float*>(buf + L::off_E);
    const int cid = first + jc;
    const int clen = min(C, dlen - jc * C);
    const int64_t row0 = (int64_t)(dstart + jc * C) * H + h;

    // S as bf16 B operands; checkpoint the entering state
    s16x8_t SB[NKT / 2];
#pragma unroll
    for (int kk = 0; kk < NKT / 2; ++kk) SB[kk] = pack_acc_pair(S[2 * kk], S[2 * kk + 1]);
    if (p.h) {
      T* hb = static_cast<T*>(p.h) + ((int64_t)cid * H + h) * D * D;
#pragma unroll
      for (int kk = 0; kk < NKT / 2; ++kk) {
        const uint4 w = __builtin_bit_cast(uint4, SB[kk]);
        store_packed_tile_nt(hb + tile_offset(D, 2 * kk, col0 / 16), w.x, w.y, lane);
        store_packed_tile_nt(hb + tile_offset(D, 2 * kk + 1, col0 / 16), w.z, w.w, lane);
      }
    }
    // W S and qg S: for each k step the eight tiles are independent accumulators
    f32x4 WS[4], QS[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) WS[rb] = QS[rb] = zero4();
#pragma unroll
    for (int kk = 0; kk < NKT / 2; ++kk) {
      s16x8_t aw[4], aq[4];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        aw[rb] = lds_a_perm(sW + 16 * rb * L::LD, L::LD, 32 * kk, lane);
        aq[rb] = lds_a_perm(sQ + 16 * rb * L::LD, L::LD, 32 * kk, lane);
      }
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        mfma_bf16(WS[rb], aw[rb], SB[kk]);
        mfma_bf16(QS[rb], aq[rb], SB[kk]);
      }
    }
    // U = u - W S
    f32x4 U[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int j = 0; j < 4; ++j) U[rb][j] = bf16_to_f32(sU[(16 * rb + q4 + j) * L::LDV + cl]) - WS[rb][j];
    T* u_out = static_cast<T*>(p.u) + row0 * D + col0;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) store_acc_global<T, FULL>(u_out, gs, U[rb], 16 * rb, 0, clen, lane);
    const s16x8_t UB[2] = {pack_acc_pair(U[0], U[1]), pack_acc_pair(U[2], U[3])};
    // O = qg S + Aqk U   (Aqk is lower triangular: row block rb needs k steps kt <= rb / 2)
    f32x4 AU[4];
    {
      s16x8_t aa[6];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) aa[rb] = lds_a_perm(sA + 16 * rb * L::LDC, L::LDC, 0, lane);
      aa[4] = lds_a_perm(sA + 32 * L::LDC, L::LDC, 32, lane);
      aa[5] = lds_a_perm(sA + 48 * L::LDC, L::LDC, 32, lane);
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        AU[rb] = zero4();
        mfma_bf16(AU[rb], aa[rb], UB[0]);
      }
      mfma_bf16(AU[2], aa[4], UB[1]);
      mfma_bf16(AU[3], aa[5], UB[1]);
    }
    if constexpr (L::STAGE_OUT) {
      T* so = reinterpret_cast<T*>(smem + L::off_Out + (jc & 1) * L::OUT) + 16 * wave;
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) store_acc_global<T, true>(so, L::LDV, QS[rb] + AU[rb], 16 * rb, 0, C, lane);
    } else {
      T* o_out = static_cast<T*>(p.o) + row0 * D + col0;
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) store_acc_global<T, FULL>(o_out, gs, QS[rb] + AU[rb], 16 * rb, 0, clen, lane);
    }
    // S <- diag(e^{G_C}) S + kg^T U
#pragma unroll
    for (int rt = 0; rt < NKT; ++rt)
#pragma unroll
      for (int j = 0; j < 4; ++j) S[rt][j] *= sE[16 * rt + q4 + j];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      s16x8_t ak[NKT];
#pragma unroll
      for (int rt = 0; rt < NKT; ++rt) ak[rt] = lds_kmajor_perm(sK + 16 * rt, L::LD, 32 * kt, lane);
#pragma unroll
      for (int rt = 0; rt < NKT; ++rt) mfma_bf16(S[rt], ak[rt], UB[kt]);
    }
  };
  for (int jc = 0; jc + 1 < count; ++jc) {
    __syncthreads();
    step(jc, std::true_type{});
  }
  if (count > 0) {
    __syncthreads();
    if (dlen - (count - 1) * C == C) step(count - 1, std::true_type{});
    else step(count - 1, std::false_type{});
  }
  if constexpr (L::STAGE_OUT) __syncthreads();  // the loaders' flush of the last chunk
  if (p.sT) {
    float* sb = p.sT + (state_row(p, n) * H + h) * D * D + col0;
#pragma unroll
    for (int rt = 0; rt < NKT; ++rt) store_acc_global<float>(sb, D, S[rt], 16 * rt, 0, D, lane);
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

template <int D, int BV, bool ALIAS, bool PACK = false>
int launch_state_fwd_rr_as(const FwdParams& p, hipStream_t s) {
  auto kern = chunk_state_fwd_rr_kernel<D, BV, ALIAS, PACK>;
  constexpr int bytes = RrFwdLayout<D, BV, ALIAS>::bytes;
  if (int st = set_smem(kern, bytes)) return st;
  hipLaunchKernelGGL(kern, doc_grid(p.geom.num_seqs, p.H, D / BV), dim3(64 * (BV / 16 + kRrLoaders)), bytes, s, p);
  return launch_status("pkda_chunk_fwd(state)");
}

// Register-resident state pass: 64 value columns per workgroup, or 32 when
// that leaves fewer workgroups than compute units.
template <int D>
int launch_state_fwd_rr(const FwdParams& p, hipStream_t s) {
  const int N = p.geom.num_seqs;
  if (N <= 0) return 0;
  const bool narrow = (int64_t)N * p.H * (D / 64) < 256;
  const bool alias = p.kw == p.k;
  if (p.tri_packed) {  // kw = k (checked at the entry point)
    return narrow ? launch_state_fwd_rr_as<D, 32, true, true>(p, s) : launch_state_fwd_rr_as<D, 64, true, true>(p, s);
  }
  if (narrow) return alias ? launch_state_fwd_rr_as<D, 32, true>(p, s) : launch_state_fwd_rr_as<D, 32, false>(p, s);
  return alias ? launch_state_fwd_rr_as<D, 64, true>(p, s) : launch_state_fwd_rr_as<D, 64, false>(p, s);
}

template <int D, int BV>
int launch_state_fwd_rr_pc_as(const FwdParams& p, hipStream_t s) {
  auto kern = chunk_state_fwd_rr_pc_kernel<D, BV>;
  constexpr int bytes = RrPcFwdLayout<D, BV>::bytes;
  if (int st = set_smem(kern, bytes)) return st;
  hipLaunchKernelGGL(kern, doc_grid(p.geom.num_seqs, p.H, D / BV), dim3(64 * (BV / 16 + kRrLoaders)), bytes, s, p);
  return launch_status("pkda_chunk_fwd(state)");
}

template <int D>
int launch_state_fwd_rr_pc(const FwdParams& p, hipStream_t s) {
  const int N = p.geom.num_seqs;
  if (N <= 0) return 0;
  const bool narrow = (int64_t)N * p.H * (D / 64) < 256;
  return narrow ? launch_state_fwd_rr_pc_as<D, 32>(p, s) : launch_state_fwd_rr_pc_as<D, 64>(p, s);
}

template <typename T, int D, int BV>
int launch_fwd(const FwdParams& p, int num_chunks, int stages, hipStream_t s) {
  const bool all = stages == 0;
  if (all || (stages & PKDA_STAGE_FWD_INTRA)) {
    const bool alias = p.kw == p.k;
    constexpr bool WU = !implicit_w<T>();
    auto kern = p.qg ? (alias ? chunk_intra_fwd_pc_kernel<T, D, true> : chunk_intra_fwd_pc_kernel<T, D, false>)
                     : (alias ? chunk_intra_fwd_kernel<T, D, true, WU> : chunk_intra_fwd_kernel<T, D, false, WU>);
    const int bytes = p.qg ? (alias ? IntraPcLayout<T, D, true>::bytes : IntraPcLayout<T, D, false>::bytes)
                           : (WU || !IntraLayout<T, D, true>::lean_fits)
                                 ? (alias ? IntraLayout<T, D, true>::bytes : IntraLayout<T, D, false>::bytes)
                                 : (alias ? IntraLayout<T, D, true>::bytes_lean : IntraLayout<T, D, false>::bytes_lean);
    if constexpr (std::is_same<T, bf16_t>::value && D == 128) {
      if (p.qg) {  // BF16 per-channel gate at d = 128: the two-half form, two workgroups per CU
        auto kern2 = alias ? chunk_intra_fwd_pc2_kernel<true> : chunk_intra_fwd_pc2_kernel<false>;
        const int bytes2 = alias ? IntraPc2Layout<true>::bytes : IntraPc2Layout<false>::bytes;
        if (int st = set_smem(kern2, bytes2)) return st;
        if (num_chunks > 0) hipLaunchKernelGGL(kern2, dim3(chunk_grid<false>(num_chunks, p.H)), dim3(kIW), bytes2, s, p);
        kern = nullptr;
      }
    }
    if (kern) {
      if (int st = set_smem(kern, bytes)) return st;
      if (num_chunks > 0) hipLaunchKernelGGL(kern, p.qg ? dim3(chunk_grid<false>(num_chunks, p.H)) : dim3(chunk_grid<true>(num_chunks, p.H)), dim3(kIW), bytes, s, p);
    }
    if (int st = launch_status("pkda_chunk_fwd(intra)")) return st;
  }
  if (all || (stages & PKDA_STAGE_FWD_STATE)) {
    if constexpr (std::is_same<T, bf16_t>::value) {
      if (!p.qg) return launch_state_fwd_rr<D>(p, s);  // BF16, per-head gate: the register-resident pass
      return launch_state_fwd_rr_pc<D>(p, s);         // BF16, per-channel gate: its register-resident pass
    }
    auto kern = p.qg ? chunk_state_fwd_kernel<T, D, BV, true> : chunk_state_fwd_kernel<T, D, BV, false>;
    const int bytes = StateLayout<T, D, BV>::bytes;
    if (int st = set_smem(kern, bytes)) return st;
    if (p.geom.num_seqs > 0)
      hipLaunchKernelGGL(kern, doc_grid(p.geom.num_seqs, p.H, D / BV), dim3(state_threads(D, BV)), bytes, s, p);
    if (int st = launch_status("pkda_chunk_fwd(state)")) return st;
  }
  return 0;
}

}  // namespace

int chunk_geom_from(const int32_t* cu, int num_seqs, int seqlen, int num_chunks, const int32_t* table, ChunkGeom& g) {
  PKDA_REQUIRE(num_seqs >= 0 && num_chunks >= 0, PKDA_EINVAL, "sizes");
  g.num_seqs = num_seqs;
  g.seqlen = seqlen;
  g.nt = cu ? 0 : (seqlen + C - 1) / C;
  g.table = reinterpret_cast<const int4*>(table);
  g.offsets = table ? table + 4 * num_chunks : nullptr;
  g.order = table ? g.offsets + num_seqs + 1 : nullptr;
  // packed documents: the kernels read the table's sanitised copy of cu
  g.cu = cu && table ? g.order + num_seqs : nullptr;
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
  PKDA_REQUIRE(!a->gate_per_channel || (a->qg && a->kg), PKDA_EINVAL, "per-channel gates need the qg and kg outputs");
  PKDA_REQUIRE(!a->gate_per_channel || a->dtype == PKDA_BF16 || a->head_dim == 64, PKDA_EUNSUPPORTED,
               "FP32 per-channel chunked forward is built for head_dim 64 only");
  FwdParams p;
  if (int st = chunk_geom_from(a->cu_seqlens, a->num_seqs, a->seqlen, a->num_chunks, a->table, p.geom)) return st;
  if (a->num_seqs == 0) return 0;
  PKDA_REQUIRE(a->q && a->k && a->v && a->gcum && a->beta && a->o && a->u && a->aqk && a->akk, PKDA_EINVAL,
               "null tensor");
  const bool needs_w = a->dtype != PKDA_BF16 || a->gate_per_channel;  // BF16, per-head gate: W is never stored
  PKDA_REQUIRE(a->w || !needs_w, PKDA_EINVAL, "this dtype / gate needs the w buffer");
  p.H = a->heads;
  p.q = a->q; p.k = a->k; p.kw = a->kw ? a->kw : a->k; p.v = a->v;
  p.gcum = a->gcum; p.beta = a->beta; p.scale = a->scale;
  p.gcum_lo = a->gate_per_channel && a->dtype == PKDA_F32 ? a->gcum_lo : nullptr;
  p.s0 = a->initial_state; p.sT = a->final_state; p.o = a->o;
  p.w = a->w; p.u = a->u; p.aqk = a->aqk; p.akk = a->akk; p.h = a->h;
  p.qg = a->gate_per_channel ? a->qg : nullptr;
  p.kg = a->gate_per_channel ? a->kg : nullptr;
  p.slot = a->slot_idx;
  PKDA_REQUIRE(!a->slot_idx || a->pool_size > 0, PKDA_EINVAL, "slot-indexed states need pool_size > 0");
  p.tri_packed = a->tri_packed != 0;
  PKDA_REQUIRE(!p.tri_packed || (a->dtype == PKDA_BF16 && !a->gate_per_channel && p.kw == p.k), PKDA_EUNSUPPORTED,
               "packed aqk / akk (tri_packed) are built for BF16 with a per-head gate and kw == k");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nc = a->num_chunks;
  const int st = a->stages;
  PKDA_REQUIRE(st >= 0 && st <= (PKDA_STAGE_FWD_INTRA | PKDA_STAGE_FWD_STATE), PKDA_EINVAL, "stages %d", st);
  if (a->dtype == PKDA_BF16) {
    return a->head_dim == 128 ? launch_fwd<bf16_t, 128, 64>(p, nc, st, s) : launch_fwd<bf16_t, 64, 64>(p, nc, st, s);
  }
  return a->head_dim == 128 ? launch_fwd<float, 128, 16>(p, nc, st, s) : launch_fwd<float, 64, 64>(p, nc, st, s);
}
