// Diagonal write-key preconditioner: forward scan and reverse (gradient) scan.
//
// Per (document, head, key channel c), with the preconditioner log-decay
// g_atk and strength beta_atk per (token, head) and the log-space center
// per head (delta_feedback_experiment/pkda.py:392-398):
//
//   A_t  = exp(g_atk_t) A_{t-1} + beta_atk_t k_t^2
//   r_t  = log(A_t + eps) - center
//   kw_t = k_t f(r_t),   f(r) = exp(-ln(x) r / (1 + |r|))
//
// Backward, with lambda_t = dL/dA_t carried in reverse
// (lambda_t = e^{g_atk_{t+1}} lambda_{t+1} + dkw_t k_t f'(r_t) / (A_t + eps),
//  f'(r) = -ln(x) f(r) / (1 + |r|)^2, and lambda after the last token = dA_T):
//
//   dk_t       += dkw_t f(r_t) + 2 beta_atk_t k_t lambda_t
//   dg_atk_t    = sum_c lambda_t e^{g_atk_t} A_{t-1}
//   dbeta_atk_t = sum_c lambda_t k_t^2
//   dcenter     = -sum_{t,c} dkw_t k_t f'(r_t)
//   dA_0        = e^{g_atk_first} lambda_first
//
// Exponentials, logarithms and reciprocals use the hardware's (v_exp_f32,
// v_log_f32, v_rcp_f32: about 1e-7 relative), the same in every pass.
//
// Both recurrences are linear with inputs known up front (lambda's input
// only needs the forward's A), so each runs chunk-parallel in three launches
// instead of one sequential walk per (document, head):
//   1. per (chunk, head): the chunk's end value from a zero start
//      (A forward, lambda in reverse);
//   2. per (document, head): the scan over the document's chunks,
//      x_out = exp(sum of the chunk's g_atk) x_in + local end, which leaves
//      the value entering each chunk in place of its local end
//      (a_chunk: A entering the chunk; lam_chunk: lambda entering it from
//      the right);
//   3. per (chunk, head): the chunk again from its entering value, writing
//      kw (forward) or the gradients (backward).
// The forward's third launch and both backward chunk launches recompute A
// inside the chunk from a_chunk with the same arithmetic, so the backward
// sees exactly the A the forward squashed.  Channel sums (dg_atk, dbeta_atk,
// dcenter) reduce in a fixed order: lanes of a 16-lane row, then rows.
#include <type_traits>

#include "pkda_chunk_common.h"

namespace pkda {
namespace {

struct PrecondParams {
  ChunkGeom geom;
  int H;
  const void* k;
  const float* g_atk;
  const float* beta_atk;
  const float* center;
  float log_x, eps;
  const float* a0;
  float* aT;
  void* kw;
  float* a_chunk;
  const void* dkw;  // backward: FP32, or k's dtype when narrow_grads
  void* dk;
  float* dg_atk;
  float* dbeta_atk;
  float* dcenter_part;
  float* dA0;
  const float* dA_T;
  const int32_t* slot;  // forward: document -> A-state row, or null
  float* lam_chunk;
  void* dk_final;  // backward: dk + the terms here in k's dtype (dk untouched), or null
  float* kw32;     // forward: kw also in FP32, or null
  bool narrow_grads;  // backward: dkw and dk in k's dtype (dk read only, dk_final written)
  float* chunk_decay;  // [num_chunks][H] exp(sum of the chunk's g_atk) from the local pass, or null
};

template <int D> struct PrecondThreads { static constexpr int v = D < 64 ? 64 : D; };

// The per-(chunk, head) passes: CH consecutive channels per lane (two at
// D = 128, so a chunk is one wave), read and written as one 4- or 8-byte
// access per row, each channel its own chain.
template <int D> struct PrecondChunk {
  static constexpr int CH = D >= 128 ? 2 : 1;
  static constexpr int NT = D / CH < 64 ? 64 : D / CH;
};
template <typename T, int CH> struct ChanIO;
template <typename T> struct ChanIO<T, 1> {
  __device__ __forceinline__ static void load(const T* p, float* x) { x[0] = io<T>::load(p); }
  __device__ __forceinline__ static void store(T* p, const float* x) { io<T>::store(p, x[0]); }
};
template <> struct ChanIO<float, 2> {
  __device__ __forceinline__ static void load(const float* p, float* x) {
    const float2 v = *reinterpret_cast<const float2*>(p);
    x[0] = v.x;
    x[1] = v.y;
  }
  __device__ __forceinline__ static void store(float* p, const float* x) {
    *reinterpret_cast<float2*>(p) = make_float2(x[0], x[1]);
  }
};
template <> struct ChanIO<bf16_t, 2> {
  __device__ __forceinline__ static void load(const bf16_t* p, float* x) {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(p);
    x[0] = __uint_as_float(v << 16);
    x[1] = __uint_as_float(v & 0xffff0000u);
  }
  __device__ __forceinline__ static void store(bf16_t* p, const float* x) {
    *reinterpret_cast<uint32_t*>(p) =
        static_cast<uint32_t>(f32_to_bf16(x[0])) | (static_cast<uint32_t>(f32_to_bf16(x[1])) << 16);
  }
};

// Per-(chunk, head) launches on chunk_grid<false>: workgroup b takes chunk
// b / H of head b % H (chunk_head<false>).

// exp(sum of g_atk over the chunk) for chunks j0 .. j0 + nb - 1 of a document
// (first chunk id first, first token dstart, dlen tokens), chunk j0 + i at
// s[i]: read from chunk_decay when the local pass wrote it there, else
// thread i sums its chunk's tokens in order, as the local passes do.  The
// chunk's C loads go out together (rows clamped to its last token, masked in
// the sum -- adding 0 changes no nonzero sum), so the sum waits for one
// memory round trip.
__device__ __forceinline__ void chunk_decays(const PrecondParams& p, int h, int first, int dstart, int dlen, int j0,
                                             int nb, float* s) {
  const int i = threadIdx.x;
  if (i < nb && p.chunk_decay) {
    s[i] = p.chunk_decay[(int64_t)(first + j0 + i) * p.H + h];  // the local pass's sum, bit for bit
  } else if (i < nb) {
    const int t0 = dstart + (j0 + i) * C;
    const int len = min(C, dlen - (j0 + i) * C);
    float v[C];
#pragma unroll
    for (int u = 0; u < C; ++u) v[u] = p.g_atk[(int64_t)(t0 + min(u, len - 1)) * p.H + h];
    float g = 0.f;
#pragma unroll
    for (int u = 0; u < C; ++u) g += u < len ? v[u] : 0.f;
    s[i] = exp_fast(g);
  }
}

// Chunk-level scan of one (document, head): buf holds, per chunk of the
// document (row (chunk * H + h) * D + channel), the chunk's local end value;
// it is replaced by the value entering the chunk, walking the chunks forward
// (REVERSE = false) or backward.  Returns the value after the last chunk
// walked.
template <int D, bool REVERSE>
__device__ __forceinline__ float chunk_scan(const PrecondParams& p, float* buf, int h, int first, int count,
                                            int dstart, int dlen, float x, float* sDecay) {
  constexpr int NB = C;  // chunks per block (<= the workgroup's threads)
  static_assert(NB <= PrecondThreads<D>::v, "one decay per thread");
  const int c = threadIdx.x;
  const int64_t step = (int64_t)p.H * D;
  for (int b = 0; b < count; b += NB) {
    const int nb = min(NB, count - b);
    const int j0 = REVERSE ? count - b - nb : b;  // first chunk of this block
    // the block's local ends go out first (indices clamped into the block),
    // then the decays' loads: both wait together, one round trip, and the
    // chain below runs on registers in the walk's order
    float* base = buf + ((int64_t)(first + j0) * p.H + h) * D + (c < D ? c : 0);
    float l[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) l[u] = base[(REVERSE ? max(nb - 1 - u, 0) : min(u, nb - 1)) * step];
    __syncthreads();
    chunk_decays(p, h, first, dstart, dlen, j0, nb, sDecay);
    __syncthreads();
    if (c < D) {
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        if (u < nb) {
          const int i = REVERSE ? nb - 1 - u : u;
          base[i * step] = x;
          x = __builtin_fmaf(sDecay[i], x, l[u]);
        }
      }
    }
  }
  return x;
}

// Forward launches 1 (APPLY = false: local end A from zero into a_chunk) and
// 3 (APPLY: A from a_chunk, kw out).  The chunk runs in sub-blocks of 8
// tokens whose k rows load before their chain runs; a short chunk
// (FULL = false) clamps its loads to its last token and leaves the state
// unchanged past it, so no load sits behind a branch.
template <typename T, int D, bool APPLY, bool FULL>
__device__ __forceinline__ void precond_fwd_chunk(const PrecondParams& p, int j, int h, int start, int len) {
  constexpr int G = 8, CH = PrecondChunk<D>::CH;
  using IO = ChanIO<T, CH>;
  using FIO = ChanIO<float, CH>;
  const int H = p.H, c0 = CH * threadIdx.x;
  const T* __restrict__ k = static_cast<const T*>(p.k);
  T* __restrict__ kw = static_cast<T*>(p.kw);
  const float* __restrict__ g_atk = p.g_atk;
  const float* __restrict__ beta_atk = p.beta_atk;
  float* slot = p.a_chunk + ((int64_t)j * H + h) * D + c0;
  float a[CH];
#pragma unroll
  for (int q = 0; q < CH; ++q) a[q] = 0.f;
  if (APPLY) FIO::load(slot, a);
  const float center = APPLY ? p.center[h] : 0.f;
  float gs = 0.f;  // local pass: the chunk's g_atk summed in token order (masked rows add 0)
  auto tok = [&](int t) -> int64_t { return (int64_t)(start + (FULL ? t : min(t, len - 1))) * H + h; };
#pragma unroll 1
  for (int g0 = 0; g0 < C; g0 += G) {
    // the group's k rows and its per-token gate values go out together
    float kc[G][CH], lg[G], bg[G];
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const int64_t th = tok(g0 + u);
      IO::load(k + th * D + c0, kc[u]);
      lg[u] = g_atk[th];
      bg[u] = beta_atk[th];
    }
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const int t = g0 + u;
      const int64_t th = tok(t);
      const float eg = exp_fast(lg[u]), bt = bg[u];
      if (!APPLY) gs += (FULL || t < len) ? lg[u] : 0.f;
      float w[CH];
#pragma unroll
      for (int q = 0; q < CH; ++q) {
        const float an = eg * a[q] + bt * (kc[u][q] * kc[u][q]);
        a[q] = (FULL || t < len) ? an : a[q];
        if (APPLY) {
          const float r = log_fast(a[q] + p.eps) - center;
          w[q] = kc[u][q] * exp_fast(-p.log_x * div_fast(r, 1.f + fabsf(r)));
        }
      }
      if (APPLY && (FULL || t < len)) {
        IO::store(kw + th * D + c0, w);
        if (p.kw32) FIO::store(p.kw32 + th * D + c0, w);
      }
    }
  }
  if (!APPLY) {
    FIO::store(slot, a);
    if (p.chunk_decay && threadIdx.x == 0) p.chunk_decay[(int64_t)j * H + h] = exp_fast(gs);
  }
}

template <typename T, int D, bool APPLY>
__global__ __launch_bounds__(PrecondChunk<D>::NT) void precond_fwd_chunk_kernel(PrecondParams p) {
  const ChunkHead ch = chunk_head<false>(p.H);
  if (threadIdx.x * PrecondChunk<D>::CH >= D) return;
  const ChunkInfo ci = chunk_info(p.geom, ch.cid);
  if (ci.len == C)
    precond_fwd_chunk<T, D, APPLY, true>(p, ch.cid, ch.h, ci.start, C);
  else if (ci.len > 0)
    precond_fwd_chunk<T, D, APPLY, false>(p, ch.cid, ch.h, ci.start, ci.len);
}

// Forward launch 2: per (document, head), A entering every chunk and the
// final A.
template <int D>
__global__ __launch_bounds__(PrecondThreads<D>::v) void precond_fwd_scan_kernel(PrecondParams p) {
  __shared__ float sDecay[PrecondThreads<D>::v];
  const DocSlot ds = doc_slot(p.geom, p.H, 1);
  const int n = ds.n, h = ds.h, c = threadIdx.x;
  int first, count, dstart, dlen;
  doc_chunks(p.geom, n, first, count, dstart, dlen);
  const int64_t sh = (int64_t)(p.slot ? p.slot[n] : n) * p.H + h;  // state row
  float a = (c < D && p.a0) ? p.a0[sh * D + c] : 0.f;
  a = chunk_scan<D, false>(p, p.a_chunk, h, first, count, dstart, dlen, a, sDecay);
  if (c < D && p.aT) p.aT[sh * D + c] = a;
}

// Sum of v over each 16-lane row, in every lane of the row (fixed order).
__device__ __forceinline__ float row_sum16(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));  // quad [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));  // quad [2,3,0,1]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)); // half-row mirror
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)); // row mirror
  return v;
}

// Backward launches 1 (APPLY = false: lambda's local value before the chunk
// from a zero start after it, into lam_chunk, and the chunk's decay into
// chunk_decay) and 3 (APPLY: from the lambda entering the chunk, the
// gradients).  The chunk is walked in reverse in sub-blocks of 8 tokens: a
// first forward pass keeps A at each sub-block's start, and each sub-block
// recomputes its A_t from there (the same arithmetic, so the same values)
// with its k, dkw and dk rows in registers.
// Loads clamp as in the forward.  The per-token channel sums leave each
// 16-lane row in lane (t mod 16) of that row (register t / 16), then cross
// the rows through LDS.
template <typename T, int D, bool APPLY, bool FULL, typename GT>
__device__ __forceinline__ void precond_bwd_chunk(const PrecondParams& p, int j, int h, int start, int len,
                                                  float (*sRow)[C][PrecondChunk<D>::NT / 16 + 1], float* sCen) {
  constexpr int CH = PrecondChunk<D>::CH;
  constexpr int NR = PrecondChunk<D>::NT / 16;  // 16-lane rows
  constexpr int G = 8;                           // tokens per sub-block (measured best for both passes)
  constexpr int NB = C / G;
  constexpr int NQ = C / 16;                     // per-token sum registers
  using IO = ChanIO<T, CH>;
  using FIO = ChanIO<float, CH>;
  using GIO = ChanIO<GT, CH>;  // dkw and dk as they come in
  const int H = p.H, c = threadIdx.x, lane16 = c & 15;
  const bool active = c * CH < D;
  const int c0 = active ? c * CH : 0;  // first channel the lane reads (idle lanes mirror 0, contribute 0)
  const T* __restrict__ k = static_cast<const T*>(p.k);
  const GT* __restrict__ dkw_p = static_cast<const GT*>(p.dkw);
  GT* __restrict__ dk_p = static_cast<GT*>(p.dk);
  T* __restrict__ dk_fin = static_cast<T*>(p.dk_final);
  const float* __restrict__ g_atk = p.g_atk;
  const float* __restrict__ beta_atk = p.beta_atk;
  const int64_t row = ((int64_t)j * H + h) * D + c0;
  float a_in[CH], lam[CH];
#pragma unroll
  for (int q = 0; q < CH; ++q) a_in[q] = lam[q] = 0.f;
  if (active) FIO::load(p.a_chunk + row, a_in);
  if (APPLY && active) FIO::load(p.lam_chunk + row, lam);
  const float center = p.center[h], lx = p.log_x, eps = p.eps;
  auto tok = [&](int t) -> int64_t { return (int64_t)(start + (FULL ? t : min(t, len - 1))) * H + h; };
  // one token of the forward's A recurrence, channel by channel (the same
  // arithmetic as the forward pass, so the same values)
  auto step = [&](int t, float* a, const float* kc, float lgv, float bt) {
    const float eg = exp_fast(lgv);
#pragma unroll
    for (int q = 0; q < CH; ++q) {
      const float an = eg * a[q] + bt * (kc[q] * kc[q]);
      a[q] = (FULL || t < len) ? an : a[q];
    }
  };
  // Register arrays indexed by the (rolled) sub-block number go through
  // compile-time selects so they stay in registers.
  // The forward walk that records them loads GL tokens per memory round
  // trip (their gate values one per lane, taken back by lane reads), so the
  // A recomputation waits C / GL times rather than NB times.
  constexpr int GL = 16;
  static_assert(GL % G == 0 && C % GL == 0 && GL <= 64, "load rounds hold whole sub-blocks");
  float a_blk[NB][CH];  // A entering each sub-block
  float gs = 0.f;       // local pass: the chunk's g_atk summed in token order (masked rows add 0)
  {
    float a[CH];
#pragma unroll
    for (int q = 0; q < CH; ++q) a[q] = a_in[q];
    const int lt = threadIdx.x & (GL - 1);  // the token whose gate values this lane loads
#pragma unroll 1
    for (int b = 0; b < C / GL; ++b) {
      float kb[GL][CH];  // k rows of the round, loaded together
#pragma unroll
      for (int u = 0; u < GL; ++u) IO::load(k + tok(b * GL + u) * D + c0, kb[u]);
      const float lgl = g_atk[tok(b * GL + lt)], bgl = beta_atk[tok(b * GL + lt)];
#pragma unroll
      for (int u = 0; u < GL; ++u) {
        if (u % G == 0) {
          const int sb = b * (GL / G) + u / G;
#pragma unroll
          for (int r = 0; r < NB; ++r)
#pragma unroll
            for (int q = 0; q < CH; ++q) a_blk[r][q] = r == sb ? a[q] : a_blk[r][q];
        }
#pragma unroll
        for (int q = 0; q < CH; ++q) kb[u][q] = active ? kb[u][q] : 0.f;
        const float lgu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lgl), u));
        step(b * GL + u, a, kb[u], lgu, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bgl), u)));
        if (!APPLY) gs += (FULL || b * GL + u < len) ? lgu : 0.f;
      }
    }
  }
  float dcen = 0.f;
  float sg[NQ], sb[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) sg[q] = sb[q] = 0.f;
#pragma unroll 1
  for (int b = NB - 1; b >= 0; --b) {
    const int g0 = b * G;
    float a_b[CH];
#pragma unroll
    for (int q = 0; q < CH; ++q) {
      a_b[q] = a_blk[0][q];
#pragma unroll
      for (int r = 1; r < NB; ++r) a_b[q] = r == b ? a_blk[r][q] : a_b[q];
    }
    float rk[G][CH], ra[G][CH], rdkw[G][CH], rdk[G][CH], lg[G], bg[G];
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const int64_t th = tok(g0 + u);
      IO::load(k + th * D + c0, rk[u]);
      GIO::load(dkw_p + th * D + c0, rdkw[u]);
      if (APPLY) GIO::load(dk_p + th * D + c0, rdk[u]);
    }
    {  // the sub-block's gate values, one per lane, read back lane by lane
      const float lgl = g_atk[tok(g0 + (threadIdx.x & (G - 1)))], bgl = beta_atk[tok(g0 + (threadIdx.x & (G - 1)))];
#pragma unroll
      for (int u = 0; u < G; ++u) {
        lg[u] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lgl), u));
        bg[u] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bgl), u));
      }
    }
    {
      float a[CH];
#pragma unroll
      for (int q = 0; q < CH; ++q) a[q] = a_b[q];
#pragma unroll
      for (int u = 0; u < G; ++u) {
#pragma unroll
        for (int q = 0; q < CH; ++q) rk[u][q] = active ? rk[u][q] : 0.f;
        step(g0 + u, a, rk[u], lg[u], bg[u]);
#pragma unroll
        for (int q = 0; q < CH; ++q) ra[u][q] = a[q];
      }
    }
#pragma unroll
    for (int u = G - 1; u >= 0; --u) {
      const int t = g0 + u;
      const bool in = FULL || t < len;
      const int64_t th = tok(t);
      const float eg = exp_fast(lg[u]);
      float vg = 0.f, vb = 0.f, dkt[CH];
#pragma unroll
      for (int q = 0; q < CH; ++q) {
        const float kc = rk[u][q], at = ra[u][q];
        const float r = log_fast(at + eps) - center;
        const float den = 1.f + fabsf(r);
        const float rden = __builtin_amdgcn_rcpf(den);
        const float f = exp_fast(-lx * (r * rden));
        const float dkw = active && in ? rdkw[u][q] : 0.f;
        const float dr = dkw * kc * f * (-lx) * (rden * rden);
        const float lam_t = lam[q] + div_fast(dr, at + eps);
        if (APPLY) {
          dcen -= dr;
          dkt[q] = rdk[u][q] + (dkw * f + 2.f * bg[u] * kc * lam_t);
          const float a_prev = u > 0 ? ra[u - 1][q] : a_b[q];
          vg += lam_t * eg * a_prev;
          vb += lam_t * kc * kc;
        }
        lam[q] = in ? lam_t * eg : lam[q];  // carry to A_{t-1}
      }
      if (APPLY) {
        if (active && in) {
          if constexpr (std::is_same<GT, float>::value) {
            if (dk_fin) IO::store(dk_fin + th * D + c0, dkt);
            else FIO::store(dk_p + th * D + c0, dkt);
          } else {
            IO::store(dk_fin + th * D + c0, dkt);  // narrow gradients always leave through dk_final
          }
        }
        vg = row_sum16(vg);
        vb = row_sum16(vb);
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          const bool mine = q == (t >> 4) && lane16 == (t & 15);
          sg[q] = mine ? vg : sg[q];
          sb[q] = mine ? vb : sb[q];
        }
      }
    }
  }
  if (!APPLY) {
    if (active) FIO::store(p.lam_chunk + row, lam);
    if (p.chunk_decay && c == 0) p.chunk_decay[(int64_t)j * H + h] = exp_fast(gs);
    return;
  }
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    sRow[0][16 * q + lane16][c >> 4] = sg[q];
    sRow[1][16 * q + lane16][c >> 4] = sb[q];
  }
  dcen = row_sum16(dcen);
  if (lane16 == 0) sCen[c >> 4] = dcen;
  __syncthreads();
  if (c < len) {
    float tg = 0.f, tb = 0.f;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      tg += sRow[0][c][r];
      tb += sRow[1][c][r];
    }
    const int64_t th = (int64_t)(start + c) * H + h;
    p.dg_atk[th] = tg;
    p.dbeta_atk[th] = tb;
  }
  if (c == 0) {
    float tot = 0.f;
#pragma unroll
    for (int r = 0; r < NR; ++r) tot += sCen[r];
    p.dcenter_part[(int64_t)j * H + h] = tot;
  }
}

template <typename T, int D, bool APPLY, typename GT>
__global__ __launch_bounds__(PrecondChunk<D>::NT) void precond_bwd_chunk_kernel(PrecondParams p) {
  __shared__ float sRow[2][C][PrecondChunk<D>::NT / 16 + 1];
  __shared__ float sCen[PrecondChunk<D>::NT / 16];
  const ChunkHead ch = chunk_head<false>(p.H);
  const ChunkInfo ci = chunk_info(p.geom, ch.cid);
  if (ci.len == C)
    precond_bwd_chunk<T, D, APPLY, true, GT>(p, ch.cid, ch.h, ci.start, C, sRow, sCen);
  else if (ci.len > 0)
    precond_bwd_chunk<T, D, APPLY, false, GT>(p, ch.cid, ch.h, ci.start, ci.len, sRow, sCen);
  else if (APPLY && threadIdx.x == 0)
    p.dcenter_part[(int64_t)ch.cid * p.H + ch.h] = 0.f;
}

// Backward launch 2: per (document, head), lambda entering every chunk from
// the right, walking the chunks last to first, and dA_0.
template <int D>
__global__ __launch_bounds__(PrecondThreads<D>::v) void precond_bwd_scan_kernel(PrecondParams p) {
  __shared__ float sDecay[PrecondThreads<D>::v];
  const DocSlot ds = doc_slot(p.geom, p.H, 1);
  const int n = ds.n, h = ds.h, c = threadIdx.x;
  int first, count, dstart, dlen;
  doc_chunks(p.geom, n, first, count, dstart, dlen);
  const int64_t sh = (int64_t)n * p.H + h;
  float lam = (c < D && p.dA_T) ? p.dA_T[sh * D + c] : 0.f;  // dL/dA after the last token
  lam = chunk_scan<D, true>(p, p.lam_chunk, h, first, count, dstart, dlen, lam, sDecay);
  if (c < D && p.dA0) p.dA0[sh * D + c] = lam;
}

// dcenter[h] = sum over the chunk partials part[j, h], fixed order: 256
// strided partial sums, then a tree.
__global__ __launch_bounds__(256) void precond_dcenter_kernel(const float* part, int M, int H, float* out) {
  __shared__ float s[256];
  const int h = blockIdx.x, i = threadIdx.x;
  float acc = 0.f;
  for (int j = i; j < M; j += 256) acc += part[(int64_t)j * H + h];
  s[i] = acc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (i < w) s[i] += s[i + w];
    __syncthreads();
  }
  if (i == 0) out[h] = s[0];
}

int precond_common(const pkda_precond_args* a, PrecondParams& p) {
  PKDA_REQUIRE(a != nullptr, PKDA_EINVAL, "null args");
  PKDA_REQUIRE(a->struct_size == (int32_t)sizeof(pkda_precond_args), PKDA_EINVAL, "pkda_precond_args size mismatch");
  PKDA_REQUIRE(a->dtype == PKDA_F32 || a->dtype == PKDA_BF16, PKDA_EUNSUPPORTED, "dtype %d", a->dtype);
  PKDA_REQUIRE(a->head_dim == 32 || a->head_dim == 64 || a->head_dim == 128, PKDA_EUNSUPPORTED,
               "head_dim %d not built (32, 64, 128)", a->head_dim);
  PKDA_REQUIRE(a->heads > 0, PKDA_EINVAL, "heads");
  PKDA_REQUIRE(a->squash_x > 0.f, PKDA_EINVAL, "squash_x must be positive");
  if (int st = chunk_geom_from(a->cu_seqlens, a->num_seqs, a->seqlen, a->num_chunks, a->table, p.geom)) return st;
  PKDA_REQUIRE(a->num_seqs == 0 || (a->k && a->g_atk && a->beta_atk && a->center), PKDA_EINVAL,
               "preconditioner needs k, g_atk, beta_atk and center");
  p.H = a->heads;
  p.k = a->k;
  p.g_atk = a->g_atk;
  p.beta_atk = a->beta_atk;
  p.center = a->center;
  p.log_x = logf(a->squash_x);
  p.eps = a->squash_eps;
  p.a0 = a->initial_A_state;
  p.aT = a->final_A_state;
  p.kw = a->kw;
  p.a_chunk = a->a_chunk;
  p.dkw = a->dkw;
  p.dk = a->dk;
  p.dg_atk = a->dg_atk;
  p.dbeta_atk = a->dbeta_atk;
  p.dcenter_part = a->dcenter_part;
  p.dA0 = a->dA0;
  p.dA_T = a->dA_T;
  p.slot = a->slot_idx;
  p.lam_chunk = a->lam_chunk;
  p.dk_final = a->dk_final;
  p.kw32 = a->kw32;
  p.narrow_grads = a->grad_dtype != PKDA_F32;
  p.chunk_decay = a->chunk_decay;
  PKDA_REQUIRE(!a->slot_idx || a->pool_size > 0, PKDA_EINVAL, "slot-indexed A states need pool_size > 0");
  return 0;
}

template <typename T, int D, typename GT>
void launch_precond_bwd_chunks(const PrecondParams& p, hipStream_t s) {
  constexpr int NT = PrecondThreads<D>::v, NTC = PrecondChunk<D>::NT;
  const dim3 chunks(chunk_grid<false>(p.geom.num_chunks, p.H));
  const dim3 docs = doc_grid(p.geom.num_seqs, p.H, 1);
  const bool any = p.geom.num_chunks > 0;
  if (any) hipLaunchKernelGGL((precond_bwd_chunk_kernel<T, D, false, GT>), chunks, dim3(NTC), 0, s, p);
  hipLaunchKernelGGL((precond_bwd_scan_kernel<D>), docs, dim3(NT), 0, s, p);
  if (any) hipLaunchKernelGGL((precond_bwd_chunk_kernel<T, D, true, GT>), chunks, dim3(NTC), 0, s, p);
}

template <typename T, int D>
int launch_precond(const PrecondParams& p, bool backward, hipStream_t s) {
  constexpr int NT = PrecondThreads<D>::v, NTC = PrecondChunk<D>::NT;
  const dim3 chunks(chunk_grid<false>(p.geom.num_chunks, p.H));
  const dim3 docs = doc_grid(p.geom.num_seqs, p.H, 1);
  const bool any = p.geom.num_chunks > 0;
  if (backward) {
    if (p.narrow_grads) launch_precond_bwd_chunks<T, D, T>(p, s);
    else launch_precond_bwd_chunks<T, D, float>(p, s);
  } else {
    if (any) hipLaunchKernelGGL((precond_fwd_chunk_kernel<T, D, false>), chunks, dim3(NTC), 0, s, p);
    hipLaunchKernelGGL((precond_fwd_scan_kernel<D>), docs, dim3(NT), 0, s, p);
    if (any) hipLaunchKernelGGL((precond_fwd_chunk_kernel<T, D, true>), chunks, dim3(NTC), 0, s, p);
  }
  return launch_status(backward ? "pkda_precond_bwd" : "pkda_precond_fwd");
}

template <typename T>
int dispatch_precond(const PrecondParams& p, int D, bool backward, hipStream_t s) {
  switch (D) {
    case 32: return launch_precond<T, 32>(p, backward, s);
    case 64: return launch_precond<T, 64>(p, backward, s);
    default: return launch_precond<T, 128>(p, backward, s);
  }
}

}  // namespace
}  // namespace pkda

using namespace pkda;

extern "C" int pkda_precond_fwd(const pkda_precond_args* a, void* stream) {
  PrecondParams p;
  if (int st = precond_common(a, p)) return st;
  if (a->num_seqs == 0) return 0;
  PKDA_REQUIRE(a->kw && a->a_chunk, PKDA_EINVAL, "preconditioner forward needs kw and a_chunk");
  hipStream_t s = static_cast<hipStream_t>(stream);
  return a->dtype == PKDA_F32 ? dispatch_precond<float>(p, a->head_dim, false, s)
                              : dispatch_precond<bf16_t>(p, a->head_dim, false, s);
}

extern "C" int pkda_precond_bwd(const pkda_precond_args* a, void* stream) {
  PrecondParams p;
  if (int st = precond_common(a, p)) return st;
  PKDA_REQUIRE(!a->slot_idx, PKDA_EUNSUPPORTED, "slot-indexed A states are a forward (prefill) feature");
  PKDA_REQUIRE(a->dcenter && a->dcenter_part, PKDA_EINVAL, "preconditioner backward needs dcenter buffers");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->num_seqs > 0) {
    PKDA_REQUIRE(a->a_chunk && a->lam_chunk && a->dkw && a->dk && a->dg_atk && a->dbeta_atk, PKDA_EINVAL,
                 "preconditioner backward needs a_chunk, lam_chunk, dkw, dk, dg_atk and dbeta_atk");
    PKDA_REQUIRE(a->grad_dtype == PKDA_F32 || a->grad_dtype == a->dtype, PKDA_EUNSUPPORTED,
                 "grad_dtype %d (FP32 or the dtype of k)", a->grad_dtype);
    PKDA_REQUIRE(a->grad_dtype == PKDA_F32 || a->dk_final, PKDA_EINVAL,
                 "dkw and dk in the dtype of k need dk_final");
    const int st = a->dtype == PKDA_F32 ? dispatch_precond<float>(p, a->head_dim, true, s)
                                        : dispatch_precond<bf16_t>(p, a->head_dim, true, s);
    if (st) return st;
  }
  hipLaunchKernelGGL(precond_dcenter_kernel, dim3(a->heads), dim3(256), 0, s, a->dcenter_part,
                     a->num_seqs > 0 ? a->num_chunks : 0, a->heads, a->dcenter);
  return launch_status("pkda_precond_bwd(dcenter)");
}
