// Chunk table for packed documents, and the gate's chunk-local cumulative
// log-decay (forward) and reverse cumsum + activation gradients (backward).
//
// Gate forms (natural log throughout):
//   PKDA_GATE_LOG_HEAD     glog[t,h]   = g[t,h]
//   PKDA_GATE_LOG_CHANNEL  glog[t,h,c] = g[t,h,c]
//   PKDA_GATE_RAW_CHANNEL  glog[t,h,c] = -exp(A_log[h]) softplus(g[t,h,c] + dt_bias[h*K+c])
//                          (delta_feedback_experiment/pkda.py:375-377)
#include <mutex>

#include "pkda_chunk_common.h"

namespace pkda {
namespace {

// ---- chunk table -------------------------------------------------------------
// One workgroup.  The caller's cu_seqlens is read here only: the table keeps a
// sanitised copy scu (nondecreasing, within [0, num_tokens]: the running
// maximum of cu clamped to that range), which every later kernel reads, so a
// malformed cu_seqlens cannot move any access outside the token tensors or
// the table.  flag = 1 when cu is not 0 = cu[0] <= ... <= cu[N] = num_tokens.
// Chunk counts come from scu and sum to at most ceil(num_tokens / 64) + N,
// the table's bound.
__global__ __launch_bounds__(kWG) void chunk_offsets_kernel(const int32_t* cu, int N, int num_tokens,
                                                            int32_t* offsets, int32_t* scu, int32_t* flag) {
  __shared__ int s_scan[kWG];
  __shared__ int s_max[kWG];
  __shared__ int s_bad;
  const int c0 = cu[0];
  const int first = min(max(c0, 0), num_tokens);
  if (threadIdx.x == 0) {
    s_bad = (c0 != 0) || (N == 0 && num_tokens != 0);
    scu[0] = first;
  }
  __syncthreads();  // s_bad's first value before any thread sets it
  int carry = 0;         // chunks before this tile
  int carry_max = first; // scu before this tile
  for (int base = 0; base < N; base += kWG) {
    const int n = base + threadIdx.x;
    int hi = carry_max;
    if (n < N) {
      const int a = cu[n], b = cu[n + 1];
      if (b < a || (n == N - 1 && b != num_tokens)) s_bad = 1;
      hi = min(max(b, 0), num_tokens);
    }
    s_max[threadIdx.x] = hi;
    __syncthreads();
    for (int off = 1; off < kWG; off <<= 1) {  // Hillis-Steele inclusive prefix maximum
      const int m = threadIdx.x >= off ? s_max[threadIdx.x - off] : hi;
      __syncthreads();
      hi = max(hi, m);
      s_max[threadIdx.x] = hi;
      __syncthreads();
    }
    const int end = max(hi, carry_max);                                          // scu[n + 1]
    const int start = threadIdx.x > 0 ? max(s_max[threadIdx.x - 1], carry_max) : carry_max;  // scu[n]
    int cnt = 0;
    if (n < N) {
      scu[n + 1] = end;
      cnt = (end - start + C - 1) / C;
    }
    __syncthreads();
    s_scan[threadIdx.x] = cnt;
    __syncthreads();
    for (int off = 1; off < kWG; off <<= 1) {  // Hillis-Steele inclusive scan
      const int add = threadIdx.x >= off ? s_scan[threadIdx.x - off] : 0;
      __syncthreads();
      s_scan[threadIdx.x] += add;
      __syncthreads();
    }
    if (n < N) offsets[n] = carry + s_scan[threadIdx.x] - cnt;
    carry += s_scan[kWG - 1];
    carry_max = max(carry_max, s_max[kWG - 1]);
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    offsets[N] = carry;
    *flag = s_bad;
  }
}

__global__ __launch_bounds__(kWG) void chunk_fill_kernel(const int32_t* scu, int N, const int32_t* offsets,
                                                         int num_chunks, int4* table) {
  const int c = blockIdx.x * kWG + threadIdx.x;
  if (c >= num_chunks) return;
  int4 e = make_int4(-1, 0, 0, 0);
  if (c < offsets[N]) {
    int lo = 0, hi = N - 1;  // last document whose first chunk id <= c
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (offsets[mid] <= c) lo = mid; else hi = mid - 1;
    }
    const int j = c - offsets[lo];
    const int start = scu[lo] + j * C;
    e = make_int4(lo, start, min(C, scu[lo + 1] - start), 0);
  }
  table[c] = e;
}

// Documents by length, longest first, ties by index: order[rank] = document.
// Each thread ranks its document against all others (a strict total order,
// so the ranks are a permutation), reading the lengths in LDS tiles.
__global__ __launch_bounds__(kWG) void chunk_order_kernel(const int32_t* cu, int N, int32_t* order) {  // cu: the sanitised copy
  __shared__ int s_len[kWG];
  const int n = blockIdx.x * kWG + threadIdx.x;
  const int len = n < N ? cu[n + 1] - cu[n] : 0;
  int rank = 0;
  for (int base = 0; base < N; base += kWG) {
    const int m = base + threadIdx.x;
    s_len[threadIdx.x] = m < N ? cu[m + 1] - cu[m] : 0;
    __syncthreads();
    const int cnt = min(kWG, N - base);
    for (int i = 0; i < cnt; ++i) {
      const int lm = s_len[i];
      rank += (lm > len) || (lm == len && base + i < n);
    }
    __syncthreads();
  }
  if (n < N) order[rank] = n;
}

// ---- gate forward --------------------------------------------------------------
struct GateParams {
  ChunkGeom geom;
  int heads, D, kind, g_dtype;
  const void* g;
  const float* A_log;
  const float* dt_bias;
  float* gcum;
  const float* dgcum;
  void* dg;  // FP32 except the per-channel backward with dg_dtype = g's dtype
  float* dA_log_part;
  float* ddt_bias_part;
  const void* up_weight;  // low-rank gate: [H*K, R]
  int rank, g_stride;
  int dg_dtype;  // per-channel backward: dg in FP32 or g's dtype
  float* gcum_lo;  // per-channel forward, optional: the FP32 residual of an FP64 cumsum
};

// Per-head form: one wave, lane t scans the chunk.
__global__ __launch_bounds__(64) void gate_fwd_kernel(GateParams p) {
  const int H = p.heads;
  const ChunkHead wg = chunk_head<true>(H);
  if (wg.cid >= p.geom.num_chunks) return;
  const ChunkInfo ci = chunk_info(p.geom, wg.cid);
  if (ci.len <= 0) return;
  const int h = wg.h;
  const int t = threadIdx.x;
  const int64_t idx = (int64_t)(ci.start + t) * H + h;
  float x = t < ci.len ? load_any(p.g, idx, p.g_dtype) : 0.f;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float y = __shfl_up(x, off);
    if (t >= off) x += y;
  }
  if (t < ci.len) p.gcum[idx] = x;
}

// Per-channel forms (log or raw), one lane per channel and chunk: a lane
// walks its chunk in groups of 16 tokens whose loads (indices clamped to the
// chunk's last token) go out before the scan runs over them, so the walk is
// not one memory latency per token.  Same arithmetic, in the same order, as
// a plain sequential scan.
template <typename G, bool RAW, int NT>
__global__ __launch_bounds__(NT) void gate_channel_fwd_kernel(GateParams p) {
  const ChunkHead wg = chunk_head<false>(p.heads);
  if (wg.cid >= p.geom.num_chunks) return;
  const ChunkInfo ci = chunk_info(p.geom, wg.cid);
  const int len = ci.len;
  if (len <= 0) return;
  const int h = wg.h, H = p.heads, D = p.D;
  const G* __restrict__ g = static_cast<const G*>(p.g);
  float* __restrict__ out = p.gcum;
  const float a_scale = RAW ? -expf(p.A_log[h]) : 0.f;
  const int64_t step = (int64_t)H * D;
  for (int c = threadIdx.x; c < D; c += NT) {
    const float bias = RAW ? p.dt_bias[h * D + c] : 0.f;
    const int64_t base = ((int64_t)ci.start * H + h) * D + c;
    if (p.gcum_lo) {  // FP64 cumsum, split into its FP32 rounding and the remainder
      double acc = 0.0;
      for (int t0 = 0; t0 < len; t0 += 16) {
        float x[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) x[u] = io<G>::load(g + base + (int64_t)min(t0 + u, len - 1) * step);
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          acc += (double)(RAW ? a_scale * softplus_sigmoid_fast(x[u] + bias).softplus : x[u]);
          const float hi = (float)acc;
          if (t0 + u < len) {
            out[base + (int64_t)(t0 + u) * step] = hi;
            p.gcum_lo[base + (int64_t)(t0 + u) * step] = (float)(acc - (double)hi);
          }
        }
      }
      continue;
    }
    float acc = 0.f;
    for (int t0 = 0; t0 < len; t0 += 16) {
      float x[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) x[u] = io<G>::load(g + base + (int64_t)min(t0 + u, len - 1) * step);
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        acc += RAW ? a_scale * softplus_sigmoid_fast(x[u] + bias).softplus : x[u];
        if (t0 + u < len) out[base + (int64_t)(t0 + u) * step] = acc;
      }
    }
  }
}

// ---- gate backward -------------------------------------------------------------
// dglog[t] = sum_{s >= t in chunk} dgcum[s]; raw form also
// dg = dglog * (-exp(A_log)) * sigmoid(g + dt_bias), dA_log += dglog * glog,
// ddt_bias += dg.  Per-chunk partials, reduced by gate_reduce_kernel.
__global__ __launch_bounds__(64) void gate_bwd_kernel(GateParams p) {
  const int H = p.heads;
  const ChunkHead wg = chunk_head<true>(H);
  if (wg.cid >= p.geom.num_chunks) return;
  const ChunkInfo ci = chunk_info(p.geom, wg.cid);
  if (ci.len <= 0) return;
  const int h = wg.h;
  const int t = threadIdx.x;
  const int64_t idx = (int64_t)(ci.start + t) * H + h;
  float x = t < ci.len ? p.dgcum[idx] : 0.f;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {  // suffix sum
    const float y = __shfl_down(x, off);
    if (t + off < 64) x += y;
  }
  if (t < ci.len) static_cast<float*>(p.dg)[idx] = x;
}

// Per-channel backward, grouped loads as in the forward (tokens walked last
// to first, indices clamped at 0).  The dA_log partial reduces over NT >= D
// lanes (a power of two) with the same halving tree a wider workgroup with
// zero-filled lanes would take.
template <typename G, bool RAW, int NT, typename DG>
__global__ __launch_bounds__(NT) void gate_channel_bwd_kernel(GateParams p) {
  __shared__ float s_red[NT];
  const ChunkHead wg = chunk_head<false>(p.heads);
  if (wg.cid >= p.geom.num_chunks) return;
  const ChunkInfo ci = chunk_info(p.geom, wg.cid);
  const int len = ci.len;
  const int h = wg.h, H = p.heads, D = p.D;
  const G* __restrict__ g = static_cast<const G*>(p.g);
  const float* __restrict__ dgcum = p.dgcum;
  DG* __restrict__ dg = reinterpret_cast<DG*>(p.dg);
  const float A = RAW ? expf(p.A_log[h]) : 0.f;
  const int64_t step = (int64_t)H * D;
  float dA_acc = 0.f;
  for (int c = threadIdx.x; c < D; c += NT) {
    const float bias = RAW ? p.dt_bias[h * D + c] : 0.f;
    const int64_t base = ((int64_t)ci.start * H + h) * D + c;
    float suffix = 0.f, ddt = 0.f;
    for (int tb = len - 1; tb >= 0; tb -= 16) {
      float dgc[16], x[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int64_t idx = base + (int64_t)max(tb - u, 0) * step;
        dgc[u] = dgcum[idx];
        if (RAW) x[u] = io<G>::load(g + idx);
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int t = tb - u;
        if (t < 0) break;
        const int64_t idx = base + (int64_t)t * step;
        suffix += dgc[u];
        if (RAW) {
          const SoftplusSigmoid f = softplus_sigmoid_fast(x[u] + bias);
          const float glog = -A * f.softplus;
          const float dgr = suffix * (-A) * f.sigmoid;
          io<DG>::store(dg + idx, dgr);
          dA_acc += suffix * glog;
          ddt += dgr;
        } else {
          io<DG>::store(dg + idx, suffix);
        }
      }
    }
    if (RAW) p.ddt_bias_part[((int64_t)wg.cid * H + h) * D + c] = len > 0 ? ddt : 0.f;
  }
  if (!RAW) return;
  s_red[threadIdx.x] = dA_acc;
  __syncthreads();
  for (int off = NT / 2; off > 0; off >>= 1) {
    if (threadIdx.x < off) s_red[threadIdx.x] += s_red[threadIdx.x + off];
    __syncthreads();
  }
  if (threadIdx.x == 0) p.dA_log_part[(int64_t)wg.cid * H + h] = s_red[0];
}

template <bool BWD, typename G, bool RAW>
void launch_gate_channel_nt(const GateParams& p, int num_chunks, hipStream_t s) {
  const dim3 grid(chunk_grid<false>(num_chunks, p.heads));
  const bool narrow = p.dg_dtype != PKDA_F32;  // backward: dg in G
  if (p.D <= 64) {
    if (!BWD) hipLaunchKernelGGL((gate_channel_fwd_kernel<G, RAW, 64>), grid, dim3(64), 0, s, p);
    else if (narrow) hipLaunchKernelGGL((gate_channel_bwd_kernel<G, RAW, 64, G>), grid, dim3(64), 0, s, p);
    else hipLaunchKernelGGL((gate_channel_bwd_kernel<G, RAW, 64, float>), grid, dim3(64), 0, s, p);
  } else if (p.D <= 128) {
    if (!BWD) hipLaunchKernelGGL((gate_channel_fwd_kernel<G, RAW, 128>), grid, dim3(128), 0, s, p);
    else if (narrow) hipLaunchKernelGGL((gate_channel_bwd_kernel<G, RAW, 128, G>), grid, dim3(128), 0, s, p);
    else hipLaunchKernelGGL((gate_channel_bwd_kernel<G, RAW, 128, float>), grid, dim3(128), 0, s, p);
  } else {
    if (!BWD) hipLaunchKernelGGL((gate_channel_fwd_kernel<G, RAW, 256>), grid, dim3(256), 0, s, p);
    else if (narrow) hipLaunchKernelGGL((gate_channel_bwd_kernel<G, RAW, 256, G>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((gate_channel_bwd_kernel<G, RAW, 256, float>), grid, dim3(256), 0, s, p);
  }
}

// Per-channel gate forms (PKDA_GATE_LOG_CHANNEL, PKDA_GATE_RAW_CHANNEL).
template <bool BWD>
void launch_gate_channel(const GateParams& p, int num_chunks, hipStream_t s) {
  const bool raw = p.kind == PKDA_GATE_RAW_CHANNEL;
  if (p.g_dtype == PKDA_BF16) {
    if (raw) launch_gate_channel_nt<BWD, bf16_t, true>(p, num_chunks, s);
    else launch_gate_channel_nt<BWD, bf16_t, false>(p, num_chunks, s);
  } else {
    if (raw) launch_gate_channel_nt<BWD, float, true>(p, num_chunks, s);
    else launch_gate_channel_nt<BWD, float, false>(p, num_chunks, s);
  }
}

// ---- low-rank gate: the decay expansion on MFMA, fused with the activation ----
// Per (chunk, head), one 4-wave workgroup, wave w owning rows 16w..16w+15:
//   raw[t, c] = sum_r hidden[t, r] up_weight[h K + c, r]
// as 16x16 MFMA tiles whose operands come straight from global memory (a lane
// reads 16 contiguous bytes of a hidden row or a weight row; the hidden rows
// are shared by every head of the chunk and the weights by every chunk, so
// both stay in L2), rounded to the activation dtype as the reference's
// materialised raw decay (F.linear output, delta_feedback_experiment/pkda.py:
// 334-339), then glog = -exp(A_log[h]) softplus(raw + dt_bias[h K + c]).  The
// chunk-local cumsum runs on the accumulators: over a lane's four rows, then
// across its wave's four lane groups (shuffles), then across the four waves
// (their totals through LDS); the result leaves with 16-byte row stores.  The
// backward recomputes raw the same way, reverse-scans dgcum and writes the raw
// gate's gradient; the two GEMMs back to the hidden rows and the weight are
// plain library products on the host side.  Rows past the chunk's end read
// the last valid row (every load stays inside the document) and are never
// stored or summed.
template <typename T> struct LrFrag;
template <> struct LrFrag<bf16_t> {  // 16x16x32: lane (i, q) holds k = 8q .. 8q + 7 of row i
  static constexpr int KS = 32;
  using F = s16x8_t;
  __device__ __forceinline__ static F load(const bf16_t* row, int k0, int lane) {
    return *reinterpret_cast<const s16x8_t*>(row + k0 + 8 * (lane >> 4));
  }
  __device__ __forceinline__ static void mfma(f32x4& acc, const F& a, const F& b) { Mma<bf16_t>::mfma(acc, a, b); }
};
template <> struct LrFrag<float> {  // 16x16x4: lane (i, q) holds k = q of row i
  static constexpr int KS = 4;
  using F = float;
  __device__ __forceinline__ static F load(const float* row, int k0, int lane) { return row[k0 + (lane >> 4)]; }
  __device__ __forceinline__ static void mfma(f32x4& acc, const F& a, const F& b) { Mma<float>::mfma(acc, a, b); }
};

// A workgroup takes kLrChunks chunks of one head: the head's weight rows
// [K x R] are staged in LDS once (row stride LDW) and read from there.
constexpr int kLrChunks = 4;
template <typename T, int R> struct LrW { static constexpr int LDW = R + Pad<T>::v; };

template <typename T, int K, int R>
__device__ __forceinline__ void stage_up_weight(const GateParams& p, int h, T* sW) {
  constexpr int V = 16 / (int)sizeof(T), LDW = LrW<T, R>::LDW;
  const T* wh = static_cast<const T*>(p.up_weight) + (int64_t)h * K * R;
  for (int i = threadIdx.x; i < K * R / V; i += kWG) {
    const int r = i / (R / V), c = (i - r * (R / V)) * V;
    *reinterpret_cast<uint4*>(sW + r * LDW + c) = *reinterpret_cast<const uint4*>(wh + (int64_t)r * R + c);
  }
}

// z = raw + dt_bias for this lane's accumulator elements: acc[ct][j] is row
// 16 wave + 4 q + j, column 16 ct + i.  sW: the head's weight in LDS.
template <typename T, int K, int R>
__device__ __forceinline__ void low_rank_z(const GateParams& p, const ChunkInfo& ci, int h, int wave, int lane,
                                           const T* sW, f32x4 (&acc)[K / 16]) {
  using Fr = LrFrag<T>;
  const int row = min(16 * wave + (lane & 15), ci.len - 1);
  const T* xrow = static_cast<const T*>(p.g) + (int64_t)(ci.start + row) * p.g_stride;
  typename Fr::F a[R / Fr::KS];
#pragma unroll
  for (int ks = 0; ks < R / Fr::KS; ++ks) a[ks] = Fr::load(xrow, ks * Fr::KS, lane);
#pragma unroll
  for (int ct = 0; ct < K / 16; ++ct) {
    const T* wrow = sW + (16 * ct + (lane & 15)) * LrW<T, R>::LDW;
    acc[ct] = zero4();
#pragma unroll
    for (int ks = 0; ks < R / Fr::KS; ++ks) Fr::mfma(acc[ct], a[ks], Fr::load(wrow, ks * Fr::KS, lane));
    const float bias = p.dt_bias[(int64_t)h * K + 16 * ct + (lane & 15)];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[ct][j] = from_e<T>(to_e<T>(acc[ct][j])) + bias;
  }
}

// Sum over the 64 lanes of a wave, fixed order; every lane gets the result.
__device__ __forceinline__ float lr_wave_sum(float x) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) x += __shfl_xor(x, off);
  return x;
}

// Inclusive prefix over this lane group's four rows and the lower lane groups
// of the wave (rows 4q + j ascending); returns the wave's column total.
__device__ __forceinline__ float wave_prefix_rows(f32x4& v, int lane) {
  v[1] += v[0];
  v[2] += v[1];
  v[3] += v[2];
  const int q = lane >> 4;
  float t = v[3];  // this group's total, then the inclusive prefix of the group totals
  float u = __shfl_up(t, 16);
  if (q >= 1) t += u;
  u = __shfl_up(t, 32);
  if (q >= 2) t += u;
  const float carry = t - v[3];
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] += carry;
  return __shfl(t, 48 + (lane & 15));  // group 3's inclusive value: the wave total
}

// The same inclusive prefix in FP64 (the gcum_lo form).
__device__ __forceinline__ double wave_prefix_rows_f64(double (&v)[4], int lane) {
  v[1] += v[0];
  v[2] += v[1];
  v[3] += v[2];
  const int q = lane >> 4;
  double t = v[3];
  double u = __shfl_up(t, 16);
  if (q >= 1) t += u;
  u = __shfl_up(t, 32);
  if (q >= 2) t += u;
  const double carry = t - v[3];
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] += carry;
  return __shfl(t, 48 + (lane & 15));
}

// Reverse (suffix) form: rows descending.
__device__ __forceinline__ float wave_suffix_rows(f32x4& v, int lane) {
  v[2] += v[3];
  v[1] += v[2];
  v[0] += v[1];
  const int q = lane >> 4;
  float t = v[0];
  float u = __shfl_down(t, 16);
  if (q <= 2) t += u;
  u = __shfl_down(t, 32);
  if (q <= 1) t += u;
  const float carry = t - v[0];
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] += carry;
  return __shfl(t, lane & 15);  // group 0's inclusive value: the wave total
}

template <typename T, int K, int R>
__global__ __launch_bounds__(kWG) void gate_low_rank_fwd_kernel(GateParams p) {
  __shared__ float s_tot[4][K];
  __shared__ double s_tot64[sizeof(T) == 4 ? 4 : 1][K];
  __shared__ __attribute__((aligned(16))) T sW[K * LrW<T, R>::LDW];
  const int h = blockIdx.y, H = p.heads;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  stage_up_weight<T, K, R>(p, h, sW);
  __syncthreads();
  const float a_scale = -expf(p.A_log[h]);
#pragma unroll 1
  for (int i = 0; i < kLrChunks; ++i) {
    const int c = blockIdx.x * kLrChunks + i;
    if (c >= p.geom.num_chunks) break;
    const ChunkInfo ci = chunk_info(p.geom, c);  // the same for every thread
    if (ci.len <= 0) continue;
    f32x4 acc[K / 16];
    low_rank_z<T, K, R>(p, ci, h, wave, lane, sW, acc);
    if constexpr (sizeof(T) == 4) {
      if (p.gcum_lo) {  // FP64 cumsum, split into its FP32 rounding and the remainder
        double v[K / 16][4];
#pragma unroll
        for (int ct = 0; ct < K / 16; ++ct) {
#pragma unroll
          for (int j = 0; j < 4; ++j) v[ct][j] = (double)(a_scale * softplus_sigmoid_fast(acc[ct][j]).softplus);
          const double tot = wave_prefix_rows_f64(v[ct], lane);
          if (lane < 16) s_tot64[wave][16 * ct + lane] = tot;
        }
        __syncthreads();
        const int64_t off = ((int64_t)ci.start * H + h) * K;
#pragma unroll
        for (int ct = 0; ct < K / 16; ++ct) {
          double carry = 0.0;
          for (int w = 0; w < wave; ++w) carry += s_tot64[w][16 * ct + (lane & 15)];
          f32x4 hi, lo;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const double x = v[ct][j] + carry;
            hi[j] = (float)x;
            lo[j] = (float)(x - (double)hi[j]);
          }
          store_acc_global<float>(p.gcum + off, (int64_t)H * K, hi, 16 * wave, 16 * ct, ci.len, lane);
          store_acc_global<float>(p.gcum_lo + off, (int64_t)H * K, lo, 16 * wave, 16 * ct, ci.len, lane);
        }
        __syncthreads();  // s_tot64 is read before the next chunk writes it
        continue;
      }
    }
#pragma unroll
    for (int ct = 0; ct < K / 16; ++ct) {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[ct][j] = a_scale * softplus_sigmoid_fast(acc[ct][j]).softplus;
      const float tot = wave_prefix_rows(acc[ct], lane);
      if (lane < 16) s_tot[wave][16 * ct + lane] = tot;
    }
    __syncthreads();
    float* out = p.gcum + ((int64_t)ci.start * H + h) * K;
#pragma unroll
    for (int ct = 0; ct < K / 16; ++ct) {
      float carry = 0.f;
      for (int w = 0; w < wave; ++w) carry += s_tot[w][16 * ct + (lane & 15)];
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[ct][j] += carry;
      store_acc_global<float>(out, (int64_t)H * K, acc[ct], 16 * wave, 16 * ct, ci.len, lane);
    }
    __syncthreads();  // s_tot is read before the next chunk writes it
  }
}

template <typename T, int K, int R>
__device__ __forceinline__ void gate_low_rank_bwd_chunk(const GateParams& p, const ChunkInfo& ci, int h, int H,
                                                        int wave, int lane, const T* sW, float A, float* dtb,
                                                        int cidx, float (&s_tot)[4][K], float (&s_col)[4][K],
                                                        float (&s_dA)[4]) {
  f32x4 z[K / 16];
  low_rank_z<T, K, R>(p, ci, h, wave, lane, sW, z);
  const int64_t base = ((int64_t)ci.start * H + h) * K;
  f32x4 suf[K / 16];
#pragma unroll
  for (int ct = 0; ct < K / 16; ++ct) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = 16 * wave + acc_row(lane, j);
      suf[ct][j] = r < ci.len ? p.dgcum[base + (int64_t)r * H * K + 16 * ct + acc_col(lane)] : 0.f;
    }
    const float tot = wave_suffix_rows(suf[ct], lane);
    if (lane < 16) s_tot[wave][16 * ct + lane] = tot;
  }
  __syncthreads();
  float dA = 0.f;
#pragma unroll
  for (int ct = 0; ct < K / 16; ++ct) {
    float carry = 0.f;
    for (int w = wave + 1; w < 4; ++w) carry += s_tot[w][16 * ct + (lane & 15)];
    f32x4 dg;
    float col = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool valid = 16 * wave + acc_row(lane, j) < ci.len;
      const float s = suf[ct][j] + carry;
      const SoftplusSigmoid f = softplus_sigmoid_fast(z[ct][j]);
      dg[j] = valid ? s * (-A) * f.sigmoid : 0.f;
      dA += valid ? s * (-A * f.softplus) : 0.f;
      col += dg[j];
    }
    store_acc_global<float>(static_cast<float*>(p.dg) + base, (int64_t)H * K, dg, 16 * wave, 16 * ct, ci.len, lane);
    col += __shfl_xor(col, 16);
    col += __shfl_xor(col, 32);
    if (lane < 16) s_col[wave][16 * ct + lane] = col;
  }
  dA = lr_wave_sum(dA);
  if (lane == 0) s_dA[wave] = dA;
  __syncthreads();
  for (int c = threadIdx.x; c < K; c += kWG) dtb[c] = ((s_col[0][c] + s_col[1][c]) + s_col[2][c]) + s_col[3][c];
  if (threadIdx.x == 0) p.dA_log_part[(int64_t)cidx * H + h] = ((s_dA[0] + s_dA[1]) + s_dA[2]) + s_dA[3];
}

template <typename T, int K, int R>
__global__ __launch_bounds__(kWG) void gate_low_rank_bwd_kernel(GateParams p) {
  __shared__ float s_tot[4][K];
  __shared__ float s_col[4][K];
  __shared__ float s_dA[4];
  __shared__ __attribute__((aligned(16))) T sW[K * LrW<T, R>::LDW];
  const int h = blockIdx.y, H = p.heads;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  stage_up_weight<T, K, R>(p, h, sW);
  __syncthreads();
  const float A = expf(p.A_log[h]);
  // ci is the same for every thread, so every thread reaches every barrier;
  // a chunk reads s_tot before its second barrier and s_col, s_dA after it,
  // and the next chunk writes them only after reaching its own first barrier
#pragma unroll 1
  for (int i = 0; i < kLrChunks; ++i) {
    const int cidx = blockIdx.x * kLrChunks + i;
    if (cidx >= p.geom.num_chunks) break;
    const ChunkInfo ci = chunk_info(p.geom, cidx);
    float* dtb = p.ddt_bias_part + ((int64_t)cidx * H + h) * K;
    if (ci.len <= 0) {  // an empty slot of the packed launch bound: zero partials
      for (int c = threadIdx.x; c < K; c += kWG) dtb[c] = 0.f;
      if (threadIdx.x == 0) p.dA_log_part[(int64_t)cidx * H + h] = 0.f;
      continue;
    }
    gate_low_rank_bwd_chunk<T, K, R>(p, ci, h, H, wave, lane, sW, A, dtb, cidx, s_tot, s_col, s_dA);
  }
}

int dispatch_low_rank(const GateParams& p, int num_chunks, bool backward, hipStream_t s) {
  if (num_chunks <= 0) return 0;
  const dim3 grid((num_chunks + kLrChunks - 1) / kLrChunks, p.heads);
#define PKDA_LOW_RANK(TT, KK)                                                                       \
  do {                                                                                              \
    if (backward) {                                                                                 \
      hipLaunchKernelGGL((gate_low_rank_bwd_kernel<TT, KK, KK>), grid, dim3(kWG), 0, s, p);         \
    } else {                                                                                        \
      hipLaunchKernelGGL((gate_low_rank_fwd_kernel<TT, KK, KK>), grid, dim3(kWG), 0, s, p);         \
    }                                                                                               \
  } while (0)
  if (p.g_dtype == PKDA_BF16) {
    if (p.D == 128) PKDA_LOW_RANK(bf16_t, 128); else PKDA_LOW_RANK(bf16_t, 64);
  } else {
    PKDA_LOW_RANK(float, 64);
  }
#undef PKDA_LOW_RANK
  return launch_status(backward ? "pkda_gate_bwd(low rank)" : "pkda_gate_fwd(low rank)");
}

int gate_common(const pkda_gate_args* a, GateParams& p) {
  PKDA_REQUIRE(a != nullptr, PKDA_EINVAL, "null args");
  PKDA_REQUIRE(a->struct_size == (int32_t)sizeof(pkda_gate_args), PKDA_EINVAL, "pkda_gate_args size mismatch");
  PKDA_REQUIRE(a->gate_kind >= 0 && a->gate_kind <= 3, PKDA_EINVAL, "gate_kind %d", a->gate_kind);
  PKDA_REQUIRE(a->g_dtype == PKDA_F32 || a->g_dtype == PKDA_BF16, PKDA_EUNSUPPORTED, "g dtype");
  PKDA_REQUIRE(a->heads > 0 && a->head_dim > 0 && a->num_seqs >= 0 && a->num_chunks >= 0, PKDA_EINVAL, "sizes");
  PKDA_REQUIRE(!a->cu_seqlens || a->table, PKDA_EINVAL, "packed documents need the chunk table");
  PKDA_REQUIRE(a->gate_kind < PKDA_GATE_RAW_CHANNEL || (a->A_log && a->dt_bias), PKDA_EINVAL,
               "raw and low-rank gates need A_log, dt_bias");
  if (a->gate_kind == PKDA_GATE_LOW_RANK) {
    PKDA_REQUIRE(a->up_weight, PKDA_EINVAL, "the low-rank gate needs up_weight");
    PKDA_REQUIRE(a->rank == a->head_dim && (a->head_dim == 64 || (a->head_dim == 128 && a->g_dtype == PKDA_BF16)),
                 PKDA_EUNSUPPORTED, "low-rank gate built for rank == head_dim in {64, 128} (128: bf16)");
    const int vec = a->g_dtype == PKDA_BF16 ? 8 : 4;
    PKDA_REQUIRE(a->g_stride >= a->rank && a->g_stride % vec == 0, PKDA_EINVAL,
                 "g_stride %d (>= rank, a multiple of %d elements)", a->g_stride, vec);
  }
  p.geom.num_seqs = a->num_seqs;
  p.geom.seqlen = a->seqlen;
  p.geom.nt = a->cu_seqlens ? 0 : (a->seqlen + C - 1) / C;
  p.geom.table = reinterpret_cast<const int4*>(a->table);
  p.geom.offsets = a->table ? a->table + 4 * a->num_chunks : nullptr;
  p.geom.order = a->table ? p.geom.offsets + a->num_seqs + 1 : nullptr;
  p.geom.cu = a->cu_seqlens && a->table ? p.geom.order + a->num_seqs : nullptr;  // the table's sanitised copy
  p.geom.num_chunks = a->num_chunks;
  PKDA_REQUIRE(a->cu_seqlens || a->num_chunks == a->num_seqs * p.geom.nt, PKDA_EINVAL,
               "num_chunks %d != num_seqs * ceil(seqlen / 64)", a->num_chunks);
  p.heads = a->heads;
  p.D = a->head_dim;
  p.kind = a->gate_kind;
  p.g_dtype = a->g_dtype;
  p.g = a->g;
  p.A_log = a->A_log;
  p.dt_bias = a->dt_bias;
  p.gcum = a->gcum;
  p.dgcum = a->dgcum;
  p.dg = a->dg;
  p.dg_dtype = a->dg_dtype;
  p.dA_log_part = a->dA_log_part;
  p.ddt_bias_part = a->ddt_bias_part;
  p.up_weight = a->up_weight;
  p.rank = a->rank;
  p.g_stride = a->g_stride;
  p.gcum_lo = a->gcum_lo;
  return 0;
}

}  // namespace
}  // namespace pkda

using namespace pkda;

extern "C" int pkda_chunk_table(const int32_t* cu_seqlens, int32_t num_seqs, int32_t num_tokens,
                                int32_t num_chunks_max, int32_t* table, void* stream) {
  PKDA_REQUIRE(cu_seqlens && table && num_seqs >= 0 && num_tokens >= 0 && num_chunks_max >= 0, PKDA_EINVAL,
               "chunk table arguments");
  PKDA_REQUIRE(num_chunks_max >= (num_tokens + C - 1) / C + num_seqs, PKDA_EINVAL,
               "num_chunks_max %d < ceil(num_tokens / 64) + num_seqs", num_chunks_max);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int32_t* offsets = table + 4 * num_chunks_max;
  int32_t* order = offsets + num_seqs + 1;
  int32_t* scu = order + num_seqs;
  int32_t* flag = scu + num_seqs + 1;
  hipLaunchKernelGGL(chunk_offsets_kernel, dim3(1), dim3(kWG), 0, s, cu_seqlens, num_seqs, num_tokens, offsets, scu,
                     flag);
  if (num_chunks_max > 0)
    hipLaunchKernelGGL(chunk_fill_kernel, dim3((num_chunks_max + kWG - 1) / kWG), dim3(kWG), 0, s, scu, num_seqs,
                       offsets, num_chunks_max, reinterpret_cast<int4*>(table));
  if (num_seqs > 0)
    hipLaunchKernelGGL(chunk_order_kernel, dim3((num_seqs + kWG - 1) / kWG), dim3(kWG), 0, s, scu, num_seqs, order);
  return launch_status("pkda_chunk_table");
}

extern "C" int pkda_gate_fwd(const pkda_gate_args* a, void* stream) {
  GateParams p;
  int st = gate_common(a, p);
  if (st) return st;
  PKDA_REQUIRE(a->g && a->gcum, PKDA_EINVAL, "gate forward needs g and gcum");
  PKDA_REQUIRE(!a->gcum_lo || a->gate_kind != PKDA_GATE_LOG_HEAD, PKDA_EUNSUPPORTED,
               "gcum_lo is formed for the per-channel gate forms");
  if (a->num_chunks == 0) return 0;
  if (a->gate_kind == PKDA_GATE_LOW_RANK)
    return dispatch_low_rank(p, a->num_chunks, false, static_cast<hipStream_t>(stream));
  if (a->gate_kind == PKDA_GATE_LOG_HEAD)
    hipLaunchKernelGGL(gate_fwd_kernel, dim3(chunk_grid<true>(a->num_chunks, a->heads)), dim3(64), 0,
                       static_cast<hipStream_t>(stream), p);
  else
    launch_gate_channel<false>(p, a->num_chunks, static_cast<hipStream_t>(stream));
  return launch_status("pkda_gate_fwd");
}

namespace pkda {
namespace {

// The gate backward.  For the raw and low-rank forms the per-chunk partials
// of dA_log [num_chunks, H] and ddt_bias [num_chunks, H*K] go to dA_part and
// ddt_part: every slot is written on every call (empty chunks write zeros), so
// nothing there needs clearing first.
int gate_bwd_impl(const pkda_gate_args* a, float* dA_part, float* ddt_part, hipStream_t s) {
  GateParams p;
  int st = gate_common(a, p);
  if (st) return st;
  p.dA_log_part = dA_part;
  p.ddt_bias_part = ddt_part;
  PKDA_REQUIRE(a->dgcum && a->dg, PKDA_EINVAL, "gate backward needs dgcum and dg");
  PKDA_REQUIRE(a->dg_dtype == PKDA_F32 ||
                   (a->dg_dtype == a->g_dtype &&
                    (a->gate_kind == PKDA_GATE_LOG_CHANNEL || a->gate_kind == PKDA_GATE_RAW_CHANNEL)),
               PKDA_EUNSUPPORTED, "dg_dtype %d: FP32, or g's dtype for the per-channel gate forms", a->dg_dtype);
  const bool raw = a->gate_kind >= PKDA_GATE_RAW_CHANNEL;
  PKDA_REQUIRE(!raw || (a->g && dA_part && ddt_part && a->dA_log && a->ddt_bias), PKDA_EINVAL,
               "raw gate backward needs g and the dA_log / ddt_bias buffers");
  if (a->num_chunks > 0) {
    if (a->gate_kind == PKDA_GATE_LOW_RANK) {
      if (int e = dispatch_low_rank(p, a->num_chunks, true, s)) return e;
    } else if (a->gate_kind == PKDA_GATE_LOG_HEAD) {
      hipLaunchKernelGGL(gate_bwd_kernel, dim3(chunk_grid<true>(a->num_chunks, a->heads)), dim3(64), 0, s, p);
    } else {
      launch_gate_channel<true>(p, a->num_chunks, s);
    }
  }
  if (raw) {
    const int nH = a->heads, nHK = a->heads * a->head_dim;
    hipLaunchKernelGGL(sum_partials_tree_kernel, dim3(nH), dim3(256), 0, s, dA_part, a->num_chunks, nH, a->dA_log);
    hipLaunchKernelGGL(sum_partials_tree_kernel, dim3(nHK), dim3(256), 0, s, ddt_part, a->num_chunks, nHK,
                       a->ddt_bias);
  }
  return launch_status("pkda_gate_bwd");
}

// ---- the gate backward without a caller workspace ------------------------------
// pkda_gate_bwd_noalloc keeps the partials in this device array instead of
// the caller's dA_log_part / ddt_bias_part.  Each device holds its own copy
// until the process ends.  In host code `scratch` names a host-side stand-in,
// not the device address: the address comes from hipGetSymbolAddress, once
// per device with that device current, and only that address is used.
constexpr int64_t kGateScratchFloats = PKDA_GATE_BWD_NOALLOC_MAX_FLOATS;
static __device__ __align__(256) float scratch[kGateScratchFloats];

constexpr int kMaxDevices = 64;
float* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

int device_scratch(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("hipGetDevice: %s", hipGetErrorString(e));
    return static_cast<int>(e);
  }
  PKDA_REQUIRE(dev >= 0 && dev < kMaxDevices, PKDA_EUNSUPPORTED, "device %d (at most %d devices)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_error("hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
      return e != hipSuccess ? static_cast<int>(e) : static_cast<int>(hipErrorInvalidSymbol);
    }
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace
}  // namespace pkda

extern "C" int pkda_gate_bwd(const pkda_gate_args* a, void* stream) {
  PKDA_REQUIRE(a != nullptr, PKDA_EINVAL, "null args");
  return gate_bwd_impl(a, a->dA_log_part, a->ddt_bias_part, static_cast<hipStream_t>(stream));
}

extern "C" int pkda_gate_bwd_noalloc(const pkda_gate_args* a, void* stream) {
  PKDA_REQUIRE(a != nullptr, PKDA_EINVAL, "null args");
  PKDA_REQUIRE(a->num_chunks >= 0 && a->heads > 0 && a->head_dim > 0, PKDA_EINVAL, "sizes");
  if (a->gate_kind < PKDA_GATE_RAW_CHANNEL)  // no partials: nothing to place
    return gate_bwd_impl(a, nullptr, nullptr, static_cast<hipStream_t>(stream));
  const int64_t nH = (int64_t)a->num_chunks * a->heads;
  const int64_t need = nH * (1 + (int64_t)a->head_dim);
  PKDA_REQUIRE(need <= pkda::kGateScratchFloats, PKDA_ERANGE,
               "pkda_gate_bwd_noalloc: num_chunks * heads * (head_dim + 1) = %lld floats exceeds its scratch of "
               "%lld floats; use pkda_gate_bwd with a workspace",
               (long long)need, (long long)pkda::kGateScratchFloats);
  float* base = nullptr;
  if (int st = pkda::device_scratch(&base)) return st;
  return gate_bwd_impl(a, base, base + nH, static_cast<hipStream_t>(stream));
}
