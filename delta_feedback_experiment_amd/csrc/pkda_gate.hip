// Chunk table for packed documents, and the gate's chunk-local cumulative
// log-decay (forward) and reverse cumsum + activation gradients (backward).
//
// Gate forms (natural log throughout):
//   PKDA_GATE_LOG_HEAD     glog[t,h]   = g[t,h]
//   PKDA_GATE_LOG_CHANNEL  glog[t,h,c] = g[t,h,c]
//   PKDA_GATE_RAW_CHANNEL  glog[t,h,c] = -exp(A_log[h]) softplus(g[t,h,c] + dt_bias[h*K+c])
//                          (delta_feedback_experiment/pkda.py:375-377)
#include "pkda_chunk_common.h"

namespace pkda {
namespace {

// ---- chunk table -------------------------------------------------------------
__global__ __launch_bounds__(kWG) void chunk_offsets_kernel(const int32_t* cu, int N, int32_t* offsets) {
  __shared__ int s_scan[kWG];
  int carry = 0;
  for (int base = 0; base < N; base += kWG) {
    const int n = base + threadIdx.x;
    int cnt = 0;
    if (n < N) {
      const int len = cu[n + 1] - cu[n];
      cnt = len > 0 ? (len + C - 1) / C : 0;
    }
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
    __syncthreads();
  }
  if (threadIdx.x == 0) offsets[N] = carry;
}

__global__ __launch_bounds__(kWG) void chunk_fill_kernel(const int32_t* cu, int N, const int32_t* offsets,
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
    const int start = cu[lo] + j * C;
    e = make_int4(lo, start, min(C, cu[lo + 1] - start), 0);
  }
  table[c] = e;
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
  float* dg;
  float* dA_log_part;
  float* ddt_bias_part;
};

__device__ __forceinline__ float gate_value(const GateParams& p, int64_t idx, int h, int c, float a_scale) {
  const float x = load_any(p.g, idx, p.g_dtype);
  if (p.kind == PKDA_GATE_RAW_CHANNEL) return a_scale * softplus_f(x + p.dt_bias[h * p.D + c]);
  return x;
}

__global__ __launch_bounds__(kWG) void gate_fwd_kernel(GateParams p) {
  const ChunkInfo ci = chunk_info(p.geom, blockIdx.x);
  if (ci.len <= 0) return;
  const int h = blockIdx.y;
  const int H = p.heads;
  if (p.kind == PKDA_GATE_LOG_HEAD) {
    // one wave: lane t scans the chunk
    if (threadIdx.x >= 64) return;
    const int t = threadIdx.x;
    const int64_t idx = (int64_t)(ci.start + t) * H + h;
    float x = t < ci.len ? load_any(p.g, idx, p.g_dtype) : 0.f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(x, off);
      if (t >= off) x += y;
    }
    if (t < ci.len) p.gcum[idx] = x;
    return;
  }
  const float a_scale = p.kind == PKDA_GATE_RAW_CHANNEL ? -expf(p.A_log[h]) : 0.f;
  for (int c = threadIdx.x; c < p.D; c += kWG) {
    float acc = 0.f;
    for (int t = 0; t < ci.len; ++t) {
      const int64_t idx = ((int64_t)(ci.start + t) * H + h) * p.D + c;
      acc += gate_value(p, idx, h, c, a_scale);
      p.gcum[idx] = acc;
    }
  }
}

// ---- gate backward -------------------------------------------------------------
// dglog[t] = sum_{s >= t in chunk} dgcum[s]; raw form also
// dg = dglog * (-exp(A_log)) * sigmoid(g + dt_bias), dA_log += dglog * glog,
// ddt_bias += dg.  Per-chunk partials, reduced by gate_reduce_kernel.
__global__ __launch_bounds__(kWG) void gate_bwd_kernel(GateParams p) {
  const ChunkInfo ci = chunk_info(p.geom, blockIdx.x);
  const int h = blockIdx.y;
  const int H = p.heads;
  const bool raw = p.kind == PKDA_GATE_RAW_CHANNEL;
  if (p.kind == PKDA_GATE_LOG_HEAD) {
    if (ci.len <= 0 || threadIdx.x >= 64) return;
    const int t = threadIdx.x;
    const int64_t idx = (int64_t)(ci.start + t) * H + h;
    float x = t < ci.len ? p.dgcum[idx] : 0.f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {  // suffix sum
      const float y = __shfl_down(x, off);
      if (t + off < 64) x += y;
    }
    if (t < ci.len) p.dg[idx] = x;
    return;
  }
  __shared__ float s_red[kWG];
  const float A = raw ? expf(p.A_log[h]) : 0.f;
  float dA_acc = 0.f;
  for (int c = threadIdx.x; c < p.D; c += kWG) {
    float suffix = 0.f;
    float ddt = 0.f;
    for (int t = ci.len - 1; t >= 0; --t) {
      const int64_t idx = ((int64_t)(ci.start + t) * H + h) * p.D + c;
      suffix += p.dgcum[idx];
      if (raw) {
        const float z = load_any(p.g, idx, p.g_dtype) + p.dt_bias[h * p.D + c];
        const float glog = -A * softplus_f(z);
        const float dgr = suffix * (-A) * sigmoid_f(z);
        p.dg[idx] = dgr;
        dA_acc += suffix * glog;
        ddt += dgr;
      } else {
        p.dg[idx] = suffix;
      }
    }
    if (raw) p.ddt_bias_part[((int64_t)blockIdx.x * H + h) * p.D + c] = ci.len > 0 ? ddt : 0.f;
  }
  if (!raw) return;
  s_red[threadIdx.x] = dA_acc;
  __syncthreads();
  for (int off = kWG / 2; off > 0; off >>= 1) {
    if (threadIdx.x < off) s_red[threadIdx.x] += s_red[threadIdx.x + off];
    __syncthreads();
  }
  if (threadIdx.x == 0) p.dA_log_part[(int64_t)blockIdx.x * H + h] = s_red[0];
}

// out[i] = sum_c part[c * n + i] for c in [0, num_chunks), fixed order.
__global__ __launch_bounds__(kWG) void sum_partials_kernel(const float* part, int num_chunks, int n, float* out) {
  const int i = blockIdx.x * kWG + threadIdx.x;
  if (i >= n) return;
  float s = 0.f;
  for (int c = 0; c < num_chunks; ++c) s += part[(int64_t)c * n + i];
  out[i] = s;
}

int gate_common(const pkda_gate_args* a, GateParams& p) {
  PKDA_REQUIRE(a != nullptr, PKDA_EINVAL, "null args");
  PKDA_REQUIRE(a->struct_size == (int32_t)sizeof(pkda_gate_args), PKDA_EINVAL, "pkda_gate_args size mismatch");
  PKDA_REQUIRE(a->gate_kind >= 0 && a->gate_kind <= 2, PKDA_EINVAL, "gate_kind %d", a->gate_kind);
  PKDA_REQUIRE(a->g_dtype == PKDA_F32 || a->g_dtype == PKDA_BF16, PKDA_EUNSUPPORTED, "g dtype");
  PKDA_REQUIRE(a->heads > 0 && a->head_dim > 0 && a->num_seqs >= 0 && a->num_chunks >= 0, PKDA_EINVAL, "sizes");
  PKDA_REQUIRE(!a->cu_seqlens || a->table, PKDA_EINVAL, "packed documents need the chunk table");
  PKDA_REQUIRE(a->gate_kind != PKDA_GATE_RAW_CHANNEL || (a->A_log && a->dt_bias), PKDA_EINVAL, "raw gate needs A_log, dt_bias");
  p.geom.num_seqs = a->num_seqs;
  p.geom.seqlen = a->seqlen;
  p.geom.nt = a->cu_seqlens ? 0 : (a->seqlen + C - 1) / C;
  p.geom.cu = a->cu_seqlens;
  p.geom.table = reinterpret_cast<const int4*>(a->table);
  p.geom.offsets = a->table ? a->table + 4 * a->num_chunks : nullptr;
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
  p.dA_log_part = a->dA_log_part;
  p.ddt_bias_part = a->ddt_bias_part;
  return 0;
}

}  // namespace
}  // namespace pkda

using namespace pkda;

extern "C" int pkda_chunk_table(const int32_t* cu_seqlens, int32_t num_seqs, int32_t num_chunks_max, int32_t* table,
                                void* stream) {
  PKDA_REQUIRE(cu_seqlens && table && num_seqs >= 0 && num_chunks_max >= 0, PKDA_EINVAL, "chunk table arguments");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int32_t* offsets = table + 4 * num_chunks_max;
  hipLaunchKernelGGL(chunk_offsets_kernel, dim3(1), dim3(kWG), 0, s, cu_seqlens, num_seqs, offsets);
  if (num_chunks_max > 0)
    hipLaunchKernelGGL(chunk_fill_kernel, dim3((num_chunks_max + kWG - 1) / kWG), dim3(kWG), 0, s, cu_seqlens,
                       num_seqs, offsets, num_chunks_max, reinterpret_cast<int4*>(table));
  return launch_status("pkda_chunk_table");
}

extern "C" int pkda_gate_fwd(const pkda_gate_args* a, void* stream) {
  GateParams p;
  int st = gate_common(a, p);
  if (st) return st;
  PKDA_REQUIRE(a->g && a->gcum, PKDA_EINVAL, "gate forward needs g and gcum");
  if (a->num_chunks == 0) return 0;
  hipLaunchKernelGGL(gate_fwd_kernel, dim3(a->num_chunks, a->heads), dim3(kWG), 0, static_cast<hipStream_t>(stream), p);
  return launch_status("pkda_gate_fwd");
}

extern "C" int pkda_gate_bwd(const pkda_gate_args* a, void* stream) {
  GateParams p;
  int st = gate_common(a, p);
  if (st) return st;
  PKDA_REQUIRE(a->dgcum && a->dg, PKDA_EINVAL, "gate backward needs dgcum and dg");
  const bool raw = a->gate_kind == PKDA_GATE_RAW_CHANNEL;
  PKDA_REQUIRE(!raw || (a->g && a->dA_log_part && a->ddt_bias_part && a->dA_log && a->ddt_bias), PKDA_EINVAL,
               "raw gate backward needs g and the dA_log / ddt_bias buffers");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->num_chunks > 0)
    hipLaunchKernelGGL(gate_bwd_kernel, dim3(a->num_chunks, a->heads), dim3(kWG), 0, s, p);
  if (raw) {
    const int nH = a->heads, nHK = a->heads * a->head_dim;
    hipLaunchKernelGGL(sum_partials_kernel, dim3((nH + kWG - 1) / kWG), dim3(kWG), 0, s, a->dA_log_part,
                       a->num_chunks, nH, a->dA_log);
    hipLaunchKernelGGL(sum_partials_kernel, dim3((nHK + kWG - 1) / kWG), dim3(kWG), 0, s, a->ddt_bias_part,
                       a->num_chunks, nHK, a->ddt_bias);
  }
  return launch_status("pkda_gate_bwd");
}
