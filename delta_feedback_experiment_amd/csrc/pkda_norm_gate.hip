// RMSNorm with a sigmoid output gate for gfx950, forward and backward: the
// consumer of the PKDA recurrence's output.
//
// Reference: delta_feedback::pkda_norm_gate and its backward op
// (delta_feedback_experiment/fla_ops.py:572-657), called by
// PreconditionedKDA.forward on the recurrence output o [B, T, H, d] with the
// gate logits [B, T, H, d] and output_norm [d]
// (delta_feedback_experiment/pkda.py:536-547).  Per row r (one head of one
// token) of width d:
//
//   rstd[r] = 1 / sqrt(mean_c x[r, c]^2 + eps)
//   y[r, c] = x[r, c] rstd[r] weight[c] sigmoid(gate[r, c])
//
// in FP32, rounded once to the activation dtype; rstd (FP32) feeds the
// backward.  With n = x rstd, s = sigmoid(gate), dy the output gradient:
//
//   dgate  = dy n weight s (1 - s)
//   dn     = dy s weight,   dx = rstd (dn - n mean_c(dn n))
//   dweight[c] = sum_r dy s n
//
// One row is d / 8 lanes of 16-byte vectors; the row reductions are shuffles
// over those lanes.  dweight is summed per thread over its rows, then per
// workgroup in LDS and over workgroups by a second kernel, each in a fixed
// order (deterministic).
#include "pkda_common.h"

namespace pkda {
namespace {

constexpr int kNgThreads = 256;
constexpr int kNgBlocks = 1024;  // workgroups of the row loop (dweight partials)

struct NgParams {
  const void* x;
  const void* gate;
  const void* weight;
  int w_dtype;
  float eps;
  void* y;
  float* rstd;
  const void* dy;
  void* dx;
  void* dgate;
  float* dw_part;  // [blocks, d]
  void* dw;
  int64_t rows;
  int blocks;
};

template <typename T> struct V8;
template <> struct V8<bf16_t> {
  __device__ __forceinline__ static void load(const bf16_t* p, float* x) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static void store(bf16_t* p, const float* x) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = static_cast<uint32_t>(f32_to_bf16(x[2 * i])) | (static_cast<uint32_t>(f32_to_bf16(x[2 * i + 1])) << 16);
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
};
template <> struct V8<float> {
  __device__ __forceinline__ static void load(const float* p, float* x) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  }
  __device__ __forceinline__ static void store(float* p, const float* x) {
    *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(x[4], x[5], x[6], x[7]);
  }
};

// Sum over the L lanes of one row (L a power of two, lanes aligned to L; the
// lanes of a row are active together).
template <int L>
__device__ __forceinline__ float row_sum(float x) {
  if constexpr (L <= 16) {
    return lane_group_sum<L>(x);
  } else {
#pragma unroll
    for (int off = 1; off < L; off <<= 1) x += __shfl_xor(x, off);
    return x;
  }
}

__device__ __forceinline__ float sigm(float a) { return 1.f / (1.f + __expf(-a)); }

// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(kNgThreads) void norm_gate_fwd_kernel(NgParams p) {
  constexpr int L = D / 8;                  // lanes per row
  constexpr int RPB = kNgThreads / L;       // rows per workgroup step
  const int lane_in_row = threadIdx.x % L;
  const int c0 = 8 * lane_in_row;
  float w[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) w[j] = load_any(p.weight, c0 + j, p.w_dtype);
  const T* xs = static_cast<const T*>(p.x);
  const T* gs = static_cast<const T*>(p.gate);
  T* ys = static_cast<T*>(p.y);
  for (int64_t r = (int64_t)blockIdx.x * RPB + threadIdx.x / L; r < p.rows; r += (int64_t)gridDim.x * RPB) {
    float x[8], g[8];
    V8<T>::load(xs + r * D + c0, x);
    V8<T>::load(gs + r * D + c0, g);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
    const float rs = rsqrtf(row_sum<L>(ss) / D + p.eps);
    float y[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) y[j] = x[j] * rs * w[j] * sigm(g[j]);
    V8<T>::store(ys + r * D + c0, y);
    if (lane_in_row == 0) p.rstd[r] = rs;
  }
}

template <typename T, int D>
__global__ __launch_bounds__(kNgThreads) void norm_gate_bwd_kernel(NgParams p) {
  constexpr int L = D / 8;
  constexpr int RPB = kNgThreads / L;
  __shared__ float s_dw[kNgThreads * 8];
  const int lane_in_row = threadIdx.x % L;
  const int c0 = 8 * lane_in_row;
  float w[8], dw[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    w[j] = load_any(p.weight, c0 + j, p.w_dtype);
    dw[j] = 0.f;
  }
  const T* xs = static_cast<const T*>(p.x);
  const T* gs = static_cast<const T*>(p.gate);
  const T* dys = static_cast<const T*>(p.dy);
  T* dxs = static_cast<T*>(p.dx);
  T* dgs = static_cast<T*>(p.dgate);
  for (int64_t r = (int64_t)blockIdx.x * RPB + threadIdx.x / L; r < p.rows; r += (int64_t)gridDim.x * RPB) {
    float x[8], g[8], dy[8];
    V8<T>::load(xs + r * D + c0, x);
    V8<T>::load(gs + r * D + c0, g);
    V8<T>::load(dys + r * D + c0, dy);
    const float rs = p.rstd[r];
    float n[8], dn[8], dg[8];
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      n[j] = x[j] * rs;
      const float s = sigm(g[j]);
      dg[j] = dy[j] * n[j] * w[j] * s * (1.f - s);
      const float dys_ = dy[j] * s;
      dw[j] += dys_ * n[j];
      dn[j] = dys_ * w[j];
      dot += dn[j] * n[j];
    }
    dot = row_sum<L>(dot) / D;
    float dx[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) dx[j] = rs * (dn[j] - n[j] * dot);
    V8<T>::store(dxs + r * D + c0, dx);
    V8<T>::store(dgs + r * D + c0, dg);
  }
  // dweight: this workgroup's rows, summed over its row slots in order
#pragma unroll
  for (int j = 0; j < 8; ++j) s_dw[threadIdx.x * 8 + j] = dw[j];
  __syncthreads();
  if (threadIdx.x < D) {
    const int c = threadIdx.x, li = c / 8, j = c % 8;
    float s = 0.f;
    for (int rr = 0; rr < RPB; ++rr) s += s_dw[(rr * L + li) * 8 + j];
    p.dw_part[(int64_t)blockIdx.x * D + c] = s;
  }
}

// dweight[c] = sum over workgroups of dw_part[b, c] in a fixed order, in two
// passes: slice y sums workgroups y, y + S, ... into dw_part[y] (only this
// thread reads that entry), then the S slice sums are added in order.
constexpr int kNgSlices = 32;

template <int D>
__global__ __launch_bounds__(D) void norm_gate_dw_slices_kernel(NgParams p, int S) {
  const int c = threadIdx.x, y = blockIdx.x;
  float s = 0.f;
  for (int b = y; b < p.blocks; b += S) s += p.dw_part[(int64_t)b * D + c];
  p.dw_part[(int64_t)y * D + c] = s;
}

template <int D>
__global__ __launch_bounds__(D) void norm_gate_dw_kernel(NgParams p, int S) {
  const int c = threadIdx.x;
  float s = 0.f;
  for (int y = 0; y < S; ++y) s += p.dw_part[(int64_t)y * D + c];
  if (p.w_dtype == PKDA_BF16) {
    static_cast<bf16_t*>(p.dw)[c] = f32_to_bf16(s);
  } else {
    static_cast<float*>(p.dw)[c] = s;
  }
}

template <typename T, int D>
int launch_ng(const NgParams& p, bool backward, hipStream_t s) {
  if (!backward) {
    hipLaunchKernelGGL((norm_gate_fwd_kernel<T, D>), dim3(p.blocks), dim3(kNgThreads), 0, s, p);
    return launch_status("pkda_norm_gate_fwd");
  }
  hipLaunchKernelGGL((norm_gate_bwd_kernel<T, D>), dim3(p.blocks), dim3(kNgThreads), 0, s, p);
  if (int st = launch_status("pkda_norm_gate_bwd")) return st;
  const int S = p.blocks < kNgSlices ? p.blocks : kNgSlices;
  hipLaunchKernelGGL((norm_gate_dw_slices_kernel<D>), dim3(S), dim3(D), 0, s, p, S);
  if (int st = launch_status("pkda_norm_gate_bwd(dweight slices)")) return st;
  hipLaunchKernelGGL((norm_gate_dw_kernel<D>), dim3(1), dim3(D), 0, s, p, S);
  return launch_status("pkda_norm_gate_bwd(dweight)");
}

int blocks_for(int64_t rows, int dim) {
  const int64_t rpb = kNgThreads / (dim / 8);
  const int64_t need = (rows + rpb - 1) / rpb;
  return static_cast<int>(need < kNgBlocks ? need : kNgBlocks);
}

int ng_call(const pkda_norm_gate_args* a, void* stream, bool backward) {
  PKDA_REQUIRE(a != nullptr, PKDA_EINVAL, "null args");
  PKDA_REQUIRE(a->struct_size == (int32_t)sizeof(pkda_norm_gate_args), PKDA_EINVAL,
               "pkda_norm_gate_args size mismatch");
  PKDA_REQUIRE(a->dtype == PKDA_F32 || a->dtype == PKDA_BF16, PKDA_EUNSUPPORTED, "dtype %d", a->dtype);
  PKDA_REQUIRE(a->w_dtype == PKDA_F32 || a->w_dtype == PKDA_BF16, PKDA_EUNSUPPORTED, "weight dtype %d", a->w_dtype);
  PKDA_REQUIRE(a->dim == 64 || a->dim == 128, PKDA_EUNSUPPORTED, "dim %d (64, 128)", a->dim);
  PKDA_REQUIRE(a->rows >= 0, PKDA_EINVAL, "rows");
  NgParams p;
  p.x = a->x; p.gate = a->gate; p.weight = a->weight; p.w_dtype = a->w_dtype; p.eps = a->eps;
  p.y = a->y; p.rstd = a->rstd; p.dy = a->dy; p.dx = a->dx; p.dgate = a->dgate;
  p.dw_part = a->dw_part; p.dw = a->dw; p.rows = a->rows;
  p.blocks = blocks_for(a->rows, a->dim);
  if (backward) {
    PKDA_REQUIRE(a->weight && a->dw && (a->rows == 0 || a->dw_part), PKDA_EINVAL, "null tensor");
    if (a->rows == 0) return 0;  // dweight stays the caller's zeros
    PKDA_REQUIRE(a->x && a->gate && a->rstd && a->dy && a->dx && a->dgate, PKDA_EINVAL, "null tensor");
  } else {
    if (a->rows == 0) return 0;
    PKDA_REQUIRE(a->x && a->gate && a->weight && a->y && a->rstd, PKDA_EINVAL, "null tensor");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->dtype == PKDA_BF16) {
    return a->dim == 128 ? launch_ng<bf16_t, 128>(p, backward, s) : launch_ng<bf16_t, 64>(p, backward, s);
  }
  return a->dim == 128 ? launch_ng<float, 128>(p, backward, s) : launch_ng<float, 64>(p, backward, s);
}

}  // namespace
}  // namespace pkda

extern "C" int64_t pkda_norm_gate_workspace(int64_t rows, int32_t dim) {
  if (dim != 64 && dim != 128) return -1;
  return (int64_t)pkda::blocks_for(rows, dim) * dim;
}

extern "C" int pkda_norm_gate_fwd(const pkda_norm_gate_args* args, void* stream) {
  return pkda::ng_call(args, stream, false);
}

extern "C" int pkda_norm_gate_bwd(const pkda_norm_gate_args* args, void* stream) {
  return pkda::ng_call(args, stream, true);
}
