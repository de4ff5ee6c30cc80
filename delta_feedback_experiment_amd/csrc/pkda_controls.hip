// PKDA control activations (forward) and the packed control gradient
// (backward) for gfx950.
//
// Reference: PreconditionedKDA._controls (delta_feedback_experiment/pkda.py:
// 318-353) splits one projection per token into
//   decay hidden [rank] | beta logits [H] | precond decay logits [H] |
//   precond beta logits [H] | output-gate hidden [gate_width]
// and activates the middle three:
//   beta          = sigmoid(logit)                                  (dtype)
//   precond_decay = -exp(A_log_p[h]) softplus(logit + dt_bias_p[h]) (FP32)
//   precond_beta  = sigmoid(logit)                                  (dtype)
// Its backward (_PackedControlSplit + pack_control_gradients,
// pkda.py:56-74, cuda_kernels.py:1081-1172) assembles the five gradients into
// one packed buffer; here the activation derivatives are applied in the same
// pass, so the packed gradient is written once:
//   d logit_beta  = dbeta y (1 - y),  y = sigmoid rounded to dtype
//   d logit_decay = dprecond_decay (-exp(A_log_p)) sigmoid(z),  z = logit + dt_bias_p
//   dA_log_p[h]   = sum_t dprecond_decay precond_decay,  ddt_bias_p[h] = sum_t d logit_decay
// The two parameter gradients are per-block partials (each head's terms summed
// over the block's rows in order) summed over blocks in a fixed order.
#include "pkda_chunk_common.h"

namespace pkda {
namespace {

constexpr int kCtlThreads = 256;
constexpr int kCtlRows = 16;  // rows per workgroup

struct CtlParams {
  int64_t rows;
  int H, rank, gw, stride, width;
  const void* packed;
  const float* A_log_p;
  const float* dt_bias_p;
  void* beta;
  float* pdecay;
  void* pbeta;
  const void* d_hidden;
  const void* dbeta;
  const float* dpdecay;
  const void* dpbeta;
  const void* d_gate;
  void* dpacked;
  float* part;
};

// x as the dtype stores it (a bf16 round trip; identity for FP32).
template <typename T> __device__ __forceinline__ float rounded(float x);
template <> __device__ __forceinline__ float rounded<float>(float x) { return x; }
template <> __device__ __forceinline__ float rounded<bf16_t>(float x) { return bf16_to_f32(f32_to_bf16(x)); }

template <typename T>
__global__ __launch_bounds__(kCtlThreads) void controls_fwd_kernel(CtlParams p) {
  const int64_t r0 = (int64_t)blockIdx.x * kCtlRows;
  const int nr = (int)min<int64_t>(kCtlRows, p.rows - r0);
  const int H = p.H;
  const T* packed = static_cast<const T*>(p.packed);
  for (int i = threadIdx.x; i < nr * 3 * H; i += kCtlThreads) {
    const int r = i / (3 * H), j = i - r * 3 * H;
    const int which = j / H, h = j - which * H;
    const int64_t row = r0 + r;
    const float x = io<T>::load(packed + row * p.stride + p.rank + j);
    if (which == 1) {
      p.pdecay[row * H + h] = -expf(p.A_log_p[h]) * softplus_sigmoid_fast(x + p.dt_bias_p[h]).softplus;
    } else {
      io<T>::store(static_cast<T*>(which == 0 ? p.beta : p.pbeta) + row * H + h, softplus_sigmoid_fast(x).sigmoid);
    }
  }
}

template <typename T>
__device__ __forceinline__ float load_or_zero(const void* base, int64_t i) {
  return base ? io<T>::load(static_cast<const T*>(base) + i) : 0.f;
}

template <typename T>
__global__ __launch_bounds__(kCtlThreads) void controls_bwd_kernel(CtlParams p) {
  const int64_t r0 = (int64_t)blockIdx.x * kCtlRows;
  const int nr = (int)min<int64_t>(kCtlRows, p.rows - r0);
  const int H = p.H, rank = p.rank, W = p.width;
  const T* packed = static_cast<const T*>(p.packed);
  T* dpacked = static_cast<T*>(p.dpacked);
  // every column but the preconditioner decay's, one element per thread
  for (int i = threadIdx.x; i < nr * W; i += kCtlThreads) {
    const int r = i / W, c = i - r * W;
    const int64_t row = r0 + r;
    float d;
    if (c < rank) {
      d = load_or_zero<T>(p.d_hidden, row * rank + c);
    } else if (c < rank + H || (c >= rank + 2 * H && c < rank + 3 * H)) {
      const bool is_beta = c < rank + H;
      const int h = c - rank - (is_beta ? 0 : 2 * H);
      const float y = rounded<T>(softplus_sigmoid_fast(io<T>::load(packed + row * p.stride + c)).sigmoid);
      d = load_or_zero<T>(is_beta ? p.dbeta : p.dpbeta, row * H + h) * (y * (1.f - y));
    } else if (c < rank + 2 * H) {
      continue;  // preconditioner decay: below
    } else {
      d = load_or_zero<T>(p.d_gate, row * p.gw + (c - rank - 3 * H));
    }
    io<T>::store(dpacked + row * W + c, d);
  }
  // preconditioner decay columns: one (row, head) per thread, the two
  // parameter terms through LDS, then summed over the rows in order per head
  extern __shared__ float s_terms[];  // [2][kCtlRows][H]
  for (int i = threadIdx.x; i < nr * H; i += kCtlThreads) {
    const int r = i / H, h = i - r * H;
    const int64_t row = r0 + r;
    const float A = expf(p.A_log_p[h]);
    const float z = io<T>::load(packed + row * p.stride + rank + H + h) + p.dt_bias_p[h];
    const float gd = p.dpdecay ? p.dpdecay[row * H + h] : 0.f;
    const SoftplusSigmoid f = softplus_sigmoid_fast(z);
    const float dz = gd * (-A) * f.sigmoid;
    io<T>::store(dpacked + row * W + rank + H + h, dz);
    s_terms[r * H + h] = gd * (-A * f.softplus);
    s_terms[(kCtlRows + r) * H + h] = dz;
  }
  __syncthreads();
  if (threadIdx.x < 2 * H) {
    const int which = threadIdx.x / H, h = threadIdx.x - which * H;
    float acc = 0.f;
    for (int r = 0; r < nr; ++r) acc += s_terms[(which * kCtlRows + r) * H + h];
    p.part[(int64_t)blockIdx.x * 2 * H + threadIdx.x] = acc;
  }
}


int controls_common(const pkda_controls_args* a, CtlParams& p) {
  PKDA_REQUIRE(a != nullptr, PKDA_EINVAL, "null args");
  PKDA_REQUIRE(a->struct_size == (int32_t)sizeof(pkda_controls_args), PKDA_EINVAL, "pkda_controls_args size mismatch");
  PKDA_REQUIRE(a->dtype == PKDA_F32 || a->dtype == PKDA_BF16, PKDA_EUNSUPPORTED, "dtype %d", a->dtype);
  PKDA_REQUIRE(a->rows >= 0 && a->heads > 0 && a->rank >= 0 && a->gate_width >= 0, PKDA_EINVAL, "sizes");
  const int width = a->rank + 3 * a->heads + a->gate_width;
  PKDA_REQUIRE(a->row_stride >= width, PKDA_EINVAL, "row_stride %d < width %d", a->row_stride, width);
  PKDA_REQUIRE(2 * a->heads <= kCtlThreads, PKDA_EUNSUPPORTED, "heads %d (at most %d)", a->heads, kCtlThreads / 2);
  PKDA_REQUIRE(a->rows == 0 || (a->packed && a->A_log_p && a->dt_bias_p), PKDA_EINVAL, "null tensor");
  p.rows = a->rows;
  p.H = a->heads;
  p.rank = a->rank;
  p.gw = a->gate_width;
  p.stride = a->row_stride;
  p.width = width;
  p.packed = a->packed;
  p.A_log_p = a->A_log_p;
  p.dt_bias_p = a->dt_bias_p;
  p.beta = a->beta;
  p.pdecay = a->precond_decay;
  p.pbeta = a->precond_beta;
  p.d_hidden = a->d_decay_hidden;
  p.dbeta = a->dbeta;
  p.dpdecay = a->dprecond_decay;
  p.dpbeta = a->dprecond_beta;
  p.d_gate = a->d_gate_hidden;
  p.dpacked = a->dpacked;
  p.part = a->part;
  return 0;
}

int64_t controls_blocks(int64_t rows) { return (rows + kCtlRows - 1) / kCtlRows; }

}  // namespace
}  // namespace pkda

using namespace pkda;

extern "C" int64_t pkda_controls_workspace(int64_t rows, int32_t heads) {
  return controls_blocks(rows) * 2 * (int64_t)heads;
}

extern "C" int pkda_controls_fwd(const pkda_controls_args* a, void* stream) {
  CtlParams p;
  if (int st = controls_common(a, p)) return st;
  if (p.rows == 0) return 0;
  PKDA_REQUIRE(a->beta && a->precond_decay && a->precond_beta, PKDA_EINVAL, "controls forward needs its outputs");
  const dim3 grid((unsigned)controls_blocks(p.rows));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->dtype == PKDA_BF16) {
    hipLaunchKernelGGL(controls_fwd_kernel<bf16_t>, grid, dim3(kCtlThreads), 0, s, p);
  } else {
    hipLaunchKernelGGL(controls_fwd_kernel<float>, grid, dim3(kCtlThreads), 0, s, p);
  }
  return launch_status("pkda_controls_fwd");
}

extern "C" int pkda_controls_bwd(const pkda_controls_args* a, void* stream) {
  CtlParams p;
  if (int st = controls_common(a, p)) return st;
  PKDA_REQUIRE(a->dA_log_p && a->ddt_bias_p, PKDA_EINVAL, "controls backward needs dA_log_p and ddt_bias_p");
  PKDA_REQUIRE(p.rows == 0 || (a->dpacked && a->part), PKDA_EINVAL, "controls backward needs dpacked and part");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int blocks = (int)controls_blocks(p.rows);
  if (blocks > 0) {
    const int bytes = 2 * kCtlRows * p.H * (int)sizeof(float);
    if (a->dtype == PKDA_BF16) {
      hipLaunchKernelGGL(controls_bwd_kernel<bf16_t>, dim3(blocks), dim3(kCtlThreads), bytes, s, p);
    } else {
      hipLaunchKernelGGL(controls_bwd_kernel<float>, dim3(blocks), dim3(kCtlThreads), bytes, s, p);
    }
    if (int st = launch_status("pkda_controls_bwd")) return st;
  }
  // part rows are [dA terms of H heads | ddt terms of H heads]
  hipLaunchKernelGGL(sum_partials_tree_kernel, dim3(p.H), dim3(256), 0, s, a->part, blocks, 2 * p.H, a->dA_log_p);
  hipLaunchKernelGGL(sum_partials_tree_kernel, dim3(p.H), dim3(256), 0, s, a->part + p.H, blocks, 2 * p.H,
                     a->ddt_bias_p);
  return launch_status("pkda_controls_bwd(reduce)");
}
