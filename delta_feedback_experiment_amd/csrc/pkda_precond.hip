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
// One workgroup per (document, head), one thread per key channel.  The
// forward checkpoints A at every chunk start; the backward walks the chunks in
// reverse, recomputes the chunk's A_t into LDS, runs the reverse recurrence
// and reduces the per-token channel sums from LDS in a fixed order.
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
  const float* dkw;
  float* dk;
  float* dg_atk;
  float* dbeta_atk;
  float* dcenter_part;
  float* dA0;
  const float* dA_T;
  const int32_t* slot;  // forward: document -> A-state row, or null
};

template <int D> struct PrecondThreads { static constexpr int v = D < 64 ? 64 : D; };

template <typename T, int D>
__global__ __launch_bounds__(PrecondThreads<D>::v) void precond_fwd_kernel(PrecondParams p) {
  const DocSlot ds = doc_slot(p.geom, p.H, 1);
  const int n = ds.n, h = ds.h, c = threadIdx.x;
  if (c >= D) return;
  const int H = p.H;
  int first, count, dstart, dlen;
  doc_chunks(p.geom, n, first, count, dstart, dlen);
  const int64_t sh = (int64_t)(p.slot ? p.slot[n] : n) * H + h;  // state row
  float a = p.a0 ? p.a0[sh * D + c] : 0.f;
  const float center = p.center[h];
  const T* k = static_cast<const T*>(p.k);
  T* kw = static_cast<T*>(p.kw);
  for (int jc = 0; jc < count; ++jc) {
    if (p.a_chunk) p.a_chunk[((int64_t)(first + jc) * H + h) * D + c] = a;
    const int t0 = dstart + jc * C;
    const int len = min(C, dlen - jc * C);
    for (int t = 0; t < len; ++t) {
      const int64_t th = (int64_t)(t0 + t) * H + h;
      const float kc = io<T>::load(k + th * D + c);
      a = expf(p.g_atk[th]) * a + p.beta_atk[th] * (kc * kc);
      const float r = logf(a + p.eps) - center;
      io<T>::store(kw + th * D + c, kc * expf(-p.log_x * (r / (1.f + fabsf(r)))));
    }
  }
  if (p.aT) p.aT[sh * D + c] = a;
}

template <typename T, int D>
__global__ __launch_bounds__(PrecondThreads<D>::v) void precond_bwd_kernel(PrecondParams p) {
  constexpr int NT = PrecondThreads<D>::v;
  constexpr int LDA = D + 1;
  // sA holds A_t of the current chunk; the reverse pass overwrites row t with
  // lambda_t e^{g_atk_t} A_{t-1} once rows t and t-1 have been read.
  extern __shared__ __attribute__((aligned(16))) float smem_f[];
  float* sA = smem_f;              // [C][LDA]
  float* sCb = sA + C * LDA;       // [C][LDA]  lambda_t k_t^2
  float* sRed = sCb + C * LDA;     // [NT]
  const DocSlot ds = doc_slot(p.geom, p.H, 1);
  const int n = ds.n, h = ds.h, c = threadIdx.x;
  const bool active = c < D;
  const int H = p.H;
  int first, count, dstart, dlen;
  doc_chunks(p.geom, n, first, count, dstart, dlen);
  const int64_t sh = (int64_t)n * H + h;
  const float center = p.center[h];
  const T* k = static_cast<const T*>(p.k);
  float lam = (active && p.dA_T) ? p.dA_T[sh * D + c] : 0.f;  // dL/dA after the last token
  float dcen = 0.f;
  for (int jc = count - 1; jc >= 0; --jc) {
    const int t0 = dstart + jc * C;
    const int len = min(C, dlen - jc * C);
    const float a_in = active ? p.a_chunk[((int64_t)(first + jc) * H + h) * D + c] : 0.f;
    if (active) {
      float a = a_in;
      for (int t = 0; t < len; ++t) {
        const int64_t th = (int64_t)(t0 + t) * H + h;
        const float kc = io<T>::load(k + th * D + c);
        a = expf(p.g_atk[th]) * a + p.beta_atk[th] * (kc * kc);
        sA[t * LDA + c] = a;
      }
      for (int t = len - 1; t >= 0; --t) {
        const int64_t th = (int64_t)(t0 + t) * H + h;
        const float kc = io<T>::load(k + th * D + c);
        const float a = sA[t * LDA + c];
        const float a_prev = t > 0 ? sA[(t - 1) * LDA + c] : a_in;
        const float r = logf(a + p.eps) - center;
        const float den = 1.f + fabsf(r);
        const float f = expf(-p.log_x * (r / den));
        const float dkw = p.dkw[th * D + c];
        const float dr = dkw * kc * f * (-p.log_x) / (den * den);
        dcen -= dr;
        lam += dr / (a + p.eps);
        const float ba = p.beta_atk[th];
        p.dk[th * D + c] += dkw * f + 2.f * ba * kc * lam;
        const float eg = expf(p.g_atk[th]);
        sA[t * LDA + c] = lam * eg * a_prev;
        sCb[t * LDA + c] = lam * kc * kc;
        lam *= eg;  // carry to A_{t-1}
      }
    }
    __syncthreads();
    // per-token channel sums, fixed order
    for (int t = threadIdx.x; t < len; t += NT) {
      float sg = 0.f, sb = 0.f;
      for (int j = 0; j < D; ++j) {
        sg += sA[t * LDA + j];
        sb += sCb[t * LDA + j];
      }
      const int64_t th = (int64_t)(t0 + t) * H + h;
      p.dg_atk[th] = sg;
      p.dbeta_atk[th] = sb;
    }
    __syncthreads();
  }
  if (active && p.dA0) p.dA0[sh * D + c] = lam;
  sRed[threadIdx.x] = active ? dcen : 0.f;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.f;
    for (int j = 0; j < NT; ++j) s += sRed[j];
    p.dcenter_part[sh] = s;
  }
}

// dcenter[h] = sum_n part[n, h], fixed order.
__global__ void precond_dcenter_kernel(const float* part, int N, int H, float* out) {
  const int h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h >= H) return;
  float s = 0.f;
  for (int n = 0; n < N; ++n) s += part[(int64_t)n * H + h];
  out[h] = s;
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
  PKDA_REQUIRE(!a->slot_idx || a->pool_size > 0, PKDA_EINVAL, "slot-indexed A states need pool_size > 0");
  return 0;
}

template <typename T, int D>
int launch_precond(const PrecondParams& p, bool backward, hipStream_t s) {
  constexpr int NT = PrecondThreads<D>::v;
  const dim3 grid = doc_grid(p.geom.num_seqs, p.H, 1);
  if (backward) {
    const int bytes = (2 * C * (D + 1) + NT) * (int)sizeof(float);
    auto kern = precond_bwd_kernel<T, D>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) {
      set_error("hipFuncSetAttribute(%d bytes): %s", bytes, hipGetErrorString(e));
      return static_cast<int>(e);
    }
    hipLaunchKernelGGL(kern, grid, dim3(NT), bytes, s, p);
  } else {
    hipLaunchKernelGGL((precond_fwd_kernel<T, D>), grid, dim3(NT), 0, s, p);
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
  PKDA_REQUIRE(a->kw, PKDA_EINVAL, "preconditioner forward needs kw");
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
    PKDA_REQUIRE(a->a_chunk && a->dkw && a->dk && a->dg_atk && a->dbeta_atk, PKDA_EINVAL,
                 "preconditioner backward needs a_chunk, dkw, dk, dg_atk and dbeta_atk");
    const int st = a->dtype == PKDA_F32 ? dispatch_precond<float>(p, a->head_dim, true, s)
                                        : dispatch_precond<bf16_t>(p, a->head_dim, true, s);
    if (st) return st;
  }
  hipLaunchKernelGGL(precond_dcenter_kernel, dim3((a->heads + 63) / 64), dim3(64), 0, s, a->dcenter_part,
                     a->num_seqs, a->heads, a->dcenter);
  return launch_status("pkda_precond_bwd(dcenter)");
}
