// Token-recurrent PKDA forward and the slot-pool decode step (gfx950).
// (recurrent_kernel: any sequence length; decode_kernel: the persistent
// one-token step over a slot pool.)
//
// One 256-thread workgroup owns one (sequence, head).  The FP32 state
// S [D x D] lives in registers for the whole sequence: thread (rg, cg) holds
// columns 4cg..4cg+3 of rows rg, rg+NRG, rg+2NRG, ...  Every token costs two
// column reductions of the *old* state, since
//
//   e_v = v_v - sum_k (alpha_k k_k) S[k,v]
//   o_v = sum_k (alpha_k qs_k) S[k,v] + beta e_v (qs . kw)
//
// (o reads the updated state, pkda.py:406; expanding S_t gives the second
// line), followed by the in-register rank-1 update
// S[k,v] <- alpha_k S[k,v] + beta kw_k e_v.  The state is read from HBM once
// and written once per sequence, which is what makes the decode step
// bandwidth-bound on the 64 KiB-per-head FP32 state.
#include "pkda_common.h"

namespace pkda {
namespace {

constexpr int kThreads = 256;

struct RecParams {
  int num_seqs, seqlen, heads;
  const int32_t* cu_seqlens;
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  int gate_kind, g_dtype;
  const float* A_log;
  const float* dt_bias;
  const float* beta;
  float scale;
  const float* g_atk;
  const float* beta_atk;
  const float* center;
  float log_x, squash_eps;
  float* state_pool;
  float* a_pool;
  const int32_t* slot_idx;
  const float* initial_state;
  const float* initial_A_state;
  float* final_state;
  float* final_A_state;
  void* o;
};

template <typename T, int D>
__global__ __launch_bounds__(kThreads) void recurrent_kernel(RecParams p) {
  constexpr int NCG = D / 4;            // column groups of 4
  constexpr int NRG = kThreads / NCG;   // row groups
  constexpr int RPT = D / NRG;          // rows per thread
  static_assert(RPT >= 1 && NRG * RPT == D, "bad head dim");

  __shared__ float s_ak[2][D];   // alpha_k * k_k            (prediction read)
  __shared__ float s_aq[2][D];   // alpha_k * scale * q_k    (output read)
  __shared__ float s_al[2][D];   // alpha_k
  __shared__ float s_bw[2][D];   // beta * kw_k               (write)
  __shared__ float s_v[2][D];
  __shared__ float s_qk[2][kThreads / 64];
  __shared__ float4 s_pe[NRG][NCG];
  __shared__ float4 s_po[NRG][NCG];

  const int n = blockIdx.x;
  const int h = blockIdx.y;
  const int H = p.heads;
  const int tid = threadIdx.x;
  const int cg = tid % NCG;
  const int rg = tid / NCG;
  const SeqBounds sb = seq_bounds(p.cu_seqlens, n, p.seqlen);

  // ---- state source --------------------------------------------------------
  const float* s_src = nullptr;
  float* s_dst = nullptr;
  const float* a_src = nullptr;
  float* a_dst = nullptr;
  if (p.state_pool) {
    const int64_t slot = p.slot_idx ? p.slot_idx[n] : n;
    s_src = s_dst = p.state_pool + (slot * H + h) * (int64_t)D * D;
    if (p.a_pool) a_src = a_dst = p.a_pool + (slot * H + h) * (int64_t)D;
  } else {
    if (p.initial_state) s_src = p.initial_state + ((int64_t)n * H + h) * D * D;
    if (p.final_state) s_dst = p.final_state + ((int64_t)n * H + h) * D * D;
    if (p.initial_A_state) a_src = p.initial_A_state + ((int64_t)n * H + h) * D;
    if (p.final_A_state) a_dst = p.final_A_state + ((int64_t)n * H + h) * D;
  }

  float4 S[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int row = rg + NRG * j;
    S[j] = s_src ? load4(s_src + row * D + 4 * cg) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const bool precond = p.g_atk != nullptr;
  float a_c = 0.f;  // preconditioner state of channel tid (tid < D)
  if (precond && tid < D && a_src) a_c = a_src[tid];

  const float A_scale = (p.gate_kind == PKDA_GATE_RAW_CHANNEL) ? -expf(p.A_log[h]) : 0.f;
  const float center = precond ? p.center[h] : 0.f;

  for (int t = 0; t < sb.len; ++t) {
    const int buf = t & 1;
    const int64_t tok = sb.start + t;
    const int64_t th = tok * H + h;
    // ---- channel phase: gate, preconditioner, operands to LDS -------------
    float qk_part = 0.f;
    if (tid < D) {
      const int c = tid;
      const float qc = io<T>::load(static_cast<const T*>(p.q) + th * D + c) * p.scale;
      const float kc = io<T>::load(static_cast<const T*>(p.k) + th * D + c);
      const float vc = io<T>::load(static_cast<const T*>(p.v) + th * D + c);
      float gl;
      if (p.gate_kind == PKDA_GATE_LOG_HEAD) {
        gl = load_any(p.g, th, p.g_dtype);
      } else if (p.gate_kind == PKDA_GATE_LOG_CHANNEL) {
        gl = load_any(p.g, th * D + c, p.g_dtype);
      } else {
        gl = A_scale * softplus_sigmoid_fast(load_any(p.g, th * D + c, p.g_dtype) + p.dt_bias[h * D + c]).softplus;
      }
      const float al = expf(gl);
      float kw = kc;
      if (precond) {
        a_c = expf(p.g_atk[th]) * a_c + p.beta_atk[th] * (kc * kc);
        const float r = logf(a_c + p.squash_eps) - center;
        kw = kc * expf(-p.log_x * (r / (1.f + fabsf(r))));
      }
      const float bt = p.beta[th];
      s_ak[buf][c] = al * kc;
      s_aq[buf][c] = al * qc;
      s_al[buf][c] = al;
      s_bw[buf][c] = bt * kw;
      s_v[buf][c] = vc;
      qk_part = qc * kw * bt;
    }
    // wave reduction of beta * (qs . kw)
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) qk_part += __shfl_xor(qk_part, off);
    if ((tid & 63) == 0) s_qk[buf][tid >> 6] = qk_part;
    __syncthreads();

    // ---- reduction phase: partial column sums of the old state -------------
    float4 pe = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 po = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int row = rg + NRG * j;
      const float ak = s_ak[buf][row];
      const float aq = s_aq[buf][row];
      pe.x += ak * S[j].x; pe.y += ak * S[j].y; pe.z += ak * S[j].z; pe.w += ak * S[j].w;
      po.x += aq * S[j].x; po.y += aq * S[j].y; po.z += aq * S[j].z; po.w += aq * S[j].w;
    }
    s_pe[rg][cg] = pe;
    s_po[rg][cg] = po;
    __syncthreads();

    // ---- finish: residual, output, rank-1 update ----------------------------
    float4 e = *reinterpret_cast<const float4*>(&s_v[buf][4 * cg]);
    float4 out = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < NRG; ++r) {
      const float4 a = s_pe[r][cg];
      const float4 b = s_po[r][cg];
      e.x -= a.x; e.y -= a.y; e.z -= a.z; e.w -= a.w;
      out.x += b.x; out.y += b.y; out.z += b.z; out.w += b.w;
    }
    float bqk = 0.f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) bqk += s_qk[buf][w];
    out.x += bqk * e.x; out.y += bqk * e.y; out.z += bqk * e.z; out.w += bqk * e.w;
    if (rg == 0) store4(static_cast<T*>(p.o) + th * D + 4 * cg, out);
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int row = rg + NRG * j;
      const float al = s_al[buf][row];
      const float bw = s_bw[buf][row];
      S[j].x = al * S[j].x + bw * e.x;
      S[j].y = al * S[j].y + bw * e.y;
      S[j].z = al * S[j].z + bw * e.z;
      S[j].w = al * S[j].w + bw * e.w;
    }
  }

  if (s_dst) {
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int row = rg + NRG * j;
      store4(s_dst + row * D + 4 * cg, S[j]);
    }
  }
  if (precond && tid < D && a_dst) a_dst[tid] = a_c;
}

// ---------------------------------------------------------------------------
// Slot-pool decode step (one token per live sequence), persistent and
// software-pipelined.  Each workgroup walks (sequence, head) items
// blockIdx.x, blockIdx.x + gridDim.x, ...; while it reduces and writes back
// one item's state it already has the next item's 64 KiB (d = 128) in flight,
// so the state stream never waits on the read-compute-write chain of a single
// item.  The state is touched once per step: loaded and stored with
// non-temporal hints (no reuse, so it is kept out of the caches' way).
// Same arithmetic as recurrent_kernel at T = 1.
// ---------------------------------------------------------------------------
typedef float f4v __attribute__((ext_vector_type(4)));

// A read, through the scalar unit (s_load), of an input the kernel never
// writes, at an address the same for the whole workgroup: its wait counts
// apart from the vector memory operations in flight.
template <typename U>
__device__ __forceinline__ U scalar_load(const U* ptr) {
  return *(const __attribute__((address_space(4))) U*)ptr;
}

template <typename T, int D, int NTH>
__global__ __launch_bounds__(NTH) void decode_kernel(RecParams p) {
  constexpr int NCG = D / 4;
  constexpr int NRG = NTH / NCG;
  constexpr int RPT = D / NRG;
  static_assert(RPT >= 1 && NRG * RPT == D, "bad head dim");
  __shared__ float s_ak[D], s_aq[D], s_al[D], s_bw[D], s_v[D];
  __shared__ float s_qk[NTH / 64];
  __shared__ float4 s_pe[NRG][NCG];
  __shared__ float4 s_po[NRG][NCG];

  const int H = p.heads;
  const int tid = threadIdx.x;
  const int cg = tid % NCG;
  const int rg = tid / NCG;
  const int total = p.num_seqs * H;
  const bool precond = p.g_atk != nullptr;
  // Every input of an item is requested one item ahead, and an iteration
  // runs the current item's channel phase before it sends the next item's
  // requests: a wait on the vector memory counter (which counts in order)
  // then never waits for the next item's 64 KiB, which stays in flight
  // through the current item's reductions and write-back.  The per-channel
  // inputs (q, k, v, g as raw bits, widened where they are used; dt_bias, A)
  // come through vector loads behind the state's, the item's uniform values
  // (its slot, beta, the preconditioner's decay and strength, A_log and
  // center of its head) through scalar loads, which count apart.
  struct ItemIn {
    int64_t slot;
    float beta, g_atk, beta_atk, A_log, center;
  };
  struct ChanIn {
    uint32_t q, k, v, g;  // T's (and g's) bits
    float dtb, a;
  };
  auto widen = [&](uint32_t bits, bool narrow) { return __uint_as_float(narrow ? bits << 16 : bits); };
  constexpr bool TN = sizeof(T) == 2;
  auto load_item = [&](int it, ItemIn& x) {
    const int n = it / H, h = it - n * H;
    const int64_t th = (int64_t)n * H + h;
    x.slot = p.slot_idx ? scalar_load(p.slot_idx + n) : n;
    x.beta = scalar_load(p.beta + th);
    x.A_log = p.gate_kind == PKDA_GATE_RAW_CHANNEL ? scalar_load(p.A_log + h) : 0.f;
    if (precond) {
      x.g_atk = scalar_load(p.g_atk + th);
      x.beta_atk = scalar_load(p.beta_atk + th);
      x.center = scalar_load(p.center + h);
    }
  };
  // (every lane loads -- the lanes past D a copy of channel D - 1, unused --
  // so the loaded registers join no divergent branch and wait for nothing)
  auto load_chan = [&](int it, const ItemIn& xi, ChanIn& x) {
    const int n = it / H, h = it - n * H;
    const int64_t th = (int64_t)n * H + h;
    const int c = min(tid, D - 1);
    using R = std::conditional_t<TN, uint16_t, uint32_t>;
    x.q = reinterpret_cast<const R*>(p.q)[th * D + c];
    x.k = reinterpret_cast<const R*>(p.k)[th * D + c];
    x.v = reinterpret_cast<const R*>(p.v)[th * D + c];
    const int64_t gi = p.gate_kind == PKDA_GATE_LOG_HEAD ? th : th * D + c;
    if (p.g_dtype == PKDA_BF16) x.g = static_cast<const uint16_t*>(p.g)[gi];
    else x.g = static_cast<const uint32_t*>(p.g)[gi];
    if (p.gate_kind == PKDA_GATE_RAW_CHANNEL) x.dtb = p.dt_bias[h * D + c];
    if (precond) x.a = p.a_pool[(xi.slot * H + h) * (int64_t)D + c];
  };
  auto state_of = [&](int it, int64_t slot) {
    const int h = it - (it / H) * H;
    return p.state_pool + (slot * H + h) * (int64_t)D * D;
  };
  f4v S[RPT], Sn[RPT];
  ItemIn ci{}, ni{};
  ChanIn cur{}, nxt_in{};
  int item = blockIdx.x;
  if (item < total) {
    load_item(item, ci);
    const float* src = state_of(item, ci.slot);
#pragma unroll
    for (int j = 0; j < RPT; ++j)
      S[j] = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(src + (rg + NRG * j) * D + 4 * cg));
    load_chan(item, ci, cur);
  }
  for (; item < total; item += gridDim.x) {
    const int nxt = item + gridDim.x;
    const int n = item / H, h = item - n * H;
    const int64_t slot = ci.slot;
    const int64_t th = (int64_t)n * H + h;
    // ---- channel phase ------------------------------------------------------
    float qk_part = 0.f;
    if (tid < D) {
      const int c = tid;
      const float qc = widen(cur.q, TN) * p.scale;
      const float kc = widen(cur.k, TN);
      const float vc = widen(cur.v, TN);
      float gl = widen(cur.g, p.g_dtype == PKDA_BF16);
      if (p.gate_kind == PKDA_GATE_RAW_CHANNEL) gl = -expf(ci.A_log) * softplus_sigmoid_fast(gl + cur.dtb).softplus;
      const float al = expf(gl);
      float kw = kc;
      if (precond) {
        const float a_c = expf(ci.g_atk) * cur.a + ci.beta_atk * (kc * kc);
        p.a_pool[(slot * H + h) * (int64_t)D + c] = a_c;
        const float r = logf(a_c + p.squash_eps) - ci.center;
        kw = kc * expf(-p.log_x * (r / (1.f + fabsf(r))));
      }
      const float bt = ci.beta;
      s_ak[c] = al * kc;
      s_aq[c] = al * qc;
      s_al[c] = al;
      s_bw[c] = bt * kw;
      s_v[c] = vc;
      qk_part = qc * kw * bt;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) qk_part += __shfl_xor(qk_part, off);
    if ((tid & 63) == 0) s_qk[tid >> 6] = qk_part;
    // ---- the next item's requests -------------------------------------------
    // (its few per-channel bytes unconditionally, for this item again when
    // there is no next one: loads behind no branch join nothing)
    const int nl = nxt < total ? nxt : item;
    load_item(nl, ni);
    if (nxt < total) {
      const float* src = state_of(nxt, ni.slot);
#pragma unroll
      for (int j = 0; j < RPT; ++j)
        Sn[j] = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(src + (rg + NRG * j) * D + 4 * cg));
    }
    load_chan(nl, ni, nxt_in);
    __syncthreads();
    // ---- column reductions of the old state ---------------------------------
    float4 pe = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 po = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int row = rg + NRG * j;
      const float ak = s_ak[row], aq = s_aq[row];
      pe.x += ak * S[j][0]; pe.y += ak * S[j][1]; pe.z += ak * S[j][2]; pe.w += ak * S[j][3];
      po.x += aq * S[j][0]; po.y += aq * S[j][1]; po.z += aq * S[j][2]; po.w += aq * S[j][3];
    }
    s_pe[rg][cg] = pe;
    s_po[rg][cg] = po;
    __syncthreads();
    // ---- residual, output, rank-1 update, write-back -------------------------
    float4 e = *reinterpret_cast<const float4*>(&s_v[4 * cg]);
    float4 out = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < NRG; ++r) {
      const float4 a = s_pe[r][cg];
      const float4 b = s_po[r][cg];
      e.x -= a.x; e.y -= a.y; e.z -= a.z; e.w -= a.w;
      out.x += b.x; out.y += b.y; out.z += b.z; out.w += b.w;
    }
    float bqk = 0.f;
#pragma unroll
    for (int w = 0; w < NTH / 64; ++w) bqk += s_qk[w];
    out.x += bqk * e.x; out.y += bqk * e.y; out.z += bqk * e.z; out.w += bqk * e.w;
    if (rg == 0) store4(static_cast<T*>(p.o) + th * D + 4 * cg, out);
    float* dst = p.state_pool + (slot * H + h) * (int64_t)D * D;
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int row = rg + NRG * j;
      const float al = s_al[row], bw = s_bw[row];
      const f4v x = {al * S[j][0] + bw * e.x, al * S[j][1] + bw * e.y, al * S[j][2] + bw * e.z,
                     al * S[j][3] + bw * e.w};
      __builtin_nontemporal_store(x, reinterpret_cast<f4v*>(dst + row * D + 4 * cg));
    }
    __syncthreads();  // LDS is reused by the next item
#pragma unroll
    for (int j = 0; j < RPT; ++j) S[j] = Sn[j];
    ci = ni;
    cur = nxt_in;
  }
}

template <typename T>
int launch_decode(const RecParams& rp, int D, hipStream_t stream) {
  const int total = rp.num_seqs * rp.heads;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const int grid = total < 12 * cus ? total : 12 * cus;  // ~12 items in flight per CU measured best at d = 128
  switch (D) {
    case 32: hipLaunchKernelGGL((decode_kernel<T, 32, 256>), dim3(grid), dim3(256), 0, stream, rp); break;
    case 64: hipLaunchKernelGGL((decode_kernel<T, 64, 512>), dim3(grid), dim3(512), 0, stream, rp); break;
    case 128: hipLaunchKernelGGL((decode_kernel<T, 128, 512>), dim3(grid), dim3(512), 0, stream, rp); break;
    default: set_error("head_dim %d not built (32, 64, 128)", D); return PKDA_EUNSUPPORTED;
  }
  return launch_status("pkda_decode_step");
}

template <typename T>
int launch_recurrent(const RecParams& rp, int D, hipStream_t stream) {
  dim3 grid(rp.num_seqs, rp.heads);
  switch (D) {
    case 32: hipLaunchKernelGGL((recurrent_kernel<T, 32>), grid, dim3(kThreads), 0, stream, rp); break;
    case 64: hipLaunchKernelGGL((recurrent_kernel<T, 64>), grid, dim3(kThreads), 0, stream, rp); break;
    case 128: hipLaunchKernelGGL((recurrent_kernel<T, 128>), grid, dim3(kThreads), 0, stream, rp); break;
    default: set_error("head_dim %d not built (32, 64, 128)", D); return PKDA_EUNSUPPORTED;
  }
  return launch_status("pkda_recurrent");
}

int recurrent_entry(const pkda_recurrent_args* a, void* stream, bool decode) {
  PKDA_REQUIRE(a != nullptr, PKDA_EINVAL, "null args");
  PKDA_REQUIRE(a->struct_size == (int32_t)sizeof(pkda_recurrent_args), PKDA_EINVAL,
               "pkda_recurrent_args size %d, library expects %d", a->struct_size, (int)sizeof(pkda_recurrent_args));
  PKDA_REQUIRE(a->dtype == PKDA_F32 || a->dtype == PKDA_BF16, PKDA_EUNSUPPORTED, "dtype %d", a->dtype);
  PKDA_REQUIRE(a->g_dtype == PKDA_F32 || a->g_dtype == PKDA_BF16, PKDA_EUNSUPPORTED, "g dtype %d", a->g_dtype);
  PKDA_REQUIRE(a->num_seqs >= 0 && a->heads > 0 && a->seqlen >= 0, PKDA_EINVAL, "bad sizes");
  PKDA_REQUIRE(a->head_dim == 32 || a->head_dim == 64 || a->head_dim == 128, PKDA_EUNSUPPORTED,
               "head_dim %d not built (32, 64, 128)", a->head_dim);
  PKDA_REQUIRE(a->gate_kind >= PKDA_GATE_LOG_HEAD && a->gate_kind <= PKDA_GATE_RAW_CHANNEL, PKDA_EINVAL,
               "gate_kind %d", a->gate_kind);
  PKDA_REQUIRE(a->gate_kind != PKDA_GATE_RAW_CHANNEL || (a->A_log && a->dt_bias), PKDA_EINVAL,
               "raw gate needs A_log and dt_bias");
  PKDA_REQUIRE(!a->g_atk || (a->beta_atk && a->center), PKDA_EINVAL, "preconditioner needs beta_atk and center");
  PKDA_REQUIRE(!a->g_atk || a->squash_x > 0.f, PKDA_EINVAL, "squash_x must be positive");
  PKDA_REQUIRE(!a->cu_seqlens || !decode, PKDA_EINVAL, "decode takes no cu_seqlens");
  if (decode) {
    PKDA_REQUIRE(a->seqlen == 1, PKDA_EINVAL, "decode step needs seqlen == 1");
    PKDA_REQUIRE(a->state_pool != nullptr, PKDA_EINVAL, "decode step needs a state pool");
  }
  if (a->state_pool) {
    PKDA_REQUIRE(a->pool_size >= 0, PKDA_EINVAL, "pool_size");
    PKDA_REQUIRE(a->slot_idx || a->num_seqs <= a->pool_size, PKDA_ERANGE, "identity slots exceed the pool");
    PKDA_REQUIRE(!a->g_atk || a->a_pool, PKDA_EINVAL, "preconditioned pool step needs a_pool");
    if (a->check_slots && a->slot_idx_host && a->num_seqs > 0) {
      // Range and uniqueness: duplicate slots would race on the in-place write.
      const int64_t P = a->pool_size;
      if (P <= (int64_t)1 << 26) {
        uint8_t* seen = static_cast<uint8_t*>(calloc((size_t)P + 1, 1));
        PKDA_REQUIRE(seen != nullptr, PKDA_EINVAL, "out of host memory");
        for (int i = 0; i < a->num_seqs; ++i) {
          const int32_t s = a->slot_idx_host[i];
          if (s < 0 || s >= P || seen[s]) {
            free(seen);
            set_error("slot_idx[%d] = %d is out of range [0, %lld) or repeated", i, s, (long long)P);
            return PKDA_ERANGE;
          }
          seen[s] = 1;
        }
        free(seen);
      }
    }
  }
  if (a->num_seqs == 0) return PKDA_OK;
  PKDA_REQUIRE(a->q && a->k && a->v && a->g && a->beta && a->o, PKDA_EINVAL, "null token tensor");

  RecParams rp;
  rp.num_seqs = a->num_seqs;
  rp.seqlen = a->seqlen;
  rp.heads = a->heads;
  rp.cu_seqlens = a->cu_seqlens;
  rp.q = a->q; rp.k = a->k; rp.v = a->v; rp.g = a->g;
  rp.gate_kind = a->gate_kind; rp.g_dtype = a->g_dtype;
  rp.A_log = a->A_log; rp.dt_bias = a->dt_bias;
  rp.beta = a->beta; rp.scale = a->scale;
  rp.g_atk = a->g_atk; rp.beta_atk = a->beta_atk; rp.center = a->center;
  rp.log_x = a->g_atk ? logf(a->squash_x) : 0.f;
  rp.squash_eps = a->squash_eps;
  rp.state_pool = a->state_pool; rp.a_pool = a->a_pool; rp.slot_idx = a->slot_idx;
  rp.initial_state = a->initial_state; rp.initial_A_state = a->initial_A_state;
  rp.final_state = a->final_state; rp.final_A_state = a->final_A_state;
  rp.o = a->o;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (decode) {
    return a->dtype == PKDA_F32 ? launch_decode<float>(rp, a->head_dim, s) : launch_decode<bf16_t>(rp, a->head_dim, s);
  }
  return a->dtype == PKDA_F32 ? launch_recurrent<float>(rp, a->head_dim, s)
                              : launch_recurrent<bf16_t>(rp, a->head_dim, s);
}

}  // namespace
}  // namespace pkda

extern "C" int pkda_recurrent_fwd(const pkda_recurrent_args* args, void* stream) {
  return pkda::recurrent_entry(args, stream, false);
}

extern "C" int pkda_decode_step(const pkda_recurrent_args* args, void* stream) {
  return pkda::recurrent_entry(args, stream, true);
}
