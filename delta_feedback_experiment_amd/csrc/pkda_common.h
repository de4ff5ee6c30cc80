// Shared device and host helpers for the gfx950 PKDA kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "pkda_gfx950.h"

namespace pkda {

// ----------------------------------------------------------------------------
// Error reporting (host).  One message per calling thread.
// ----------------------------------------------------------------------------
void set_error(const char* fmt, ...);

#define PKDA_REQUIRE(cond, code, ...)          \
  do {                                         \
    if (!(cond)) {                             \
      ::pkda::set_error(__VA_ARGS__);          \
      return (code);                           \
    }                                          \
  } while (0)

inline int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return static_cast<int>(e);
  }
  return 0;
}

// ----------------------------------------------------------------------------
// bf16 <-> f32 (round to nearest even, NaN preserved), on raw 16-bit storage.
// ----------------------------------------------------------------------------
typedef uint16_t bf16_t;

__device__ __forceinline__ float bf16_to_f32(bf16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// gfx950 converts natively (v_cvt_pk_bf16_f32: round to nearest even).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(bf16_t, static_cast<__bf16>(f));
}

// e^x as 2^(x log2 e) on the hardware exp2 (v_exp_f32).  The rounding of the
// scaled argument costs a relative error of about |x| 6e-8; the chunk
// kernels take it on decay factors e^(G_t - G_s) <= 1.
constexpr float kLog2e = 1.44269504088896341f;
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
// 2^x on the hardware exp2: e^y for an argument already scaled, x = y log2 e
// (a cumulative log decay staged once as G log2 e saves the multiply on every
// pair that differences it)
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// ln x as log2(x) ln 2 on the hardware log2 (v_log_f32), for x > 0 normal.
__device__ __forceinline__ float log_fast(float x) { return __builtin_amdgcn_logf(x) * 0.693147180559945309f; }

// a / b as a * (1 / b) on the hardware reciprocal (v_rcp_f32, 1 ulp).
__device__ __forceinline__ float div_fast(float a, float b) { return a * __builtin_amdgcn_rcpf(b); }

template <typename T> struct io;
template <> struct io<float> {
  static constexpr int dtype = PKDA_F32;
  __device__ __forceinline__ static float load(const float* p) { return *p; }
  __device__ __forceinline__ static void store(float* p, float v) { *p = v; }
};
template <> struct io<bf16_t> {
  static constexpr int dtype = PKDA_BF16;
  __device__ __forceinline__ static float load(const bf16_t* p) { return bf16_to_f32(*p); }
  __device__ __forceinline__ static void store(bf16_t* p, float v) { *p = f32_to_bf16(v); }
};

// Load four consecutive elements as floats (16-byte or 8-byte vector loads).
__device__ __forceinline__ float4 load4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 load4(const bf16_t* p) {
  uint2 r = *reinterpret_cast<const uint2*>(p);
  return make_float4(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u),
                     __uint_as_float(r.y << 16), __uint_as_float(r.y & 0xffff0000u));
}
__device__ __forceinline__ void store4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
__device__ __forceinline__ void store4(bf16_t* p, float4 v) {
  uint2 r;
  r.x = static_cast<uint32_t>(f32_to_bf16(v.x)) | (static_cast<uint32_t>(f32_to_bf16(v.y)) << 16);
  r.y = static_cast<uint32_t>(f32_to_bf16(v.z)) | (static_cast<uint32_t>(f32_to_bf16(v.w)) << 16);
  *reinterpret_cast<uint2*>(p) = r;
}

// Scalar load of a runtime-typed element.
__device__ __forceinline__ float load_any(const void* p, int64_t i, int dtype) {
  return dtype == PKDA_BF16 ? bf16_to_f32(static_cast<const bf16_t*>(p)[i])
                            : static_cast<const float*>(p)[i];
}

// torch.nn.functional.softplus with beta = 1, threshold = 20.
// softplus(z) and sigmoid(z) from one e = e^{-|z|} in (0, 1] on the hardware
// exp2 / log2 / reciprocal units:
//   softplus = max(z, 0) + log1p(e),   sigmoid = (z >= 0 ? 1 : e) / (1 + e),
// with log1p(e) = log(u) e / (u - 1), u = 1 + e, which cancels the rounding
// of 1 + e (D. Goldberg, "What every computer scientist should know about
// floating-point arithmetic", 1991, Theorem 4); u == 1 leaves log1p(e) = e.
// A few ulps from the correctly rounded values; for z > 20 softplus is z
// (log1p(e) < ulp(z)), as torch's softplus with its threshold of 20 gives.
struct SoftplusSigmoid {
  float softplus, sigmoid;
};
__device__ __forceinline__ SoftplusSigmoid softplus_sigmoid_fast(float z) {
  const float e = __builtin_amdgcn_exp2f(-fabsf(z) * 1.44269504088896341f);
  const float u = 1.f + e;
  const float l = u == 1.f ? e : __builtin_amdgcn_logf(u) * 0.693147180559945309f * (e * __builtin_amdgcn_rcpf(u - 1.f));
  return {fmaxf(z, 0.f) + l, (z >= 0.f ? 1.f : e) * __builtin_amdgcn_rcpf(u)};
}

// Sequence bounds for flat token tensors: packed documents or equal rows.
struct SeqBounds {
  int64_t start;
  int32_t len;
};
__device__ __forceinline__ SeqBounds seq_bounds(const int32_t* cu, int n, int seqlen) {
  SeqBounds b;
  if (cu) {
    b.start = cu[n];
    b.len = cu[n + 1] - cu[n];
  } else {
    b.start = static_cast<int64_t>(n) * seqlen;
    b.len = seqlen;
  }
  return b;
}

// Sum over each aligned group of N = 2, 4, 8 or 16 consecutive lanes (a
// pair, a quad, a DPP half-row or row), every lane of the group getting it:
// the butterfly over lane ^ 1, lane ^ 2, lane ^ 4 and lane ^ 8, each step
// own + moved, with DPP lane moves (VALU) instead of permutes through the LDS
// crossbar.  After the two quad steps every lane of a quad holds the quad's
// sum, so the half-row and row mirrors bring the same partner values as
// lane ^ 4 and lane ^ 8: the same additions in the same order as the
// shuffle butterfly.  Every lane of each group must be active (lanes of
// other groups need not be).
template <int N>
__device__ __forceinline__ float lane_group_sum(float v) {
  static_assert(N == 2 || N == 4 || N == 8 || N == 16, "2, 4, 8 or 16 lanes");
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));  // quad [1,0,3,2]
  if constexpr (N >= 4)
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));  // quad [2,3,0,1]
  if constexpr (N >= 8)
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));  // half-row mirror
  if constexpr (N == 16)
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));  // row mirror
  return v;
}

}  // namespace pkda
