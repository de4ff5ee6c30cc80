// Fused Q/K/V short convolution + SiLU + per-head L2 normalisation for gfx950,
// forward and backward: the producer of the PKDA recurrence's q, k, v.
//
// Reference: delta_feedback::pkda_qkv_conv and its backward
// (delta_feedback_experiment/fla_ops.py:134-249); the same function in
// portable form is PreconditionedKDA._causal_conv + _l2norm
// (delta_feedback_experiment/pkda.py:37-44,197-220,290-316).  Per channel c of
// x [B, T, C] and token t, with W taps and zero history before t = 0:
//
//   a[t, c] = sum_{w < W} weight[c, w] x[t - (W - 1) + w, c]
//   y[t, c] = silu(a[t, c])
//   out     = y / sqrt(sum_{head} y^2 + eps)   for c < norm_channels (q and k)
//           = y                                 otherwise (v)
//
// all in FP32, cast once to the output dtype; channels [0, P), [P, 2P),
// [2P, 3P) leave as the three slabs q, k, v [B, T, P].
//
// Layout and threads: one thread owns 8 consecutive channels (one 16-byte
// vector of a token row) and walks a tile of tokens with the W - 1 previous
// rows in registers, so each row of x is read once (plus a W - 1 row halo per
// tile) with fully coalesced 16-byte loads; the head's sum of squares is a
// shuffle reduction over the head_dim / 8 lanes that share the head.  The
// backward recomputes a and y for its tile plus the W - 1 rows after it (the
// rows whose gradient reaches the tile's x), and writes dx with the same
// 16-byte stores.  dw is summed per tile in registers and the tiles are
// reduced in a fixed order by a second kernel: deterministic.
#include "pkda_common.h"

namespace pkda {
namespace {

constexpr int kConvThreads = 128;  // 128 x 8 = 1024 channels per workgroup
#ifndef PKDA_CONV_TILE_BWD
#define PKDA_CONV_TILE_BWD 64
#endif
#ifndef PKDA_CONV_GROUP
#define PKDA_CONV_GROUP 4
#endif
#ifndef PKDA_CONV_GROUP_BWD
#define PKDA_CONV_GROUP_BWD 4
#endif
constexpr int kConvTileFwd = 32;                 // tokens per workgroup, forward (swept: 16..64)
constexpr int kConvTile = PKDA_CONV_TILE_BWD;    // tokens per workgroup, backward (and dw partials)
constexpr int kGroup = PKDA_CONV_GROUP;          // token rows loaded together, forward
constexpr int kGroupBwd = PKDA_CONV_GROUP_BWD;   // and backward
constexpr int kDwSlices = 32;                    // first pass of the dw reduction

struct ConvParams {
  const void* x;
  const void* weight;
  int w_dtype;
  const void* dq;  // backward: gradients of the three slabs
  const void* dk;
  const void* dv;
  void* q;         // forward outputs
  void* k;
  void* v;
  void* dx;        // backward outputs
  float* dw_part;  // [tiles, C, W] FP32
  void* dw;        // [C, W] in w_dtype
  const int32_t* slot;   // cached rows: row -> history slot, or null
  const void* hist_in;   // [pool, W - 1, C] or null (zero history)
  void* hist_out;        // [pool, W - 1, C] or null
  int B, T, C, P, head_dim, norm_channels, x_dtype;
  float eps;
  int tiles_per_row;
};

template <typename T> struct Vec8;
template <> struct Vec8<bf16_t> {
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
template <> struct Vec8<float> {
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

// Eight elements kept as raw 16-byte pieces (unpacked when used), so a
// prefetched row costs 4 registers in BF16.
template <typename T>
struct Raw8 {
  static constexpr int N = 8 * sizeof(T) / 16;
  uint4 r[N];
  __device__ __forceinline__ void load(const T* p) {
#pragma unroll
    for (int i = 0; i < N; ++i) r[i] = reinterpret_cast<const uint4*>(p)[i];
  }
  __device__ __forceinline__ void unpack(float* x) const {
    if constexpr (sizeof(T) == 2) {
      const uint32_t w[4] = {r[0].x, r[0].y, r[0].z, r[0].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[2 * i] = __uint_as_float(w[i] << 16);
        x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        x[4 * i] = __uint_as_float(r[i].x); x[4 * i + 1] = __uint_as_float(r[i].y);
        x[4 * i + 2] = __uint_as_float(r[i].z); x[4 * i + 3] = __uint_as_float(r[i].w);
      }
    }
  }
};

// Sum over the G lanes of one head (G a power of two, lanes aligned to G;
// the lanes of a head are active together).
template <int G>
__device__ __forceinline__ float head_sum(float x) {
  if constexpr (G <= 16) {
    return lane_group_sum<G>(x);
  } else {
#pragma unroll
    for (int off = 1; off < G; off <<= 1) x += __shfl_xor(x, off);
    return x;
  }
}

__device__ __forceinline__ float sigmoid_fast(float a) { return 1.f / (1.f + __expf(-a)); }

// The slab (q, k or v) and the offset inside it of channel c.
template <typename T>
__device__ __forceinline__ T* slab_ptr(void* q, void* k, void* v, int P, int c, int64_t row, int& off) {
  const int s = c / P;
  off = c - s * P;
  T* base = static_cast<T*>(s == 0 ? q : s == 1 ? k : v);
  return base + row * P;
}
template <typename T>
__device__ __forceinline__ const T* slab_ptr(const void* q, const void* k, const void* v, int P, int c, int64_t row,
                                             int& off) {
  const int s = c / P;
  off = c - s * P;
  const T* base = static_cast<const T*>(s == 0 ? q : s == 1 ? k : v);
  return base + row * P;
}

// The 8 W taps of this thread's channels are contiguous: one branch on the
// dtype (uniform) around straight-line loads, so they go out together (a
// per-element dtype test made each load wait for the one before).
template <int W>
__device__ __forceinline__ void load_weights(const ConvParams& p, int c0, float (&wt)[8][W]) {
  const int64_t base = (int64_t)c0 * W;
  if (p.w_dtype == PKDA_BF16) {
    const bf16_t* w8 = static_cast<const bf16_t*>(p.weight) + base;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int w = 0; w < W; ++w) wt[j][w] = bf16_to_f32(w8[j * W + w]);
  } else {
    const float* w8 = static_cast<const float*>(p.weight) + base;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int w = 0; w < W; ++w) wt[j][w] = w8[j * W + w];
  }
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <typename T, int W, int G>
__global__ __launch_bounds__(kConvThreads) void qkv_conv_fwd_kernel(ConvParams p) {
  const int tpr = (p.T + kConvTileFwd - 1) / kConvTileFwd;
  const int b = blockIdx.x / tpr;
  const int t0 = (blockIdx.x - b * tpr) * kConvTileFwd;
  const int t1 = min(t0 + kConvTileFwd, p.T);
  const int c0 = (blockIdx.y * kConvThreads + threadIdx.x) * 8;
  if (c0 >= p.C) return;  // whole heads: the lanes of one head leave together
  const bool norm = c0 < p.norm_channels;
  float wt[8][W];
  load_weights<W>(p, c0, wt);
  const T* xs = static_cast<const T*>(p.x) + (int64_t)b * p.T * p.C + c0;
  float hist[W > 1 ? W - 1 : 1][8];  // x at t - (W - 1) .. t - 1
  {
    // the halo rows load unconditionally (row 0 stands in before the row's
    // start) and are replaced below where t < 0, so no branch holds them back
    Raw8<T> hr[W > 1 ? W - 1 : 1];
#pragma unroll
    for (int w = 0; w < W - 1; ++w) hr[w].load(xs + (int64_t)max(t0 - (W - 1) + w, 0) * p.C);
#pragma unroll
    for (int w = 0; w < W - 1; ++w) {
      const int t = t0 - (W - 1) + w;
      if (t >= 0) {
        hr[w].unpack(hist[w]);
      } else if (p.hist_in) {  // the row's cached projections before its first token
        const int64_t sb = p.slot ? p.slot[b] : b;
        Vec8<T>::load(static_cast<const T*>(p.hist_in) + (sb * (W - 1) + (W - 1) + t) * p.C + c0, hist[w]);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) hist[w][j] = 0.f;
      }
    }
  }
  int off;
  T* out = slab_ptr<T>(p.q, p.k, p.v, p.P, c0, (int64_t)b * p.T, off) + off;
  // tokens in groups of kGroup rows, the next group's loads in flight while
  // the current one computes
  Raw8<T> xa[kGroup], xb[kGroup];
  auto load_group = [&](int tg, Raw8<T> (&dst)[kGroup]) {  // rows past the tile clamp (never used)
#pragma unroll
    for (int i = 0; i < kGroup; ++i) dst[i].load(xs + (int64_t)min(tg + i, t1 - 1) * p.C);
  };
  load_group(t0, xa);
  for (int tg = t0; tg < t1; tg += kGroup) {
    if (tg + kGroup < t1) load_group(tg + kGroup, xb);
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
      if (tg + i >= t1) break;
      float xt[8];
      xa[i].unpack(xt);
      float y[8];
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float a = wt[j][W - 1] * xt[j];
#pragma unroll
        for (int w = 0; w < W - 1; ++w) a += wt[j][w] * hist[w][j];
        y[j] = a * sigmoid_fast(a);
        ss += y[j] * y[j];
      }
      if (norm) {
        const float r = rsqrtf(head_sum<G>(ss) + p.eps);
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] *= r;
      }
      Vec8<T>::store(out + (int64_t)(tg + i) * p.P, y);
#pragma unroll
      for (int w = 0; w + 1 < W - 1; ++w)
#pragma unroll
        for (int j = 0; j < 8; ++j) hist[w][j] = hist[w + 1][j];
      if (W > 1)
#pragma unroll
        for (int j = 0; j < 8; ++j) hist[W > 1 ? W - 2 : 0][j] = xt[j];
    }
#pragma unroll
    for (int i = 0; i < kGroup; ++i) xa[i] = xb[i];
  }
  // a row that is one tile (a decode token, a short prompt) leaves its
  // history here: hist holds its last W - 1 rows of history ++ x, and this
  // thread read its slot's old history at the start (in place is safe)
  if constexpr (W > 1) {
    if (p.hist_out && tpr == 1) {
      const int64_t sb = p.slot ? p.slot[b] : b;
#pragma unroll
      for (int w = 0; w < W - 1; ++w) Vec8<T>::store(static_cast<T*>(p.hist_out) + (sb * (W - 1) + w) * p.C + c0, hist[w]);
    }
  }
}

// ---------------------------------------------------------------------------
// backward
//   n = y r, r = (sum y^2 + eps)^-1/2:  dy = r (dn - n sum(n dn))   (q, k)
//   da = dy silu'(a),  silu'(a) = s (1 + a (1 - s)),  s = sigmoid(a)
//   dx[t] = sum_w weight[w] da[t + W - 1 - w],  dw[w] += da[t] x[t - (W - 1) + w]
// ---------------------------------------------------------------------------
template <typename T, int W, int G>
__global__ __launch_bounds__(kConvThreads) void qkv_conv_bwd_kernel(ConvParams p) {
  const int b = blockIdx.x / p.tiles_per_row;
  const int tile = blockIdx.x;
  const int t0 = (blockIdx.x - b * p.tiles_per_row) * kConvTile;
  const int t1 = min(t0 + kConvTile, p.T);
  const int c0 = (blockIdx.y * kConvThreads + threadIdx.x) * 8;
  if (c0 >= p.C) return;
  const bool norm = c0 < p.norm_channels;
  float wt[8][W];
  load_weights<W>(p, c0, wt);
  const T* xs = static_cast<const T*>(p.x) + (int64_t)b * p.T * p.C + c0;
  int off;
  const T* dn_base = slab_ptr<T>(p.dq, p.dk, p.dv, p.P, c0, (int64_t)b * p.T, off) + off;
  T* dxs = static_cast<T*>(p.dx) + (int64_t)b * p.T * p.C + c0;

  float hist[W][8];   // x at t - (W - 1) .. t (hist[W - 1] = x[t] once loaded)
  float dwin[W][8];   // da at t - (W - 1) .. t
  float dw[8][W];
#pragma unroll
  for (int w = 0; w < W; ++w)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      dwin[w][j] = 0.f;
      dw[j][w] = 0.f;
    }
  {
    // halo rows unconditionally (row 0 stands in before the row's start, then zeroed)
    Raw8<T> hr[W > 1 ? W - 1 : 1];
#pragma unroll
    for (int w = 0; w < W - 1; ++w) hr[w].load(xs + (int64_t)max(t0 - (W - 1) + w, 0) * p.C);
#pragma unroll
    for (int w = 0; w < W - 1; ++w) {
      hr[w].unpack(hist[w]);
      if (t0 - (W - 1) + w < 0)
#pragma unroll
        for (int j = 0; j < 8; ++j) hist[w][j] = 0.f;
    }
  }
  const int tend = t1 + W - 1;  // da of the W - 1 rows after the tile reaches its dx
  Raw8<T> xa[kGroupBwd], xb[kGroupBwd], na[kGroupBwd], nb[kGroupBwd];
  const int tlast = min(tend, p.T);
  auto load_group = [&](int tg, Raw8<T> (&dx_)[kGroupBwd], Raw8<T> (&dn_)[kGroupBwd]) {
    // rows past the last clamp (never used): no branch holds a load back
#pragma unroll
    for (int i = 0; i < kGroupBwd; ++i) {
      const int t = min(tg + i, tlast - 1);
      dx_[i].load(xs + (int64_t)t * p.C);
      dn_[i].load(dn_base + (int64_t)t * p.P);
    }
  };
  load_group(t0, xa, na);
  for (int tg = t0; tg < tend; tg += kGroupBwd) {
    if (tg + kGroupBwd < tlast) load_group(tg + kGroupBwd, xb, nb);
#pragma unroll
    for (int i = 0; i < kGroupBwd; ++i) {
      const int t = tg + i;
      if (t >= tend) break;
      float da[8];
      if (t < p.T) {
        xa[i].unpack(hist[W - 1]);
        float dn[8];
        na[i].unpack(dn);
        float a[8], y[8];
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          a[j] = 0.f;
#pragma unroll
          for (int w = 0; w < W; ++w) a[j] += wt[j][w] * hist[w][j];
          y[j] = a[j] * sigmoid_fast(a[j]);
          ss += y[j] * y[j];
        }
        float dy[8];
        if (norm) {
          const float r = rsqrtf(head_sum<G>(ss) + p.eps);
          float nd = 0.f;
#pragma unroll
          for (int j = 0; j < 8; ++j) nd += y[j] * r * dn[j];
          nd = head_sum<G>(nd);
#pragma unroll
          for (int j = 0; j < 8; ++j) dy[j] = r * (dn[j] - y[j] * r * nd);
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) dy[j] = dn[j];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float s = sigmoid_fast(a[j]);
          da[j] = dy[j] * s * (1.f + a[j] * (1.f - s));
        }
        if (t < t1) {
#pragma unroll
          for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int w = 0; w < W; ++w) dw[j][w] += da[j] * hist[w][j];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) da[j] = 0.f;
      }
      // slide the windows: dwin holds da[t - (W - 1) .. t]
#pragma unroll
      for (int w = 0; w + 1 < W; ++w)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          dwin[w][j] = dwin[w + 1][j];
          hist[w][j] = hist[w + 1][j];
        }
#pragma unroll
      for (int j = 0; j < 8; ++j) dwin[W - 1][j] = da[j];
      const int s = t - (W - 1);  // every da that reaches x[s] is known now
      if (s >= t0) {
        float dx[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float acc = 0.f;
#pragma unroll
          for (int w = 0; w < W; ++w) acc += wt[j][w] * dwin[W - 1 - w][j];
          dx[j] = acc;
        }
        Vec8<T>::store(dxs + (int64_t)s * p.C, dx);
      }
    }
#pragma unroll
    for (int i = 0; i < kGroupBwd; ++i) {
      xa[i] = xb[i];
      na[i] = nb[i];
    }
  }
  float* part = p.dw_part + ((int64_t)tile * p.C + c0) * W;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int w = 0; w < W; ++w) part[j * W + w] = dw[j][w];
}

// dw[c, w] = sum over tiles of dw_part[tile, c, w] in a fixed order, in two
// passes: slice y sums tiles y, y + S, y + 2S, ... and leaves the sum in place
// of tile y (only this thread ever reads that entry), then the S slice sums
// are added in order.
__global__ __launch_bounds__(256) void qkv_conv_dw_slices_kernel(ConvParams p, int W, int tiles, int S) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  const int y = blockIdx.y;
  const int64_t CW = (int64_t)p.C * W;
  if (e >= CW) return;
  float s = 0.f;
  for (int t = y; t < tiles; t += S) s += p.dw_part[t * CW + e];
  p.dw_part[y * CW + e] = s;
}

__global__ __launch_bounds__(256) void qkv_conv_dw_kernel(ConvParams p, int W, int S) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  const int64_t CW = (int64_t)p.C * W;
  if (e >= CW) return;
  float s = 0.f;
  for (int y = 0; y < S; ++y) s += p.dw_part[y * CW + e];
  if (p.w_dtype == PKDA_BF16) {
    static_cast<bf16_t*>(p.dw)[e] = f32_to_bf16(s);
  } else {
    static_cast<float*>(p.dw)[e] = s;
  }
}

// ---------------------------------------------------------------------------
// decode tokens: rows of one token, each continuing its slot's history.  A
// thread owns 8 channels of kTokRows rows: it loads its weights once, and
// every row's W - 1 history rows and new projection row before computing;
// out = the normalised silu(conv), and the slot's history shifts by one row
// in place (each thread reads its channels' rows before writing them).
// ---------------------------------------------------------------------------
constexpr int kTokRows = 8;

template <typename T, int W, int G>
__global__ __launch_bounds__(kConvThreads) void qkv_conv_token_kernel(ConvParams p) {
  const int c0 = (blockIdx.y * kConvThreads + threadIdx.x) * 8;
  if (c0 >= p.C) return;
  const bool norm = c0 < p.norm_channels;
  float wt[8][W];
  load_weights<W>(p, c0, wt);
  const int b0 = blockIdx.x * kTokRows;
  const int nb = min(kTokRows, p.B - b0);
  Raw8<T> hr[kTokRows][W - 1], xr[kTokRows];
#pragma unroll
  for (int r = 0; r < kTokRows; ++r) {
    if (r >= nb) break;
    const int b = b0 + r;
    const int64_t sb = p.slot ? p.slot[b] : b;
    xr[r].load(static_cast<const T*>(p.x) + (int64_t)b * p.C + c0);
#pragma unroll
    for (int w = 0; w < W - 1; ++w) {
      if (p.hist_in) {
        hr[r][w].load(static_cast<const T*>(p.hist_in) + (sb * (W - 1) + w) * p.C + c0);
      } else {
#pragma unroll
        for (int i = 0; i < Raw8<T>::N; ++i) hr[r][w].r[i] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kTokRows; ++r) {
    if (r >= nb) break;
    const int b = b0 + r;
    const int64_t sb = p.slot ? p.slot[b] : b;
    float xt[8], hist[W - 1][8];
    xr[r].unpack(xt);
#pragma unroll
    for (int w = 0; w < W - 1; ++w) hr[r][w].unpack(hist[w]);
    float y[8];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float a = wt[j][W - 1] * xt[j];
#pragma unroll
      for (int w = 0; w < W - 1; ++w) a += wt[j][w] * hist[w][j];
      y[j] = a * sigmoid_fast(a);
      ss += y[j] * y[j];
    }
    if (norm) {
      const float rn = rsqrtf(head_sum<G>(ss) + p.eps);
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] *= rn;
    }
    int off;
    T* out = slab_ptr<T>(p.q, p.k, p.v, p.P, c0, (int64_t)b, off) + off;
    Vec8<T>::store(out, y);
    if (p.hist_out) {
      T* ho = static_cast<T*>(p.hist_out) + sb * (W - 1) * p.C + c0;
#pragma unroll
      for (int w = 0; w + 1 < W - 1; ++w) Vec8<T>::store(ho + (int64_t)w * p.C, hist[w + 1]);
      Vec8<T>::store(ho + (int64_t)(W - 2) * p.C, xt);
    }
  }
}

// ---------------------------------------------------------------------------
// cached rows longer than one forward tile: the history left for the next
// call, the last W - 1 rows of history ++ x.  One thread per 8 channels of
// one row reads every row it needs before writing any, so history_out may
// alias history_in; it runs after the forward kernel (whose first tile of a
// row reads history_in) on the same stream.
// ---------------------------------------------------------------------------
template <typename T, int W>
__global__ __launch_bounds__(kConvThreads) void qkv_conv_history_kernel(ConvParams p) {
  const int b = blockIdx.x;
  const int c0 = (blockIdx.y * kConvThreads + threadIdx.x) * 8;
  if (c0 >= p.C) return;
  const int64_t sb = p.slot ? p.slot[b] : b;
  const T* xs = static_cast<const T*>(p.x) + (int64_t)b * p.T * p.C + c0;
  float rows[W - 1][8];
#pragma unroll
  for (int j = 0; j < W - 1; ++j) {
    const int t = p.T - (W - 1) + j;  // position relative to the row's first token
    if (t >= 0) {
      Vec8<T>::load(xs + (int64_t)t * p.C, rows[j]);
    } else if (p.hist_in) {
      Vec8<T>::load(static_cast<const T*>(p.hist_in) + (sb * (W - 1) + (W - 1) + t) * p.C + c0, rows[j]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) rows[j][e] = 0.f;
    }
  }
#pragma unroll
  for (int j = 0; j < W - 1; ++j) Vec8<T>::store(static_cast<T*>(p.hist_out) + (sb * (W - 1) + j) * p.C + c0, rows[j]);
}

template <typename T, int W, int G>
int launch_conv(const ConvParams& p, bool backward, hipStream_t s) {
  const int cblocks = (p.C + 8 * kConvThreads - 1) / (8 * kConvThreads);
  if (!backward) {
    if constexpr (W > 1) {
      if (p.T == 1 && (p.hist_in || p.hist_out)) {  // decode tokens
        hipLaunchKernelGGL((qkv_conv_token_kernel<T, W, G>), dim3((p.B + kTokRows - 1) / kTokRows, cblocks),
                           dim3(kConvThreads), 0, s, p);
        return launch_status("pkda_qkv_conv_fwd(token)");
      }
    }
    if (p.T > 0) {
      const int tiles = p.B * ((p.T + kConvTileFwd - 1) / kConvTileFwd);
      hipLaunchKernelGGL((qkv_conv_fwd_kernel<T, W, G>), dim3(tiles, cblocks), dim3(kConvThreads), 0, s, p);
      if (int st = launch_status("pkda_qkv_conv_fwd")) return st;
    }
    if constexpr (W > 1) {
      if (p.hist_out && (p.T == 0 || p.T > kConvTileFwd)) {  // else the forward kernel wrote it
        hipLaunchKernelGGL((qkv_conv_history_kernel<T, W>), dim3(p.B, cblocks), dim3(kConvThreads), 0, s, p);
        return launch_status("pkda_qkv_conv_fwd(history)");
      }
    }
    return 0;
  }
  const int tiles = p.B * p.tiles_per_row;
  hipLaunchKernelGGL((qkv_conv_bwd_kernel<T, W, G>), dim3(tiles, cblocks), dim3(kConvThreads), 0, s, p);
  if (int st = launch_status("pkda_qkv_conv_bwd")) return st;
  const int S = min(kDwSlices, tiles);
  const int eblocks = (p.C * W + 255) / 256;
  hipLaunchKernelGGL(qkv_conv_dw_slices_kernel, dim3(eblocks, S), dim3(256), 0, s, p, W, tiles, S);
  if (int st = launch_status("pkda_qkv_conv_bwd(dw slices)")) return st;
  hipLaunchKernelGGL(qkv_conv_dw_kernel, dim3(eblocks), dim3(256), 0, s, p, W, S);
  return launch_status("pkda_qkv_conv_bwd(dw)");
}

template <typename T, int G>
int dispatch_w(const ConvParams& p, int W, bool backward, hipStream_t s) {
  switch (W) {
    case 1: return launch_conv<T, 1, G>(p, backward, s);
    case 2: return launch_conv<T, 2, G>(p, backward, s);
    case 3: return launch_conv<T, 3, G>(p, backward, s);
    case 4: return launch_conv<T, 4, G>(p, backward, s);
    default: set_error("conv_size %d not built (1..4)", W); return PKDA_EUNSUPPORTED;
  }
}

template <typename T>
int dispatch(const ConvParams& p, int W, bool backward, hipStream_t s) {
  switch (p.head_dim / 8) {
    case 4: return dispatch_w<T, 4>(p, W, backward, s);
    case 8: return dispatch_w<T, 8>(p, W, backward, s);
    case 16: return dispatch_w<T, 16>(p, W, backward, s);
    default: set_error("head_dim %d not built (32, 64, 128)", p.head_dim); return PKDA_EUNSUPPORTED;
  }
}

int conv_call(const pkda_qkv_conv_args* a, void* stream, bool backward) {
  PKDA_REQUIRE(a != nullptr, PKDA_EINVAL, "null args");
  PKDA_REQUIRE(a->struct_size == (int32_t)sizeof(pkda_qkv_conv_args), PKDA_EINVAL, "pkda_qkv_conv_args size mismatch");
  PKDA_REQUIRE(a->dtype == PKDA_F32 || a->dtype == PKDA_BF16, PKDA_EUNSUPPORTED, "dtype %d", a->dtype);
  PKDA_REQUIRE(a->w_dtype == PKDA_F32 || a->w_dtype == PKDA_BF16, PKDA_EUNSUPPORTED, "weight dtype %d", a->w_dtype);
  PKDA_REQUIRE(a->batch >= 0 && a->seqlen >= 0 && a->width > 0, PKDA_EINVAL, "sizes");
  PKDA_REQUIRE(a->head_dim == 32 || a->head_dim == 64 || a->head_dim == 128, PKDA_EUNSUPPORTED, "head_dim %d",
               a->head_dim);
  PKDA_REQUIRE(a->width % a->head_dim == 0, PKDA_EINVAL, "slab width %d is not a multiple of head_dim %d", a->width,
               a->head_dim);
  PKDA_REQUIRE(a->norm_channels >= 0 && a->norm_channels <= 3 * a->width && a->norm_channels % a->head_dim == 0,
               PKDA_EINVAL, "norm_channels %d", a->norm_channels);
  PKDA_REQUIRE(a->conv_size >= 1 && a->conv_size <= 4, PKDA_EUNSUPPORTED, "conv_size %d (1..4)", a->conv_size);
  ConvParams p;
  p.B = a->batch;
  p.T = a->seqlen;
  p.P = a->width;
  p.C = 3 * a->width;
  p.head_dim = a->head_dim;
  p.norm_channels = a->norm_channels;
  p.x_dtype = a->dtype;
  p.eps = a->eps;
  p.tiles_per_row = (a->seqlen + kConvTile - 1) / kConvTile;
  p.x = a->x;
  p.weight = a->weight;
  p.w_dtype = a->w_dtype;
  p.q = a->q; p.k = a->k; p.v = a->v;
  p.dq = a->dq; p.dk = a->dk; p.dv = a->dv;
  p.dx = a->dx; p.dw = a->dw; p.dw_part = a->dw_part;
  p.slot = a->slot_idx;
  p.hist_in = a->history_in;
  p.hist_out = a->history_out;
  const bool cached = a->history_in || a->history_out;
  PKDA_REQUIRE(!backward || !cached, PKDA_EUNSUPPORTED, "conv histories are a forward (cached rows) feature");
  PKDA_REQUIRE(!cached || a->conv_size > 1, PKDA_EINVAL, "conv_size 1 keeps no history");
  PKDA_REQUIRE(!a->slot_idx || a->pool_size > 0, PKDA_EINVAL, "slot-indexed histories need pool_size > 0");
  if (p.B == 0 || (p.T == 0 && !(a->history_out && !backward))) {
    PKDA_REQUIRE(!backward || a->dw, PKDA_EINVAL, "null dw");
    return 0;  // an empty batch: nothing to launch (dw is the caller's zeros)
  }
  if (backward) {
    PKDA_REQUIRE(a->x && a->weight && a->dq && a->dk && a->dv && a->dx && a->dw && a->dw_part, PKDA_EINVAL,
                 "null tensor");
  } else {
    PKDA_REQUIRE(p.T == 0 || (a->x && a->weight && a->q && a->k && a->v), PKDA_EINVAL, "null tensor");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  return a->dtype == PKDA_BF16 ? dispatch<bf16_t>(p, a->conv_size, backward, s)
                               : dispatch<float>(p, a->conv_size, backward, s);
}

}  // namespace
}  // namespace pkda

extern "C" int64_t pkda_qkv_conv_workspace(int32_t batch, int32_t seqlen, int32_t width, int32_t conv_size) {
  const int64_t tiles = (int64_t)batch * ((seqlen + pkda::kConvTile - 1) / pkda::kConvTile);
  return tiles * 3 * (int64_t)width * conv_size;
}

extern "C" int pkda_qkv_conv_fwd(const pkda_qkv_conv_args* args, void* stream) {
  return pkda::conv_call(args, stream, false);
}

extern "C" int pkda_qkv_conv_bwd(const pkda_qkv_conv_args* args, void* stream) {
  return pkda::conv_call(args, stream, true);
}
