// Chunk geometry, LDS tile movement and wave64 MFMA tiles for the chunked
// PKDA kernels (gfx950).
//
// Token tensors are flat [N_tok, H, D].  A "document" is either one of
// `num_seqs` equal rows of `seqlen` tokens or a cu_seqlens span; chunks of
// C = 64 tokens start at each document's first token, so the last chunk of a
// document may be partial.  Per-chunk kernels see a chunk as
// (document n, first token, length, chunk id); per-document kernels walk the
// chunk ids of their document in order.
#pragma once

#include "pkda_common.h"

namespace pkda {

constexpr int C = PKDA_CHUNK;  // 64
constexpr int kWG = 256;       // 4 waves
// Sequential state passes: 16 waves when the [D x BV] state slice splits
// into whole pairs of 16x16 tiles per wave, else 8.
constexpr int state_threads(int D, int BV) { return ((D / 16) * (BV / 16)) % 16 == 0 ? 1024 : 512; }
// BF16 with a per-head gate: the state passes form W S and W^T dU from T and K
// (W = T diag(beta e^G) K, u = T diag(beta) V are never stored).
template <typename T> constexpr bool implicit_w() { return __is_same(T, bf16_t); }

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// ----------------------------------------------------------------------------
// Chunk geometry
// ----------------------------------------------------------------------------
struct ChunkGeom {
  int num_seqs;
  int seqlen;          // equal rows (cu == nullptr)
  int nt;              // chunks per row, equal rows
  const int32_t* cu;   // [num_seqs+1] or nullptr
  const int4* table;   // [num_chunks] {n, start, len, -} (varlen)
  const int32_t* offsets;  // [num_seqs+1] first chunk id of each document (varlen)
  const int32_t* order;    // [num_seqs] documents by length, longest first (varlen)
  int num_chunks;      // launch bound
};

struct ChunkInfo {
  int n;
  int start;
  int len;  // 0: empty slot of the varlen launch bound
};

// Host: fill a ChunkGeom from the entry-point arguments (validates them).
int chunk_geom_from(const int32_t* cu, int num_seqs, int seqlen, int num_chunks, const int32_t* table, ChunkGeom& g);

// (chunk, head) of a workgroup on the 1-D grid of chunk_grid<XCD>(num_chunks,
// H) workgroups, heads fastest: the workgroups resident together read the H
// heads' adjacent pieces of the same token rows of a [token][head][channel]
// tensor (4 KB spans at H D = 2048 BF16), not one head's pieces of rows that
// far apart.  Workgroup b runs on XCD b % 8.  With XCD, slot l = b / 8 of
// XCD x is head l % H of chunk 8 (l / H) + x: an XCD takes whole chunks, all
// H heads in a row, so the per-token lines of [token][head] values (the
// per-head gate, beta: 16 heads share a line) come through one L2 instead of
// eight, and the eight XCDs work on eight adjacent chunks at a time; the
// chunk count is padded to a multiple of 8, and a workgroup with
// cid >= num_chunks has no work.  Without XCD, b = cid H + h.  (The per-head
// kernels take the XCD order; the per-channel kernels, whose per-token lines
// belong to one head, measured faster without it.)
constexpr int kXcds = 8;
struct ChunkHead {
  int cid, h;
};
template <bool XCD>
__host__ __device__ inline unsigned chunk_grid(int num_chunks, int H) {
  const int64_t nc = XCD ? (int64_t)(num_chunks + kXcds - 1) / kXcds * kXcds : num_chunks;
  return (unsigned)(nc * H);
}
template <bool XCD>
__device__ __forceinline__ ChunkHead chunk_head(int H) {
  const int b = blockIdx.x;
  if constexpr (XCD) {
    const int l = b / kXcds;
    const int cl = l / H;
    return {cl * kXcds + (b - l * kXcds), l - cl * H};
  } else {
    const int c = b / H;
    return {c, b - c * H};
  }
}

__device__ __forceinline__ ChunkInfo chunk_info(const ChunkGeom& g, int c) {
  ChunkInfo ci;
  if (g.cu) {
    const int4 e = g.table[c];
    ci.n = e.x;
    ci.start = e.y;
    ci.len = e.z;
  } else {
    ci.n = c / g.nt;
    const int j = c - ci.n * g.nt;
    ci.start = ci.n * g.seqlen + j * C;
    ci.len = min(C, g.seqlen - j * C);
  }
  return ci;
}

// First chunk id, chunk count and first token of document n.
// Per-document launches run on a 1-D grid of num_seqs * H * S workgroups
// (S value slices per head): the H * S workgroups of one document are
// consecutive, slice-major (the slices of one (document, head) are H apart,
// so on one XCD and its L2 when H % 8 == 0), and packed documents come
// longest first, so the longest sequential passes start before the short
// ones fill in behind them.
struct DocSlot {
  int n, h, z;
};
__device__ __forceinline__ DocSlot doc_slot(const ChunkGeom& g, int H, int S) {
  const int hs = H * S;
  const int rank = blockIdx.x / hs;
  const int r = blockIdx.x - rank * hs;
  DocSlot d;
  d.n = g.order ? g.order[rank] : rank;
  d.z = r / H;
  d.h = r - d.z * H;
  return d;
}
inline dim3 doc_grid(int num_seqs, int H, int S) { return dim3((unsigned)((int64_t)num_seqs * H * S)); }

__device__ __forceinline__ void doc_chunks(const ChunkGeom& g, int n, int& first, int& count, int& start, int& len) {
  if (g.cu) {
    first = g.offsets[n];
    count = g.offsets[n + 1] - first;
    start = g.cu[n];
    len = g.cu[n + 1] - start;
  } else {
    first = n * g.nt;
    count = g.nt;
    start = n * g.seqlen;
    len = g.seqlen;
  }
}

// ----------------------------------------------------------------------------
// MFMA 16x16 tiles.  C layout (both types): lane l holds
//   acc[j] = C[4*(l>>4) + j][l & 15],  j = 0..3.
// Operand views in LDS:
//   A (M x K): ROW -> A[m*lda + k];  COL -> A[k*lda + m]
//   B (K x N): ROW -> B[k*ldb + n];  COL -> B[n*ldb + k]
// bf16 tiles read as A=ROW, B=COL take one 16-byte LDS read per lane; the
// k-major views (A=COL, B=ROW) take two transposing 8-byte reads, so every
// tile can stay in its natural row-major layout.  FP32 tiles read one element
// per lane and are cheap in every view.  k-major bf16 tiles need ld % 4 == 0
// and 8-byte aligned tile origins.
// ----------------------------------------------------------------------------
enum { ROW = 0, COL = 1 };

template <typename E> struct Mma;

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;

// Eight k-consecutive bf16 of one column of a k-major LDS tile (element
// (k, n) at p[k * ld + n], p already offset to the tile's column 0), as the
// MFMA 16x16x32 operand of this lane: lane 16q + i receives column i, rows
// k0 + 8q .. k0 + 8q + 7.  Two ds_read_b64_tr_b16: inside each 16-lane group
// lane 4r + c addresses row r, columns 4c .. 4c + 3 of a 4 x 16 block and
// lane i receives column i of the four rows.
__device__ __forceinline__ s16x8_t lds_read_kmajor(const bf16_t* p, int ld, int k0, int lane) {
  const int i = lane & 15, q = lane >> 4;
  const bf16_t* src = p + (k0 + 8 * q + (i >> 2)) * ld + 4 * (i & 3);
  const bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(src));
  const bf16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(src + 4 * ld));
  const s16x4_t l = __builtin_bit_cast(s16x4_t, lo), h = __builtin_bit_cast(s16x4_t, hi);
  return s16x8_t{l[0], l[1], l[2], l[3], h[0], h[1], h[2], h[3]};
}

// Four k-consecutive bf16 of one column of a k-major LDS tile (element (k, n)
// at p[k * ld + n]), as the operand of a 16x16x16 MFMA step: lane 16q + i
// receives column i, rows k0 + 4q .. k0 + 4q + 3 (one ds_read_b64_tr_b16).
__device__ __forceinline__ s16x4_t lds_read_kmajor4(const bf16_t* p, int ld, int k0, int lane) {
  const int i = lane & 15, q = lane >> 4;
  const bf16_t* src = p + (k0 + 4 * q + (i >> 2)) * ld + 4 * (i & 3);
  return __builtin_bit_cast(s16x4_t, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(src)));
}

// acc += A B over one 16-deep k-step (bf16 operands, four k per lane: lane
// 16q + i holds row / column i, k = 4q .. 4q + 3).
__device__ __forceinline__ void mfma16_bf16(f32x4& acc, const s16x4_t& a, const s16x4_t& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, acc, 0, 0, 0);
}

// Four floats rounded to bf16 (nearest even), packed as an operand.
__device__ __forceinline__ s16x4_t pack_bf16x4(const float* x) {
  return s16x4_t{static_cast<short>(f32_to_bf16(x[0])), static_cast<short>(f32_to_bf16(x[1])),
                 static_cast<short>(f32_to_bf16(x[2])), static_cast<short>(f32_to_bf16(x[3]))};
}

// Operand fragments of one MFMA k-step, loaded on their own (frag_a / frag_b
// on tiles already offset to row m0 / column n0) so a phase can hold
// operands that several products share, and mfma() on them.
template <> struct Mma<bf16_t> {
  static constexpr int KS = 32;
  using Frag = s16x8_t;
  template <int LA>
  __device__ __forceinline__ static Frag frag_a(const bf16_t* A, int lda, int k0, int lane) {
    if constexpr (LA == ROW) {
      return *reinterpret_cast<const s16x8_t*>(A + (lane & 15) * lda + k0 + (lane >> 4) * 8);
    } else {
      return lds_read_kmajor(A, lda, k0, lane);
    }
  }
  template <int LB>
  __device__ __forceinline__ static Frag frag_b(const bf16_t* B, int ldb, int k0, int lane) {
    return frag_a<LB == COL ? ROW : COL>(B, ldb, k0, lane);
  }
  __device__ __forceinline__ static void mfma(f32x4& acc, const Frag& a, const Frag& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                  acc, 0, 0, 0);
  }
  template <int LA, int LB>
  __device__ __forceinline__ static void step(f32x4& acc, const bf16_t* A, int lda, const bf16_t* B, int ldb,
                                              int k0, int lane) {
    mfma(acc, frag_a<LA>(A, lda, k0, lane), frag_b<LB>(B, ldb, k0, lane));
  }
};

template <> struct Mma<float> {
  static constexpr int KS = 4;
  using Frag = float;
  template <int LA>
  __device__ __forceinline__ static Frag frag_a(const float* A, int lda, int k0, int lane) {
    const int r = lane & 15, kq = lane >> 4;
    return (LA == ROW) ? A[r * lda + k0 + kq] : A[(k0 + kq) * lda + r];
  }
  template <int LB>
  __device__ __forceinline__ static Frag frag_b(const float* B, int ldb, int k0, int lane) {
    return frag_a<LB == COL ? ROW : COL>(B, ldb, k0, lane);
  }
  __device__ __forceinline__ static void mfma(f32x4& acc, const Frag& a, const Frag& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
  }
  template <int LA, int LB>
  __device__ __forceinline__ static void step(f32x4& acc, const float* A, int lda, const float* B, int ldb, int k0,
                                              int lane) {
    mfma(acc, frag_a<LA>(A, lda, k0, lane), frag_b<LB>(B, ldb, k0, lane));
  }
};

// acc += A[m0:m0+16, 0:K] * B[0:K, n0:n0+16]
template <typename E, int LA, int LB>
__device__ __forceinline__ void mma_tile(f32x4& acc, const E* A, int lda, int m0, const E* B, int ldb, int n0, int K,
                                         int lane) {
  const E* a = (LA == ROW) ? A + m0 * lda : A + m0;
  const E* b = (LB == COL) ? B + n0 * ldb : B + n0;
  for (int k0 = 0; k0 < K; k0 += Mma<E>::KS) Mma<E>::template step<LA, LB>(acc, a, lda, b, ldb, k0, lane);
}

// acc += A[m0:m0+16, kb:ke] * B[kb:ke, n0:n0+16]; kb, ke multiples of Mma<E>::KS.
template <typename E, int LA, int LB>
__device__ __forceinline__ void mma_tile_range(f32x4& acc, const E* A, int lda, int m0, const E* B, int ldb, int n0,
                                               int kb, int ke, int lane) {
  const E* a = (LA == ROW) ? A + m0 * lda : A + m0;
  const E* b = (LB == COL) ? B + n0 * ldb : B + n0;
  for (int k0 = kb; k0 < ke; k0 += Mma<E>::KS) Mma<E>::template step<LA, LB>(acc, a, lda, b, ldb, k0, lane);
}

// One lane's operand elements of a 16x16 MFMA k-step whose k index is
// contiguous in memory (N consecutive k from off(lane)), and the MFMA on
// operands given as floats.
template <typename E> struct FragK;
template <> struct FragK<bf16_t> {
  static constexpr int N = 8;
  __device__ __forceinline__ static int off(int lane) { return 8 * (lane >> 4); }
  __device__ __forceinline__ static void mfma(f32x4& acc, const float* a, const float* b) {
    s16x8_t av, bv;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      av[j] = static_cast<short>(f32_to_bf16(a[j]));
      bv[j] = static_cast<short>(f32_to_bf16(b[j]));
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av), __builtin_bit_cast(bf16x8_t, bv),
                                                  acc, 0, 0, 0);
  }
};
template <> struct FragK<float> {
  static constexpr int N = 1;
  __device__ __forceinline__ static int off(int lane) { return lane >> 4; }
  __device__ __forceinline__ static void mfma(f32x4& acc, const float* a, const float* b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], acc, 0, 0, 0);
  }
};

// Round x down / up to a multiple of the MFMA k-step of E.
template <typename E> __device__ __forceinline__ int kfloor(int x) { return x / Mma<E>::KS * Mma<E>::KS; }
template <typename E> __device__ __forceinline__ int kceil(int x) {
  return (x + Mma<E>::KS - 1) / Mma<E>::KS * Mma<E>::KS;
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

__device__ __forceinline__ int acc_row(int lane, int j) { return 4 * (lane >> 4) + j; }
__device__ __forceinline__ int acc_col(int lane) { return lane & 15; }

template <typename E> __device__ __forceinline__ E to_e(float x);
template <> __device__ __forceinline__ float to_e<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16_t to_e<bf16_t>(float x) { return f32_to_bf16(x); }
template <typename E> __device__ __forceinline__ float from_e(E x);
template <> __device__ __forceinline__ float from_e<float>(float x) { return x; }
template <> __device__ __forceinline__ float from_e<bf16_t>(bf16_t x) { return bf16_to_f32(x); }

// Row padding of LDS tiles: keeps 16-byte alignment and spreads rows over banks.
template <typename E> struct Pad;
#ifndef PKDA_BF16_PAD
#define PKDA_BF16_PAD 8
#endif
template <> struct Pad<bf16_t> { static constexpr int v = PKDA_BF16_PAD; };
template <> struct Pad<float> { static constexpr int v = 4; };

// Identity value map for the tile loads below.
struct Ident {
  __device__ __forceinline__ float operator()(int, int, float x) const { return x; }
};

// ----------------------------------------------------------------------------
// Vectorised tile loads: 16-byte global accesses, every load of a thread
// issued before its LDS stores.  Rows r >= nvalid read as zero.  NT threads
// (the whole workgroup) share the tile; f(r, c, x) maps each value.
// ----------------------------------------------------------------------------
template <typename T> struct Vec16;
template <> struct Vec16<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void unpack(const uint4& v, float* x) {
    x[0] = __uint_as_float(v.x); x[1] = __uint_as_float(v.y);
    x[2] = __uint_as_float(v.z); x[3] = __uint_as_float(v.w);
  }
  __device__ __forceinline__ static void load(const float* p, float* x) {
    unpack(*reinterpret_cast<const uint4*>(p), x);
  }
};
template <> struct Vec16<bf16_t> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void unpack(const uint4& v, float* x) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static void load(const bf16_t* p, float* x) {
    unpack(*reinterpret_cast<const uint4*>(p), x);
  }
};

// Round-to-nearest-even of two floats into one packed BF16 pair.
__device__ __forceinline__ uint32_t pack_bf16x2_(float a, float b) {
  return static_cast<uint32_t>(f32_to_bf16(a)) | (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
}

// Store n (4 or 8) consecutive floats to LDS as E with one 8- or 16-byte write.
template <int N> __device__ __forceinline__ void store_vec(float* dst, const float* x) {
  if constexpr (N == 4) {
    *reinterpret_cast<float4*>(dst) = make_float4(x[0], x[1], x[2], x[3]);
  } else {
    *reinterpret_cast<float4*>(dst) = make_float4(x[0], x[1], x[2], x[3]);
    *reinterpret_cast<float4*>(dst + 4) = make_float4(x[4], x[5], x[6], x[7]);
  }
}
template <int N> __device__ __forceinline__ void store_vec(bf16_t* dst, const float* x) {
  uint32_t w[N / 2];
#pragma unroll
  for (int i = 0; i < N / 2; ++i)
    w[i] = static_cast<uint32_t>(f32_to_bf16(x[2 * i])) | (static_cast<uint32_t>(f32_to_bf16(x[2 * i + 1])) << 16);
  if constexpr (N == 4) {
    *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
  } else {
    *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// V floats rounded to T (nearest even) and packed into one 16-byte piece.
template <typename T> __device__ __forceinline__ uint4 pack_vec16(const float* x);
template <> __device__ __forceinline__ uint4 pack_vec16<bf16_t>(const float* x) {
  return make_uint4(pack_bf16x2_(x[0], x[1]), pack_bf16x2_(x[2], x[3]), pack_bf16x2_(x[4], x[5]),
                    pack_bf16x2_(x[6], x[7]));
}
template <> __device__ __forceinline__ uint4 pack_vec16<float>(const float* x) {
  return make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3]));
}

template <int NT, int ROWS, int NC, typename T, typename E, typename F>
__device__ __forceinline__ void load_tile(E* lds, int ld, const T* g, int64_t gstride, int nvalid, F f) {
  constexpr int V = Vec16<T>::N;
  constexpr int PER_ROW = NC / V;
  constexpr int TOTAL = ROWS * PER_ROW;
  constexpr int ITER = (TOTAL + NT - 1) / NT;
  static_assert(NC % V == 0, "tile width");
  float x[ITER][V];
#pragma unroll
  for (int i = 0; i < ITER; ++i) {
    const int idx = threadIdx.x + i * NT;
    const int r = idx / PER_ROW;
    const int c = (idx - r * PER_ROW) * V;
    if (idx < TOTAL && r < nvalid) {
      Vec16<T>::load(g + r * gstride + c, x[i]);
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) x[i][j] = 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < ITER; ++i) {
    const int idx = threadIdx.x + i * NT;
    if (TOTAL % NT != 0 && idx >= TOTAL) break;
    const int r = idx / PER_ROW;
    const int c = (idx - r * PER_ROW) * V;
#pragma unroll
    for (int j = 0; j < V; ++j) x[i][j] = f(r, c + j, x[i][j]);
    store_vec<V>(lds + r * ld + c, x[i]);
  }
}

// Coalesced store of rows [0, nvalid) of an LDS tile [ROWS][NC] (element type
// T) to global memory with 16-byte accesses.
template <int NT, int ROWS, int NC, typename T>
__device__ __forceinline__ void store_tile(T* g, int64_t gstride, const T* lds, int ld, int nvalid) {
  constexpr int V = Vec16<T>::N;
  constexpr int PER_ROW = NC / V;
  constexpr int TOTAL = ROWS * PER_ROW;
  for (int idx = threadIdx.x; idx < TOTAL; idx += NT) {
    const int r = idx / PER_ROW;
    const int c = (idx - r * PER_ROW) * V;
    if (r < nvalid) *reinterpret_cast<uint4*>(g + r * gstride + c) = *reinterpret_cast<const uint4*>(lds + r * ld + c);
  }
}

// Rows [0, nvalid) of an FP32 LDS tile [ROWS][NC] (ld a multiple of 4) to
// global memory in T, 16-byte stores (8 BF16 or 4 FP32 per piece).
template <int NT, int ROWS, int NC, typename T>
__device__ __forceinline__ void store_tile_from_f32(T* g, int64_t gstride, const float* lds, int ld, int nvalid) {
  constexpr int V = Vec16<T>::N;
  constexpr int PER_ROW = NC / V;
  constexpr int TOTAL = ROWS * PER_ROW;
  for (int idx = threadIdx.x; idx < TOTAL; idx += NT) {
    const int r = idx / PER_ROW;
    const int c = (idx - r * PER_ROW) * V;
    if (r >= nvalid) continue;
    float x[V];
#pragma unroll
    for (int j = 0; j < V; j += 4) {
      const float4 f = *reinterpret_cast<const float4*>(lds + r * ld + c + j);
      x[j] = f.x; x[j + 1] = f.y; x[j + 2] = f.z; x[j + 3] = f.w;
    }
    uint4 out;
    if constexpr (sizeof(T) == 2) {
      out = make_uint4(pack_bf16x2_(x[0], x[1]), pack_bf16x2_(x[2], x[3]), pack_bf16x2_(x[4], x[5]),
                       pack_bf16x2_(x[6], x[7]));
    } else {
      out = make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3]));
    }
    *reinterpret_cast<uint4*>(g + r * gstride + c) = out;
  }
}

// V consecutive LDS elements as floats.
template <int V> __device__ __forceinline__ void lds_vec(const float* p, float* x) {
#pragma unroll
  for (int j = 0; j < V; ++j) x[j] = p[j];
}
template <int V> __device__ __forceinline__ void lds_vec(const bf16_t* p, float* x) {
#pragma unroll
  for (int j = 0; j < V; ++j) x[j] = bf16_to_f32(p[j]);
}

// Four consecutive LDS elements as floats in one read (8-byte aligned for
// bf16, 16-byte for FP32).
__device__ __forceinline__ void lds4(const float* p, float* x) {
  const float4 w = *reinterpret_cast<const float4*>(p);
  x[0] = w.x;
  x[1] = w.y;
  x[2] = w.z;
  x[3] = w.w;
}
__device__ __forceinline__ void lds4(const bf16_t* p, float* x) {
  const uint2 w = *reinterpret_cast<const uint2*>(p);
  x[0] = __uint_as_float(w.x << 16);
  x[1] = __uint_as_float(w.x & 0xffff0000u);
  x[2] = __uint_as_float(w.y << 16);
  x[3] = __uint_as_float(w.y & 0xffff0000u);
}

// A [ROWS x NC] global tile held in registers as raw 16-byte pieces, so the
// next chunk's operands can be in flight while the current chunk computes.
// Rows r >= nvalid hold zeros.  store() copies the pieces to an LDS tile of
// the same element type.
template <int NT, int ROWS, int NC, typename T>
struct RegTile {
  static constexpr int V = Vec16<T>::N;
  static constexpr int PER_ROW = NC / V;
  static constexpr int TOTAL = ROWS * PER_ROW;
  static constexpr int ITER = (TOTAL + NT - 1) / NT;
  uint4 r[ITER];
  __device__ __forceinline__ void load(const T* g, int64_t gstride, int nvalid) { load_as(threadIdx.x, g, gstride, nvalid); }
  // as thread t of the NT that share the tile (t < NT: with a literal nvalid of
  // ROWS, every row test then folds away and no branch holds a load back)
  __device__ __forceinline__ void load_as(int t, const T* g, int64_t gstride, int nvalid) {
    __builtin_assume(t >= 0 && t < NT);
#pragma unroll
    for (int i = 0; i < ITER; ++i) {
      const int idx = t + i * NT;
      const int row = idx / PER_ROW;
      const int c = (idx - row * PER_ROW) * V;
      r[i] = (idx < TOTAL && row < nvalid) ? *reinterpret_cast<const uint4*>(g + row * gstride + c)
                                           : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  // rows r >= nvalid (nvalid >= 1) repeat row nvalid - 1
  // (every piece is assigned on every path: a conditionally assigned piece
  // keeps the array out of registers)
  __device__ __forceinline__ void load_clamped(const T* g, int64_t gstride, int nvalid) {
    __builtin_assume(threadIdx.x < NT);
#pragma unroll
    for (int i = 0; i < ITER; ++i) {
      const int idx = threadIdx.x + i * NT;
      const int row = min(idx / PER_ROW, nvalid - 1);
      const int c = (idx % PER_ROW) * V;
      r[i] = (TOTAL % NT == 0 || idx < TOTAL) ? *reinterpret_cast<const uint4*>(g + row * gstride + c)
                                              : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  __device__ __forceinline__ void store(T* lds, int ld) const { store_as(threadIdx.x, lds, ld); }
  // every value times a, in the registers (a float tile)
  __device__ __forceinline__ void scale(float a) {
    static_assert(sizeof(T) == 4, "scale() is for float tiles");
#pragma unroll
    for (int i = 0; i < ITER; ++i) {
      r[i].x = __float_as_uint(__uint_as_float(r[i].x) * a);
      r[i].y = __float_as_uint(__uint_as_float(r[i].y) * a);
      r[i].z = __float_as_uint(__uint_as_float(r[i].z) * a);
      r[i].w = __float_as_uint(__uint_as_float(r[i].w) * a);
    }
  }
  __device__ __forceinline__ void store_as(int t, T* lds, int ld) const {
    __builtin_assume(t >= 0 && t < NT);
#pragma unroll
    for (int i = 0; i < ITER; ++i) {
      const int idx = t + i * NT;
      if (TOTAL % NT != 0 && idx >= TOTAL) break;
      const int row = idx / PER_ROW;
      const int c = (idx - row * PER_ROW) * V;
      *reinterpret_cast<uint4*>(lds + row * ld + c) = r[i];
    }
  }
  // store with f(r, c, x) applied to every value (rounded back to T)
  template <typename F>
  __device__ __forceinline__ void store(T* lds, int ld, F f) const {
#pragma unroll
    for (int i = 0; i < ITER; ++i) {
      const int idx = threadIdx.x + i * NT;
      if (TOTAL % NT != 0 && idx >= TOTAL) break;
      const int row = idx / PER_ROW;
      const int c = (idx - row * PER_ROW) * V;
      float x[V];
      Vec16<T>::unpack(r[i], x);
#pragma unroll
      for (int j = 0; j < V; ++j) x[j] = f(row, c + j, x[j]);
      store_vec<V>(lds + row * ld + c, x);
    }
  }
};

// A tile-major [D x D] state checkpoint (see tile_offset) held in registers:
// NT threads read it as consecutive 16-byte pieces (fully coalesced); pos()
// gives the (row, first column) of piece i of this thread in the [D x D]
// matrix, and store() writes the pieces to a row-major LDS tile.
template <int NT, int D, typename T>
struct TiledTile {
  static constexpr int V = Vec16<T>::N;
  static constexpr int TOTAL = D * D / V;
  static constexpr int ITER = (TOTAL + NT - 1) / NT;
  static constexpr int PER_TILE = 256 / V;
  static_assert(TOTAL % NT == 0, "pieces split evenly over the threads");
  uint4 r[ITER];
  __device__ __forceinline__ void load(const T* g) {
#pragma unroll
    for (int i = 0; i < ITER; ++i) r[i] = reinterpret_cast<const uint4*>(g)[threadIdx.x + i * NT];
  }
  __device__ __forceinline__ static void pos(int i, int& row, int& col) {
    const int k = threadIdx.x + i * NT;
    const int tile = k / PER_TILE, e = (k % PER_TILE) * V;
    row = (tile / (D / 16)) * 16 + e / 16;
    col = (tile % (D / 16)) * 16 + e % 16;
  }
  __device__ __forceinline__ void store(T* lds, int ld) const {
#pragma unroll
    for (int i = 0; i < ITER; ++i) {
      int row, col;
      pos(i, row, col);
      *reinterpret_cast<uint4*>(lds + row * ld + col) = r[i];
    }
  }
};

// Row-scaled variant helper: f(r, c, x) = s[r] * x.
struct RowScale {
  const float* s;
  __device__ __forceinline__ float operator()(int r, int, float x) const { return s[r] * x; }
};


// Store an accumulator tile (origin m0, n0) to global with row mask.  The
// four lanes of a quad (16q + 4c + t, t = 0..3) hold columns 4c..4c+3 of rows
// 4q..4q+3; two DPP exchanges inside the quad transpose that 4 x 4 block so
// lane t holds row 4q + t, columns 4c..4c+3, written with one 8-byte (bf16)
// or 16-byte (FP32) store instead of four scattered element stores.
// Requires g + n0 and gstride to keep 4-element alignment.
// Round-to-nearest-even of two floats into one packed pair (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2_t v;
  v[0] = static_cast<__bf16>(a);
  v[1] = static_cast<__bf16>(b);
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint32_t quad_swap(uint32_t x, int ctrl_is_pair) {
  return ctrl_is_pair ? __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true)   // lane ^ 1
                      : __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true);  // lane ^ 2
}

// 4 x 4 transpose of 16-bit elements in a quad: in, lane t holds column t as
// (v0 = rows 0,1; v1 = rows 2,3); out, row t as (v0 = cols 0,1; v1 = cols 2,3).
// Branch-free: the lane-dependent halves are picked by a byte permute
// (v_perm_b32 with a per-lane selector) and bit masks, so no divergent
// if/else splits the caller's code around every store.
__device__ __forceinline__ void quad_transpose_b16(uint32_t& v0, uint32_t& v1, int lane) {
  // v_perm_b32(a, b, sel): byte i of the result is byte sel_i of {b (0..3), a (4..7)}
  //   even lane: own low half, then the partner's low half   -> bytes 0 1 4 5
  //   odd lane:  the partner's high half, then own high half -> bytes 6 7 2 3
  const uint32_t sel = (lane & 1) ? 0x03020706u : 0x05040100u;
  const uint32_t hm = (lane & 2) ? 0xffffffffu : 0u;
  const uint32_t p0 = quad_swap(v0, 1), p1 = quad_swap(v1, 1);
  v0 = __builtin_amdgcn_perm(p0, v0, sel);
  v1 = __builtin_amdgcn_perm(p1, v1, sel);
  const uint32_t s = quad_swap((v0 & hm) | (v1 & ~hm), 0);
  v0 = (s & hm) | (v0 & ~hm);
  v1 = (v1 & hm) | (s & ~hm);
}

// 4 x 4 transpose of 32-bit elements in a quad (a[j] = row j of column t in,
// column j of row t out).
__device__ __forceinline__ void quad_transpose_b32(float* a, int lane) {
  // every lane-dependent choice is a bit-mask select (no divergent branches)
  const uint32_t om = (lane & 1) ? 0xffffffffu : 0u, hm = (lane & 2) ? 0xffffffffu : 0u;
  auto sel = [](uint32_t m, uint32_t x, uint32_t y) { return (x & m) | (y & ~m); };  // m ? x : y
  uint32_t u[4] = {__float_as_uint(a[0]), __float_as_uint(a[1]), __float_as_uint(a[2]), __float_as_uint(a[3])};
  const uint32_t r0 = quad_swap(sel(om, u[0], u[1]), 1);
  const uint32_t r1 = quad_swap(sel(om, u[2], u[3]), 1);
  u[0] = sel(om, r0, u[0]);
  u[1] = sel(om, u[1], r0);
  u[2] = sel(om, r1, u[2]);
  u[3] = sel(om, u[3], r1);
  const uint32_t s0 = quad_swap(sel(hm, u[0], u[2]), 0);
  const uint32_t s1 = quad_swap(sel(hm, u[1], u[3]), 0);
  u[0] = sel(hm, s0, u[0]);
  u[1] = sel(hm, s1, u[1]);
  u[2] = sel(hm, u[2], s0);
  u[3] = sel(hm, u[3], s1);
#pragma unroll
  for (int j = 0; j < 4; ++j) a[j] = __uint_as_float(u[j]);
}

// Row and first column of the lane's piece after the transpose.
__device__ __forceinline__ int quad_row(int lane) { return 4 * (lane >> 4) + (lane & 3); }
__device__ __forceinline__ int quad_col(int lane) { return 4 * ((lane >> 2) & 3); }

// Store packed bf16 pairs of an accumulator-layout tile (v0 = rows 4q, 4q+1;
// v1 = rows 4q+2, 4q+3 of column lane & 15) by rows.  FULL: every row is
// valid (a whole chunk), so no row test splits the caller's code into
// branches.
template <bool FULL = false>
__device__ __forceinline__ void store_packed_rows(bf16_t* g, int64_t gstride, uint32_t v0, uint32_t v1, int m0, int n0,
                                                  int nvalid, int lane) {
  quad_transpose_b16(v0, v1, lane);
  const int r = m0 + quad_row(lane);
  if (FULL || r < nvalid) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<u32x2*>(g + r * gstride + n0 + quad_col(lane)) = u32x2{v0, v1};
  }
}


// Tile-major [D x D] state checkpoints: 16 x 16 tiles, each row-major and
// contiguous (256 elements), tile (rt, ct) at element (rt * (D / 16) + ct) * 256.
// One accumulator tile is one contiguous 512-byte write.
__device__ __forceinline__ void store_packed_tile(bf16_t* tile, uint32_t v0, uint32_t v1, int lane) {
  quad_transpose_b16(v0, v1, lane);
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  *reinterpret_cast<u32x2*>(tile + quad_row(lane) * 16 + quad_col(lane)) = u32x2{v0, v1};
}
// The same with a non-temporal hint: for the chunk-state checkpoints h and
// dh, which are read back only by a later kernel.
__device__ __forceinline__ void store_packed_tile_nt(bf16_t* tile, uint32_t v0, uint32_t v1, int lane) {
  quad_transpose_b16(v0, v1, lane);
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  __builtin_nontemporal_store(u32x2{v0, v1}, reinterpret_cast<u32x2*>(tile + quad_row(lane) * 16 + quad_col(lane)));
}
// A 16-byte piece of a streamed output (the reverse state passes' dU / dv
// rows, read only by a later kernel) with a non-temporal hint.
__device__ __forceinline__ void store16_nt(void* dst, const uint4 x) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(u32x4{x.x, x.y, x.z, x.w}, reinterpret_cast<u32x4*>(dst));
}
__device__ __forceinline__ void store_acc_tile(bf16_t* tile, const f32x4& acc, int lane) {
  store_packed_tile(tile, pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]), lane);
}
__device__ __forceinline__ void store_acc_tile(float* tile, const f32x4& acc, int lane) {
  float a[4] = {acc[0], acc[1], acc[2], acc[3]};
  quad_transpose_b32(a, lane);
  *reinterpret_cast<float4*>(tile + quad_row(lane) * 16 + quad_col(lane)) = make_float4(a[0], a[1], a[2], a[3]);
}
__device__ __forceinline__ int64_t tile_offset(int D, int rt, int ct) { return ((int64_t)rt * (D / 16) + ct) * 256; }

template <typename T, bool FULL = false>
struct AccStore;
template <bool FULL>
struct AccStore<bf16_t, FULL> {
  __device__ __forceinline__ static void run(bf16_t* g, int64_t gstride, const f32x4& acc, int m0, int n0, int nvalid,
                                             int lane) {
    bf16x2_t a, b;
    a[0] = static_cast<__bf16>(acc[0]);
    a[1] = static_cast<__bf16>(acc[1]);
    b[0] = static_cast<__bf16>(acc[2]);
    b[1] = static_cast<__bf16>(acc[3]);
    store_packed_rows<FULL>(g, gstride, __builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b), m0, n0,
                            nvalid, lane);
  }
};
template <bool FULL>
struct AccStore<float, FULL> {
  __device__ __forceinline__ static void run(float* g, int64_t gstride, const f32x4& acc, int m0, int n0, int nvalid,
                                             int lane) {
    float a[4] = {acc[0], acc[1], acc[2], acc[3]};
    quad_transpose_b32(a, lane);
    const int r = m0 + quad_row(lane);
    if (FULL || r < nvalid)
      *reinterpret_cast<float4*>(g + r * gstride + n0 + quad_col(lane)) = make_float4(a[0], a[1], a[2], a[3]);
  }
};
// Store an accumulator tile by rows, rows >= nvalid masked (FULL: none are).
template <typename T, bool FULL = false>
__device__ __forceinline__ void store_acc_global(T* g, int64_t gstride, const f32x4& acc, int m0, int n0, int nvalid,
                                                 int lane) {
  AccStore<T, FULL>::run(g, gstride, acc, m0, n0, nvalid, lane);
}

// ----------------------------------------------------------------------------
// Lower-triangular chunk matrices stored packed (T and Aqk of the BF16 per-head
// path with kw = k): per (chunk, head) the ten 16 x 16 blocks on and below the
// diagonal, block by block in lower_block order, each row-major -- 10 x 256
// BF16, 5 KB instead of 8 KB.  Rows past a chunk's end hold zeros; the six
// blocks above the diagonal are not stored (their LDS copies are zeroed once).
// ----------------------------------------------------------------------------
constexpr int kTriBlocks = 10;
constexpr int kTriElems = kTriBlocks * 256;

// Row and column block of lower block i (0..9) of a 64 x 64 chunk matrix,
// row-block-major, and of upper block u (0..5).
__device__ __forceinline__ void lower_block(int i, int& tb, int& sb) {
  tb = i < 1 ? 0 : i < 3 ? 1 : i < 6 ? 2 : 3;
  sb = i - tb * (tb + 1) / 2;
}
__device__ __forceinline__ void upper_block(int u, int& tb, int& sb) {
  tb = u < 3 ? 0 : u < 5 ? 1 : 2;
  sb = u < 3 ? u + 1 : u < 5 ? u - 1 : 3;
}

// A packed lower-triangular tile in registers, 16-byte pieces shared by NT
// threads (piece p: block p / 32, row (p % 32) / 2, columns 8 (p % 2) ..).
template <int NT>
struct TriRegTile {
  static constexpr int TOTAL = kTriBlocks * 32;
  static constexpr int ITER = (TOTAL + NT - 1) / NT;
  uint4 r[ITER];
  __device__ __forceinline__ void load_as(int t, const bf16_t* g) {
    __builtin_assume(t >= 0 && t < NT);
#pragma unroll
    for (int i = 0; i < ITER; ++i) {
      const int idx = t + i * NT;
      r[i] = (TOTAL % NT == 0 || idx < TOTAL) ? *reinterpret_cast<const uint4*>(g + 8 * idx) : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  // into a [64][ld] LDS tile (its upper blocks are left as they are)
  __device__ __forceinline__ void store_as(int t, bf16_t* lds, int ld) const {
    __builtin_assume(t >= 0 && t < NT);
#pragma unroll
    for (int i = 0; i < ITER; ++i) {
      const int idx = t + i * NT;
      if (TOTAL % NT != 0 && idx >= TOTAL) break;
      int tb, sb;
      lower_block(idx >> 5, tb, sb);
      const int row = (idx & 31) >> 1, half = idx & 1;
      *reinterpret_cast<uint4*>(lds + (16 * tb + row) * ld + 16 * sb + 8 * half) = r[i];
    }
  }
};

// Zeros into the six blocks above the diagonal of a [64][ld] BF16 LDS tile,
// pieces t, t + NT, ... of the 192.
template <int NT>
__device__ __forceinline__ void zero_upper_blocks(int t, bf16_t* lds, int ld) {
  for (int idx = t; idx < 6 * 32; idx += NT) {
    int tb, sb;
    upper_block(idx >> 5, tb, sb);
    const int row = (idx & 31) >> 1, half = idx & 1;
    *reinterpret_cast<uint4*>(lds + (16 * tb + row) * ld + 16 * sb + 8 * half) = make_uint4(0u, 0u, 0u, 0u);
  }
}

// The ten lower blocks of an FP32 [64][ldf] LDS tile to packed BF16 in
// global memory, rows >= nvalid as zeros (NT threads, one 16-byte piece each).
template <int NT>
__device__ __forceinline__ void store_tri_from_f32(bf16_t* g, const float* lds, int ldf, int nvalid) {
  for (int idx = threadIdx.x; idx < kTriBlocks * 32; idx += NT) {
    int tb, sb;
    lower_block(idx >> 5, tb, sb);
    const int r = 16 * tb + ((idx & 31) >> 1), c = 16 * sb + 8 * (idx & 1);
    const float4 a = *reinterpret_cast<const float4*>(lds + r * ldf + c);
    const float4 b = *reinterpret_cast<const float4*>(lds + r * ldf + c + 4);
    const uint4 w = r < nvalid ? make_uint4(pack_bf16x2_(a.x, a.y), pack_bf16x2_(a.z, a.w), pack_bf16x2_(b.x, b.y),
                                            pack_bf16x2_(b.z, b.w))
                               : make_uint4(0u, 0u, 0u, 0u);
    *reinterpret_cast<uint4*>(g + 8 * idx) = w;
  }
}

// Output tiles of a loop that produces one 16-column tile per pass with long
// work in between.  A BF16 tile row is a 32-byte piece; stored alone, long
// before the row's next piece, it reaches memory as a partial line (the
// counters show ~1.7x the bytes).  put(.., pos) keeps the tiles of passes
// pos = 0 .. NG - 2 in registers (packed and quad-transposed, shifted along so
// every register stays fixed in a loop that is not unrolled) and stores the
// NG tiles together at pos = NG - 1, so each row gets NG adjacent pieces at
// once (tile pos at n0 - 16 (NG - 1 - pos)).  FP32 rows are 64-byte pieces
// already and are stored as they come.
template <typename T, int NG>
struct TileGroupStore {
  __device__ __forceinline__ void put(T* g, int64_t gstride, const f32x4& acc, int m0, int n0, int nvalid, int lane,
                                      int pos) {
    store_acc_global<T>(g, gstride, acc, m0, n0, nvalid, lane);
  }
};
template <int NG>
struct TileGroupStore<bf16_t, NG> {
  static_assert(NG >= 2 && NG <= 4, "2 to 4 tiles per group");
  uint32_t p0[NG - 1], p1[NG - 1];  // [i]: the tile NG - 1 - i passes back
  __device__ __forceinline__ void put(bf16_t* g, int64_t gstride, const f32x4& acc, int m0, int n0, int nvalid,
                                      int lane, int pos) {
    bf16x2_t a, b;  // the same rounding as store_acc_global
    a[0] = static_cast<__bf16>(acc[0]);
    a[1] = static_cast<__bf16>(acc[1]);
    b[0] = static_cast<__bf16>(acc[2]);
    b[1] = static_cast<__bf16>(acc[3]);
    uint32_t v0 = __builtin_bit_cast(uint32_t, a), v1 = __builtin_bit_cast(uint32_t, b);
    quad_transpose_b16(v0, v1, lane);
    if (pos == NG - 1) {  // uniform: the pass index
      const int r = m0 + quad_row(lane);
      if (r < nvalid) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        bf16_t* row = g + r * gstride + n0 + quad_col(lane);
#pragma unroll
        for (int i = NG - 2; i >= 0; --i) *reinterpret_cast<u32x2*>(row - 16 * (i + 1)) = u32x2{p0[i], p1[i]};
        *reinterpret_cast<u32x2*>(row) = u32x2{v0, v1};
      }
    } else {
#pragma unroll
      for (int i = NG - 2; i > 0; --i) {
        p0[i] = p0[i - 1];
        p1[i] = p1[i - 1];
      }
      p0[0] = v0;
      p1[0] = v1;
    }
  }
};

template <typename E>
__device__ __forceinline__ void store_acc_lds(E* lds, int ld, const f32x4& acc, int m0, int n0, int lane) {
#pragma unroll
  for (int j = 0; j < 4; ++j) lds[(m0 + acc_row(lane, j)) * ld + n0 + acc_col(lane)] = to_e<E>(acc[j]);
}


// out[i] = sum over p of part[p * n + i], p in [0, count): one 256-thread
// workgroup per output element (grid = n); thread t adds the partials
// t, t + 256, ... in order, then a fixed halving tree combines the threads.
// Deterministic, and every load of a thread is independent of its sum, so the
// partials stream in rather than paying one memory latency each.
namespace {  // one copy per translation unit
__global__ __launch_bounds__(256) void sum_partials_tree_kernel(const float* part, int count, int n, float* out) {
  __shared__ float s[256];
  const int i = blockIdx.x;
  float acc = 0.f;
  for (int q = threadIdx.x; q < count; q += 256) acc += part[(int64_t)q * n + i];
  s[threadIdx.x] = acc;
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if (threadIdx.x < off) s[threadIdx.x] += s[threadIdx.x + off];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[i] = s[0];
}
}  // namespace


// ----------------------------------------------------------------------------
// Register-resident bf16 MFMA operands.  An accumulator tile X (lane 16q + i
// holds X[4q + j][i]) serves as the B operand of a 16x16x32 step over X's rows
// without leaving registers when the step takes its 32 k indices in the order
//   lane group q: rows 4q..4q+3 of tile 2kk, then rows 4q..4q+3 of tile 2kk+1,
// i.e. k = 32kk + {4q..4q+3} and 32kk + 16 + {4q..4q+3}.  The A operand of
// the same step is read from LDS in that order.  The k order inside one MFMA
// does not change the product.
// ----------------------------------------------------------------------------

// B operand of step kk from accumulator tiles a (rows 32kk..) and b (rows 32kk + 16..).
__device__ __forceinline__ s16x8_t pack_acc_pair(const f32x4& a, const f32x4& b) {
  const uint4 w = make_uint4(pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(b[0], b[1]),
                             pack_bf16x2(b[2], b[3]));
  return __builtin_bit_cast(s16x8_t, w);
}

// The same with every element scaled: sa[j] for tile a, sb[j] for tile b.
__device__ __forceinline__ s16x8_t pack_acc_pair_scaled(const f32x4& a, const float* sa, const f32x4& b,
                                                        const float* sb) {
  const uint4 w = make_uint4(pack_bf16x2(a[0] * sa[0], a[1] * sa[1]), pack_bf16x2(a[2] * sa[2], a[3] * sa[3]),
                             pack_bf16x2(b[0] * sb[0], b[1] * sb[1]), pack_bf16x2(b[2] * sb[2], b[3] * sb[3]));
  return __builtin_bit_cast(s16x8_t, w);
}

// A operand in that k order from a row-major LDS tile (element (m, k) at
// A[m * lda + k], A offset to row m0): two 8-byte reads per lane.
__device__ __forceinline__ s16x8_t lds_a_perm(const bf16_t* A, int lda, int k0, int lane) {
  const bf16_t* p = A + (lane & 15) * lda + k0 + 4 * (lane >> 4);
  const uint2 lo = *reinterpret_cast<const uint2*>(p);
  const uint2 hi = *reinterpret_cast<const uint2*>(p + 16);
  return __builtin_bit_cast(s16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
}

// A operand in that k order from a k-major LDS tile (element (m, k) at
// A[k * lda + m], A offset to column m0), and equally the B operand of a
// k-major tile (element (k, n) at B[k * ldb + n]): two transposing reads.
__device__ __forceinline__ s16x8_t lds_kmajor_perm(const bf16_t* A, int lda, int k0, int lane) {
  const int i = lane & 15, q = lane >> 4;
  const bf16_t* src = A + (k0 + 4 * q + (i >> 2)) * lda + 4 * (i & 3);
  const bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(src));
  const bf16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(src + 16 * lda));
  const s16x4_t l = __builtin_bit_cast(s16x4_t, lo), h = __builtin_bit_cast(s16x4_t, hi);
  return s16x8_t{l[0], l[1], l[2], l[3], h[0], h[1], h[2], h[3]};
}

// Every element of an operand in that k order scaled by the factor of its k
// index (sf: 8 factors, lane's order), rounded back to bf16.
__device__ __forceinline__ s16x8_t scale_frag(const s16x8_t& x, const float* sf) {
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    w[e] = pack_bf16x2(bf16_to_f32(static_cast<bf16_t>(x[2 * e])) * sf[2 * e],
                       bf16_to_f32(static_cast<bf16_t>(x[2 * e + 1])) * sf[2 * e + 1]);
  return __builtin_bit_cast(s16x8_t, make_uint4(w[0], w[1], w[2], w[3]));
}

__device__ __forceinline__ void mfma_bf16(f32x4& acc, const s16x8_t& a, const s16x8_t& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), acc,
                                                0, 0, 0);
}

}  // namespace pkda
