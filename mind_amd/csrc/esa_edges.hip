// Edge-token gather, CSR construction and deterministic segmented sums on
// gfx950.  All three are HBM-bound byte/integer work: 16-byte vector
// accesses, one wave per output row (segment sums) or one lane per 16-byte
// chunk (gather), nontemporal stores for the streamed gather output.
//
// Gather semantics: h_e = [x[src_e] || x[dst_e]] (core/pretraining_model.py:153-155,
// esa/models.py:307-309).  Segment sum semantics: out_n = sum over the CSR
// segment of n in ascending position (GET/utils/sorted_segment_ops.py:40-41),
// fp32 accumulation, rounded once.
#include <algorithm>

#include "esa_common.h"
#include "esa_csr.h"
#include "esa_profile.h"
#include "../../include/esa_hip.h"

namespace {

// ------------------------------------------------------------------ gather

// One lane moves one 16-byte chunk; a block covers `epb` consecutive edges.
// Rows whose node index is outside [0, num_nodes) are written as zeros.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void edge_gather_kernel(const u32x4* __restrict__ x,
                                                          const int* __restrict__ src,
                                                          const int* __restrict__ dst, long num_edges,
                                                          int num_nodes, int chunks, int epb,
                                                          u32x4* __restrict__ out) {
  const long e0 = (long)blockIdx.x * epb;
  const long rem = num_edges - e0;
  const int ne = rem < epb ? (int)rem : epb;
  const int per_edge = 2 * chunks;
  const int items = ne * per_edge;
#pragma unroll 4
  for (int it = threadIdx.x; it < items; it += blockDim.x) {
    const int el = it / per_edge;
    const int c = it - el * per_edge;
    const long e = e0 + el;
    const bool first = c < chunks;
    const int node = first ? src[e] : dst[e];
    const int cc = first ? c : c - chunks;
    u32x4 v = {0u, 0u, 0u, 0u};
    if ((unsigned)node < (unsigned)num_nodes) v = x[(size_t)node * chunks + cc];
    __builtin_nontemporal_store(v, &out[(size_t)e * per_edge + c]);
  }
}

// Row mode (rows of 2 * chunks 16-byte pieces, chunks a multiple of 32): a
// wave writes whole output rows, P pieces per lane per row, U = 16 / P edges
// per step.  The step's src / dst ids arrive with one vector load (lanes
// 0..U-1 and 32..32+U-1) and are broadcast with readlane, so all U * P gather
// loads are in flight before the first store.  Loads go through a buffer
// resource over x: a node id outside [0, num_nodes) reads zeros.  Each XCD
// (hardware block b runs on XCD b % 8) walks one contiguous range of edges,
// so the node rows an edge range touches stay in that XCD's L2.
#ifndef ESA_GATHER_LOADS
#define ESA_GATHER_LOADS 32   // 16-byte loads in flight per lane per step
#endif
#ifndef ESA_GATHER_STEPS
#define ESA_GATHER_STEPS 1    // steps per wave (a wave moves ESA_GATHER_LOADS / P edges per step)
#endif

template <int P>
__global__ __launch_bounds__(256) void edge_gather_rows_kernel(const void* x, uint32_t x_bytes,
                                                               const int* __restrict__ src,
                                                               const int* __restrict__ dst, long num_edges,
                                                               int num_nodes, int chunks, int edges_per_wave,
                                                               int blocks_per_xcd, u32x4* __restrict__ out) {
  constexpr int U = ESA_GATHER_LOADS / P;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, x_bytes);
  const int lane = threadIdx.x & 63;
  const int lb = (int)(blockIdx.x & 7) * blocks_per_xcd + (int)(blockIdx.x >> 3);
  const long wave = (long)lb * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const long e_beg = wave * edges_per_wave;
  const long e_end = min(e_beg + (long)edges_per_wave, num_edges);
  const uint32_t row_bytes = (uint32_t)chunks * 16u;
  const int per_row = 2 * chunks;
  for (long e0 = e_beg; e0 < e_end; e0 += U) {
    const long ei = min(e0 + (lane & 31), num_edges - 1);
    const int idx = lane < 32 ? src[ei] : dst[ei];
    u32x4 v[U][P];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = __builtin_amdgcn_readlane(idx, u), d = __builtin_amdgcn_readlane(idx, 32 + u);
#pragma unroll
      for (int j = 0; j < P; ++j) {
        const int p = lane + 64 * j;
        const bool first = p < chunks;
        const int node = first ? s : d;
        const uint32_t c = (uint32_t)(first ? p : p - chunks);
        const uint32_t off = (unsigned)node < (unsigned)num_nodes ? (uint32_t)node * row_bytes + 16u * c : 0xFFFFFFF0u;
        v[u][j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (e0 + u < e_end) {
#pragma unroll
        for (int j = 0; j < P; ++j)
          __builtin_nontemporal_store(v[u][j], &out[(size_t)(e0 + u) * per_row + lane + 64 * j]);
      }
    }
  }
}

// Element-wise fallback for rows that are not a multiple of 16 bytes.
template <typename T>
__global__ void edge_gather_scalar_kernel(const T* __restrict__ x, const int* __restrict__ src,
                                          const int* __restrict__ dst, long num_edges, int num_nodes,
                                          int features, T* __restrict__ out) {
  const long n = num_edges * 2 * features;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const long e = i / (2 * features);
    const int c = (int)(i - e * 2 * features);
    const bool first = c < features;
    const int node = first ? src[e] : dst[e];
    const int f = first ? c : c - features;
    out[i] = (unsigned)node < (unsigned)num_nodes ? x[(size_t)node * features + f] : (T)0.f;
  }
}

// ------------------------------------------------------------------ gather-add
// out_e = a[src_e] + b[dst_e] + bias: the edge-token Linear of
// core/pretraining_model.py:153-198 (Linear over [x_src || x_dst],
// esa/mlp_utils.py:28-32) with its weight split by input half, so a = x W_s^T
// and b = x W_d^T are node-level GEMM outputs (rows lda / ldb elements apart)
// and the 2F-wide token matrix is never formed.  Sums in fp32 in the order
// (a + b) + bias, rounded once to the output type.  A node id outside
// [0, num_nodes) contributes zeros.
//
// A lane owns one 16-byte column chunk (lanes per edge L = min(C, 64), C =
// chunks per row; P = C / L chunks per lane), a wave step covers U * 64 / L
// edges with all their loads in flight before the adds, and each wave walks
// a contiguous edge range (XCD-contiguous, as the row gather).

template <typename T>
DEVI float4 chunk_f32(u32x4 v, int k);   // elements 4k..4k+3 of a 16-byte bf16 chunk as fp32
template <>
DEVI float4 chunk_f32<bf16>(u32x4 v, int k) {
  const uint32_t lo = k == 0 ? v.x : v.z, hi = k == 0 ? v.y : v.w;
  return make_float4(__uint_as_float(lo << 16), __uint_as_float(lo & 0xFFFF0000u), __uint_as_float(hi << 16),
                     __uint_as_float(hi & 0xFFFF0000u));
}

template <typename T>
DEVI u32x4 add3_chunk(u32x4 x, u32x4 y, u32x4 z) {
  if constexpr (sizeof(T) == 4) {
    return u32x4{__float_as_uint((__uint_as_float(x.x) + __uint_as_float(y.x)) + __uint_as_float(z.x)),
                 __float_as_uint((__uint_as_float(x.y) + __uint_as_float(y.y)) + __uint_as_float(z.y)),
                 __float_as_uint((__uint_as_float(x.z) + __uint_as_float(y.z)) + __uint_as_float(z.z)),
                 __float_as_uint((__uint_as_float(x.w) + __uint_as_float(y.w)) + __uint_as_float(z.w))};
  } else {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const float4 a = chunk_f32<bf16>(x, k), b = chunk_f32<bf16>(y, k), c = chunk_f32<bf16>(z, k);
      const bf16 r0 = (bf16)((a.x + b.x) + c.x), r1 = (bf16)((a.y + b.y) + c.y);
      const bf16 r2 = (bf16)((a.z + b.z) + c.z), r3 = (bf16)((a.w + b.w) + c.w);
      w[2 * k] = (uint32_t)__builtin_bit_cast(uint16_t, r0) | ((uint32_t)__builtin_bit_cast(uint16_t, r1) << 16);
      w[2 * k + 1] = (uint32_t)__builtin_bit_cast(uint16_t, r2) | ((uint32_t)__builtin_bit_cast(uint16_t, r3) << 16);
    }
    return u32x4{w[0], w[1], w[2], w[3]};
  }
}

template <typename T, int P>
__global__ __launch_bounds__(256) void edge_gather_add_kernel(const u32x4* __restrict__ a, long lda16,
                                                              const u32x4* __restrict__ b, long ldb16,
                                                              const u32x4* __restrict__ bias,
                                                              const int* __restrict__ src,
                                                              const int* __restrict__ dst, long num_edges,
                                                              int num_nodes, int lanes_per_edge, long steps_per_wave,
                                                              int blocks_per_xcd, u32x4* __restrict__ out) {
  constexpr int U = 8 / P;   // edges per lane per step (8 chunk pairs in flight)
  const int lane = threadIdx.x & 63;
  const int lb = (int)(blockIdx.x & 7) * blocks_per_xcd + (int)(blockIdx.x >> 3);
  const long wave = (long)lb * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int L = lanes_per_edge, R = 64 / L;        // edges per wave row
  const int j = lane / L, c = lane - j * L;        // edge slot, chunk
  const int C = L * P;                             // chunks per output row
  u32x4 bz[P];
#pragma unroll
  for (int p = 0; p < P; ++p) bz[p] = bias ? bias[c + L * p] : u32x4{0u, 0u, 0u, 0u};
  const long per_step = (long)U * R;
  const long e_beg = wave * steps_per_wave * per_step;
  const long e_end = min(e_beg + steps_per_wave * per_step, num_edges);
  for (long e0 = e_beg; e0 < e_end; e0 += per_step) {
    u32x4 va[U][P], vb[U][P];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long e = e0 + (long)u * R + j;
      const long ec = min(e, num_edges - 1);
      const int s = src[ec], d = dst[ec];
      const bool sok = (unsigned)s < (unsigned)num_nodes, dok = (unsigned)d < (unsigned)num_nodes;
#pragma unroll
      for (int p = 0; p < P; ++p) {
        va[u][p] = sok ? a[(size_t)s * lda16 + c + L * p] : u32x4{0u, 0u, 0u, 0u};
        vb[u][p] = dok ? b[(size_t)d * ldb16 + c + L * p] : u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long e = e0 + (long)u * R + j;
      if (e < e_end) {
#pragma unroll
        for (int p = 0; p < P; ++p)
          __builtin_nontemporal_store(add3_chunk<T>(va[u][p], vb[u][p], bz[p]), &out[(size_t)e * C + c + L * p]);
      }
    }
  }
}

// Whole-row variant for rows of a multiple of 64 chunks (one wave per output
// row, P chunks per lane): a step's U = 16 / P edge ids arrive with one
// vector load (lanes 0..U-1 src, 32..32+U-1 dst) and are broadcast with
// readlane, so the row bases are wave-uniform and 16 chunk loads per lane
// are in flight before the adds.
#ifndef ESA_GADD_ROWS
#define ESA_GADD_ROWS 1
#endif
template <typename T, int P>
__global__ __launch_bounds__(256) void edge_gather_add_rows_kernel(const char* __restrict__ a, long lda_bytes,
                                                                   const char* __restrict__ b, long ldb_bytes,
                                                                   const u32x4* __restrict__ bias,
                                                                   const int* __restrict__ src,
                                                                   const int* __restrict__ dst, long num_edges,
                                                                   int num_nodes, int edges_per_wave,
                                                                   int blocks_per_xcd, u32x4* __restrict__ out) {
  constexpr int U = 8 / P;
  constexpr int C = 64 * P;
  const int lane = threadIdx.x & 63;
  const int lb = (int)(blockIdx.x & 7) * blocks_per_xcd + (int)(blockIdx.x >> 3);
  const long wave = (long)lb * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const long e_beg = wave * edges_per_wave;
  const long e_end = min(e_beg + (long)edges_per_wave, num_edges);
  u32x4 bz[P];
#pragma unroll
  for (int p = 0; p < P; ++p) bz[p] = bias ? bias[lane + 64 * p] : u32x4{0u, 0u, 0u, 0u};
  const u32x4 zero = {0u, 0u, 0u, 0u};
  for (long e0 = e_beg; e0 < e_end; e0 += U) {
    const long ei = min(e0 + (lane & 31), num_edges - 1);
    const int idx = lane < 32 ? src[ei] : dst[ei];
    u32x4 va[U][P], vb[U][P];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = __builtin_amdgcn_readlane(idx, u), d = __builtin_amdgcn_readlane(idx, 32 + u);
      const u32x4* ra = reinterpret_cast<const u32x4*>(a + (size_t)(unsigned)s * lda_bytes);
      const u32x4* rb = reinterpret_cast<const u32x4*>(b + (size_t)(unsigned)d * ldb_bytes);
      const bool sok = (unsigned)s < (unsigned)num_nodes, dok = (unsigned)d < (unsigned)num_nodes;
#pragma unroll
      for (int p = 0; p < P; ++p) {
        va[u][p] = sok ? ra[lane + 64 * p] : zero;
        vb[u][p] = dok ? rb[lane + 64 * p] : zero;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (e0 + u < e_end) {
#pragma unroll
        for (int p = 0; p < P; ++p)
          __builtin_nontemporal_store(add3_chunk<T>(va[u][p], vb[u][p], bz[p]), &out[(size_t)(e0 + u) * C + lane + 64 * p]);
      }
    }
  }
}

// Element-wise fallback for rows or strides that are not 16-byte multiples.
template <typename T>
__global__ void edge_gather_add_scalar_kernel(const T* __restrict__ a, long lda, const T* __restrict__ b, long ldb,
                                              const T* __restrict__ bias, const int* __restrict__ src,
                                              const int* __restrict__ dst, long num_edges, int num_nodes,
                                              int features, T* __restrict__ out) {
  const long n = num_edges * features;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const long e = i / features;
    const int f = (int)(i - e * features);
    const int s = src[e], d = dst[e];
    const float x = (unsigned)s < (unsigned)num_nodes ? (float)a[(size_t)s * lda + f] : 0.f;
    const float y = (unsigned)d < (unsigned)num_nodes ? (float)b[(size_t)d * ldb + f] : 0.f;
    const float z = bias ? (float)bias[f] : 0.f;
    out[i] = (T)((x + y) + z);
  }
}

// ------------------------------------------------------------------ CSR

// perm by a stable LSD radix sort of (key, edge id) over 8-bit digits, so
// every edge's position follows from counts alone (no atomic ordering, no
// per-segment sort): per pass, each block counts the digits of its tile of
// kSortTile consecutive edges (hist, one row of kRadixBins counts per tile,
// written and read as whole rows); an exclusive scan of hist in (digit, tile)
// order gives each (digit, tile) its first output slot; the scatter pass then
// places element i of the tile at that slot + the number of earlier elements
// of the tile with the same digit.  Earlier means earlier in edge order: wave
// w of the block owns the tile's edges [w * 1024, (w + 1) * 1024), walked in
// rounds j of 64 consecutive edges (lane order inside a round), so (wave,
// round, lane) order is edge order.  Each pass is therefore stable, and the
// passes over digits 0, 1, ... leave the edges sorted by key with ties in
// ascending edge id.  Keys outside [0, num_nodes) sort as num_nodes, after
// every valid key (past indptr[num_nodes]).
//
// Between passes the edges travel as interleaved (key, edge id) pairs: the
// scatter's output runs (one per digit and tile, 16 elements on average) are
// then 128 bytes instead of two 64-byte pieces.  Pass 0 reads the caller's keys
// (the ids are the positions); the last pass writes the sorted keys and perm
// as two arrays.
constexpr int kSortThreads = 256;
constexpr int kSortItems = 16;
constexpr int kSortTile = kSortThreads * kSortItems;
constexpr int kRadixBits = 8;
constexpr int kRadixBins = 1 << kRadixBits;
static_assert(kRadixBins == kSortThreads, "one digit per thread in the per-digit steps");

DEVI int clamp_key(int k, int num_nodes) { return (unsigned)k < (unsigned)num_nodes ? k : num_nodes; }

// Tile of block b.  Hardware block b runs on XCD b % 8; the tiles are dealt so
// that each XCD takes one contiguous range of them.  A digit's output runs of
// consecutive tiles are adjacent in the output, so a line shared by two runs
// is then mostly completed in one XCD's L2 instead of being written in parts
// from two.
DEVI int xcd_tile(int b, int ntiles) {
  const int q = ntiles >> 3, rem = ntiles & 7, x = b & 7, s = b >> 3;
  return x * q + min(x, rem) + s;
}

// A CSR build the caller has made unnecessary (a device flag it set) skips
// every launch: each block returns before touching memory.
DEVI bool skipped(const int* skip) { return skip && *skip; }

// One row of hist: the digit counts of the tile.  PAIRS: the input is (key, id)
// pairs; else the caller's keys (clamped).  Digit order inside the tile is
// irrelevant here, so full tiles read 16-byte vectors.
// fill / fill_n: also set fill[0, fill_n) to -1 (indptr before its run pass),
// so that no launch of its own is spent on it.
template <bool PAIRS>
__global__ __launch_bounds__(kSortThreads) void radix_hist_kernel(const int* __restrict__ in, long n, int num_nodes,
                                                                 int shift, bool vec, int* __restrict__ hist,
                                                                 int* __restrict__ fill, long fill_n,
                                                                 const int* __restrict__ skip) {
  if (skipped(skip)) return;
  __shared__ int h[kRadixBins];
  const int tid = threadIdx.x;
  h[tid] = 0;
  if (fill)
    for (long i = (long)blockIdx.x * kSortThreads + tid; i < fill_n; i += (long)gridDim.x * kSortThreads) fill[i] = -1;
  const long tile = (long)blockIdx.x * kSortTile;
  int d[kSortItems];
  if (vec && tile + kSortTile <= n) {
    if (PAIRS) {
      const int4* p = reinterpret_cast<const int4*>(in + 2 * tile);
#pragma unroll
      for (int r = 0; r < kSortItems / 2; ++r) {
        const int4 x = p[r * kSortThreads + tid];
        d[2 * r] = (x.x >> shift) & (kRadixBins - 1);
        d[2 * r + 1] = (x.z >> shift) & (kRadixBins - 1);
      }
    } else {
      const int4* p = reinterpret_cast<const int4*>(in + tile);
#pragma unroll
      for (int r = 0; r < kSortItems / 4; ++r) {
        const int4 x = p[r * kSortThreads + tid];
        d[4 * r] = (clamp_key(x.x, num_nodes) >> shift) & (kRadixBins - 1);
        d[4 * r + 1] = (clamp_key(x.y, num_nodes) >> shift) & (kRadixBins - 1);
        d[4 * r + 2] = (clamp_key(x.z, num_nodes) >> shift) & (kRadixBins - 1);
        d[4 * r + 3] = (clamp_key(x.w, num_nodes) >> shift) & (kRadixBins - 1);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
      const long i = tile + (long)j * kSortThreads + tid;
      const int k = i < n ? (PAIRS ? in[2 * i] : clamp_key(in[i], num_nodes)) : -1;
      d[j] = k >= 0 ? (k >> shift) & (kRadixBins - 1) : -1;
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kSortItems; ++j)
    if (d[j] >= 0) atomicAdd(&h[d[j]], 1);
  __syncthreads();
  hist[(long)blockIdx.x * kRadixBins + tid] = h[tid];
}

// The (digit, tile)-order exclusive scan of hist, in place, over its
// [tile][digit] rows: per chunk of kHistChunk tiles the column sums (part);
// one block scans part down each digit's column and adds the digit's base
// (the exclusive scan of the digit totals); per chunk, each digit's column
// is then walked down its kHistChunk rows.
constexpr int kHistChunk = 64;

int hist_chunks(int ntiles) { return (ntiles + kHistChunk - 1) / kHistChunk; }

__global__ __launch_bounds__(kRadixBins) void hist_chunk_sum_kernel(const int* __restrict__ hist, int ntiles,
                                                                   int* __restrict__ part, const int* __restrict__ skip) {
  if (skipped(skip)) return;
  const int b0 = blockIdx.x * kHistChunk, tid = threadIdx.x;
  int x[kHistChunk];
#pragma unroll
  for (int r = 0; r < kHistChunk; ++r) x[r] = b0 + r < ntiles ? hist[(long)(b0 + r) * kRadixBins + tid] : 0;
  int s = 0;
#pragma unroll
  for (int r = 0; r < kHistChunk; ++r) s += x[r];
  part[(long)blockIdx.x * kRadixBins + tid] = s;
}

__global__ __launch_bounds__(4 * kRadixBins) void hist_chunk_scan_kernel(int* __restrict__ part, int nchunks,
                                                                        const int* __restrict__ skip) {
  if (skipped(skip)) return;
  // thread: digit d, quarter q of the chunks
  __shared__ int qsum[4][kRadixBins];
  __shared__ int wtot[4][kRadixBins / 64];
  const int d = threadIdx.x & (kRadixBins - 1), q = threadIdx.x / kRadixBins;
  const int lane = threadIdx.x & 63, wv = d >> 6;
  const int per = (nchunks + 3) / 4, c0 = min(nchunks, q * per), c1 = min(nchunks, c0 + per);
  int s = 0;
#pragma unroll 8
  for (int c = c0; c < c1; ++c) s += part[(long)c * kRadixBins + d];
  qsum[q][d] = s;
  __syncthreads();
  int tot = 0, base = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int x = qsum[w][d];
    base += w < q ? x : 0;
    tot += x;
  }
  // exclusive scan of the digit totals (each quarter computes the same one)
  int x = tot;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) wtot[q][wv] = x;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kRadixBins / 64; ++w) base += w < wv ? wtot[q][w] : 0;
  base += x - tot;
  for (int c = c0; c < c1; ++c) {
    const int y = part[(long)c * kRadixBins + d];
    part[(long)c * kRadixBins + d] = base;
    base += y;
  }
}

__global__ __launch_bounds__(kRadixBins) void hist_chunk_apply_kernel(int* __restrict__ hist, int ntiles,
                                                                     const int* __restrict__ part,
                                                                     const int* __restrict__ skip) {
  if (skipped(skip)) return;
  const int b0 = blockIdx.x * kHistChunk, tid = threadIdx.x;
  int x[kHistChunk];
#pragma unroll
  for (int r = 0; r < kHistChunk; ++r) x[r] = b0 + r < ntiles ? hist[(long)(b0 + r) * kRadixBins + tid] : 0;
  int run = part[(long)blockIdx.x * kRadixBins + tid];
#pragma unroll
  for (int r = 0; r < kHistChunk; ++r) {
    if (b0 + r < ntiles) hist[(long)(b0 + r) * kRadixBins + tid] = run;
    run += x[r];
  }
}

// The same scan in one block of 4 x 256 threads when ntiles <= 4 kHistChunk:
// thread (q, d) holds rows [64 q, 64 q + 64) of digit d's column in registers;
// the quarters' sums and the digit totals' exclusive scan go through LDS.
constexpr int kSmallScanTiles = 4 * kHistChunk;

__global__ __launch_bounds__(4 * kRadixBins) void hist_scan_small_kernel(int* __restrict__ hist, int ntiles,
                                                                        const int* __restrict__ skip) {
  if (skipped(skip)) return;
  __shared__ int qsum[4][kRadixBins];
  __shared__ int wtot[kRadixBins / 64];
  const int d = threadIdx.x & (kRadixBins - 1), q = threadIdx.x / kRadixBins;
  const int lane = threadIdx.x & 63, wv = d >> 6, r0 = q * kHistChunk;
  int x[kHistChunk];
  int s = 0;
#pragma unroll
  for (int r = 0; r < kHistChunk; ++r) {
    x[r] = r0 + r < ntiles ? hist[(long)(r0 + r) * kRadixBins + d] : 0;
    s += x[r];
  }
  qsum[q][d] = s;
  __syncthreads();
  int tot = 0, run = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int y = qsum[w][d];
    run += w < q ? y : 0;
    tot += y;
  }
  // exclusive scan of the digit totals, by the first quarter's waves
  int incl = tot;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (q == 0 && lane == 63) wtot[wv] = incl;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kRadixBins / 64; ++w) run += w < wv ? wtot[w] : 0;
  run += incl - tot;
#pragma unroll
  for (int r = 0; r < kHistChunk; ++r) {
    if (r0 + r < ntiles) hist[(long)(r0 + r) * kRadixBins + d] = run;
    run += x[r];
  }
}

// Exclusive scan of one value per thread over a 256-thread block (sh: 4 ints).
DEVI int block_exclusive_scan256(int v, int* sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) sh[wave] = x;
  __syncthreads();
  int before = 0;
#pragma unroll
  for (int w = 0; w < kSortThreads / 64; ++w) before += w < wave ? sh[w] : 0;
  __syncthreads();
  return before + x - v;
}

// offsets: the exclusive scan of hist in (digit, tile) order, in hist's
// [tile][digit] rows: offsets[t * kRadixBins + d] is the first output slot of
// tile t's digit-d elements.  IN_PAIRS: the input is (key, id) pairs, else the
// caller's keys (clamped) with the positions as ids.  OUT_PAIRS: the output is
// pairs, else keys_out and vals_out.  Each wave ranks its 1024 edges on its
// own (a running count per digit in its own LDS row, peers of a round found
// by ballots over the digit bits); the block then turns the per-wave counts
// into the tile-local start of each digit and each wave's first slot in it,
// places the tile into LDS in (digit, edge) order and writes it out in that
// order, so consecutive threads write consecutive slots of one digit's run
// instead of one slot per digit.  vec: the input may be read as 16-byte
// vectors (full waves read theirs through their LDS slice).
template <bool IN_PAIRS, bool OUT_PAIRS>
__global__ __launch_bounds__(kSortThreads) void radix_scatter_kernel(const int* __restrict__ in, long n,
                                                                    int num_nodes, int shift, bool vec,
                                                                    const int* __restrict__ offsets,
                                                                    int* __restrict__ out,
                                                                    int* __restrict__ vals_out,
                                                                    const int* __restrict__ skip) {
  if (skipped(skip)) return;
  constexpr int kWaves = kSortThreads / 64;
  constexpr int kWaveItems = kSortItems * 64;
  __shared__ int gbase[kRadixBins];         // output slot of the tile's local slot 0, per digit
  __shared__ int wrun[kWaves][kRadixBins];  // per wave: running count, then first tile-local slot, per digit
  __shared__ int2 skv[kSortTile];           // the wave's inputs in edge order, then the tile in output order
  __shared__ int sh[kWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t_idx = xcd_tile(blockIdx.x, gridDim.x);
  const long tile = (long)t_idx * kSortTile;
  const long wbase = tile + (long)wave * kWaveItems;
  int2* stage = skv + wave * kWaveItems;
  int k[kSortItems], v[kSortItems];
  if (wbase + kWaveItems <= n && (IN_PAIRS || vec)) {
    // 16-byte loads of the wave's edges into its own LDS slice in edge order, read back lane-strided
    if (IN_PAIRS) {
      const int4* p = reinterpret_cast<const int4*>(in + 2 * wbase);
      int4 x[kSortItems / 2];
#pragma unroll
      for (int r = 0; r < kSortItems / 2; ++r) x[r] = p[r * 64 + lane];
#pragma unroll
      for (int r = 0; r < kSortItems / 2; ++r) reinterpret_cast<int4*>(stage)[r * 64 + lane] = x[r];
    } else {
      const int4* p = reinterpret_cast<const int4*>(in + wbase);
      int4 x[kSortItems / 4];
#pragma unroll
      for (int r = 0; r < kSortItems / 4; ++r) x[r] = p[r * 64 + lane];
#pragma unroll
      for (int r = 0; r < kSortItems / 4; ++r) {
        const int e = 4 * (r * 64 + lane);
        reinterpret_cast<int4*>(stage)[(r * 64 + lane) * 2] =
            int4{clamp_key(x[r].x, num_nodes), (int)(wbase + e), clamp_key(x[r].y, num_nodes), (int)(wbase + e + 1)};
        reinterpret_cast<int4*>(stage)[(r * 64 + lane) * 2 + 1] =
            int4{clamp_key(x[r].z, num_nodes), (int)(wbase + e + 2), clamp_key(x[r].w, num_nodes), (int)(wbase + e + 3)};
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
      const int2 x = stage[j * 64 + lane];
      k[j] = x.x;
      v[j] = x.y;
    }
  } else {
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
      const long i = wbase + (long)j * 64 + lane;
      if (IN_PAIRS) {
        const int2 x = i < n ? reinterpret_cast<const int2*>(in)[i] : int2{-1, 0};
        k[j] = x.x;
        v[j] = x.y;
      } else {
        k[j] = i < n ? clamp_key(in[i], num_nodes) : -1;
        v[j] = (int)i;
      }
    }
  }
  const int g0 = offsets[(long)t_idx * kRadixBins + tid];
#pragma unroll
  for (int w = 0; w < kWaves; ++w) wrun[w][tid] = 0;
  __syncthreads();
  // rank inside the wave: slot among the wave's earlier edges of the same digit
  const uint64_t below_mask = (1ull << lane) - 1;
  int* run = wrun[wave];
  int r[kSortItems];
#pragma unroll
  for (int j = 0; j < kSortItems; ++j) {
    const bool valid = k[j] >= 0;
    const int d = valid ? (k[j] >> shift) & (kRadixBins - 1) : 0;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < kRadixBits; ++b) {
      const bool bit = (d >> b) & 1;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const int below = __popcll(peers & below_mask);
    const int before = valid ? run[d] : 0;
    __builtin_amdgcn_wave_barrier();
    if (valid && below == 0) run[d] = before + __popcll(peers);
    __builtin_amdgcn_wave_barrier();
    r[j] = before + below;
  }
  __syncthreads();
  // digit tid: tile-local start, and each wave's first slot in it
  {
    int c[kWaves], tot = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) { c[w] = wrun[w][tid]; tot += c[w]; }
    int acc = block_exclusive_scan256(tot, sh);
    gbase[tid] = g0 - acc;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) { wrun[w][tid] = acc; acc += c[w]; }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kSortItems; ++j)
    if (k[j] >= 0) skv[run[(k[j] >> shift) & (kRadixBins - 1)] + r[j]] = int2{k[j], v[j]};
  __syncthreads();
  const int m = (int)min((long)kSortTile, n - tile);
  for (int t = tid; t < m; t += kSortThreads) {
    const int2 x = skv[t];
    const int g = gbase[(x.x >> shift) & (kRadixBins - 1)] + t;
    if (OUT_PAIRS) {
      reinterpret_cast<int2*>(out)[g] = x;
    } else {
      out[g] = x.x;
      vals_out[g] = x.y;
    }
  }
}

// indptr from the sorted keys s (values in [0, num_nodes], num_nodes standing
// for the invalid keys): indptr[j] = the number of keys below j.  Boundary i
// in [0, n] lies between prev = s[i - 1] (-1 at i = 0) and cur = s[i]
// (num_nodes at i = n); every j in (prev, cur] gets i.  Each j has exactly one
// such boundary, so there are no write conflicts and no atomics.  A boundary
// fills at most kGapFill entries itself; longer gaps (runs of absent keys) get
// only indptr[cur] and leave the rest at -1 for indptr_gap_kernel.  Thread t
// owns boundaries [4t, 4t + 4).
constexpr int kGapFill = 64;

__global__ void fill_int_kernel(int* __restrict__ p, long n, int value, const int* __restrict__ skip) {
  if (skipped(skip)) return;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) p[i] = value;
}

__global__ __launch_bounds__(256) void indptr_runs_kernel(const int* __restrict__ s, long n, int num_nodes,
                                                         int* __restrict__ indptr, const int* __restrict__ skip) {
  if (skipped(skip)) return;
  const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long i0 = 4 * t;
  if (i0 > n) return;
  int cur[4];
  if (i0 + 4 <= n) {
    const int4 x = reinterpret_cast<const int4*>(s)[t];
    cur[0] = x.x; cur[1] = x.y; cur[2] = x.z; cur[3] = x.w;
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) cur[q] = i0 + q < n ? s[i0 + q] : num_nodes;
  }
  int prev = i0 == 0 ? -1 : s[i0 - 1];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const long i = i0 + q;
    if (i > n) break;
    const int c = cur[q];
    if (c > prev) {
      if (c - prev <= kGapFill) {
        for (int j = prev + 1; j <= c; ++j) indptr[j] = (int)i;
      } else {
        indptr[c] = (int)i;
      }
    }
    prev = c;
  }
}

// Entries left at -1 (inside a gap longer than kGapFill): the first position
// whose key is >= j, by binary search.
__global__ void indptr_gap_kernel(const int* __restrict__ s, long n, int num_nodes, int* __restrict__ indptr,
                                  const int* __restrict__ skip) {
  if (skipped(skip)) return;
  for (long j = (long)blockIdx.x * blockDim.x + threadIdx.x; j <= num_nodes; j += (long)gridDim.x * blockDim.x) {
    if (indptr[j] >= 0) continue;
    long lo = 0, hi = n;
    while (lo < hi) {
      const long mid = (lo + hi) >> 1;
      if (s[mid] < (int)j) lo = mid + 1; else hi = mid;
    }
    indptr[j] = (int)lo;
  }
}

// ------------------------------------------------------------------ segment sums

template <typename T> struct Vec16;
template <> struct Vec16<float> { static constexpr int N = 4; };
template <> struct Vec16<bf16> { static constexpr int N = 8; };

template <typename T>
DEVI void load16(const T* p, float* v);
template <>
DEVI void load16<float>(const float* p, float* v) {
  const f32x4 x = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = x[i];
}
template <>
DEVI void load16<bf16>(const bf16* p, float* v) {
  const bf16x8 x = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (float)x[i];
}
template <typename T>
DEVI void store16(T* p, const float* v);
template <>
DEVI void store16<float>(float* p, const float* v) {
  f32x4 x;
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = v[i];
  *reinterpret_cast<f32x4*>(p) = x;
}
template <>
DEVI void store16<bf16>(bf16* p, const float* v) {
  bf16x8 x;
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = (bf16)v[i];
  *reinterpret_cast<bf16x8*>(p) = x;
}

// Adds segment [a, b) of rows y[perm[i]*ld + off ...] into acc, ascending i.
// Loads are issued four rows ahead; the additions stay in ascending order.
template <typename T>
DEVI void accumulate_segment(const T* __restrict__ y, const int* __restrict__ perm, int a, int b, long ld,
                             int off, float* acc) {
  constexpr int V = Vec16<T>::N;
  int i = a;
  for (; i + 4 <= b; i += 4) {
    float r[4][V];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const long e = perm ? perm[i + u] : i + u;
      load16<T>(y + e * ld + off, r[u]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int k = 0; k < V; ++k) acc[k] += r[u][k];
  }
  for (; i < b; ++i) {
    const long e = perm ? perm[i] : i;
    float r[V];
    load16<T>(y + e * ld + off, r);
#pragma unroll
    for (int k = 0; k < V; ++k) acc[k] += r[k];
  }
}

// One wave per node (grid-stride); each lane owns 16-byte column chunks.
// out[n] = seg(y, csr1, off1) (+ seg(y, csr2, off2) when indptr2 != null).
template <typename T>
__global__ __launch_bounds__(256) void segment_sum_kernel(const T* __restrict__ y, long ld,
                                                          const int* __restrict__ perm1,
                                                          const int* __restrict__ indptr1, int off1,
                                                          const int* __restrict__ perm2,
                                                          const int* __restrict__ indptr2, int off2,
                                                          int num_nodes, int features, T* __restrict__ out) {
  constexpr int V = Vec16<T>::N;
  const int lane = threadIdx.x & 63;
  const int chunks = features / V;
  const int waves = gridDim.x * (blockDim.x >> 6);
  for (int n = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)); n < num_nodes;
       n += waves) {
    const int a1 = indptr1[n], b1 = indptr1[n + 1];
    int a2 = 0, b2 = 0;
    if (indptr2) { a2 = indptr2[n]; b2 = indptr2[n + 1]; }
    for (int c = lane; c < chunks; c += 64) {
      float acc[V];
#pragma unroll
      for (int k = 0; k < V; ++k) acc[k] = 0.f;
      accumulate_segment<T>(y, perm1, a1, b1, ld, off1 + c * V, acc);
      if (indptr2) accumulate_segment<T>(y, perm2, a2, b2, ld, off2 + c * V, acc);
      store16<T>(out + (size_t)n * features + c * V, acc);
    }
  }
}

// Row mode: one wave per node and the whole row across the wave (VB bytes of
// each row per lane, rows of 64 * VB bytes).  The CSR bounds and perm entries
// are wave-uniform (scalar loads); U rows are in flight per step and are
// added in ascending position, so the sum is the same fp32 left-to-right sum
// as the one-lane-per-chunk kernel.
constexpr int kSegU = 8;

template <typename T, int VB> struct RowVec;
template <> struct RowVec<float, 16> { typedef f32x4 type; static constexpr int N = 4; };
template <> struct RowVec<bf16, 16> { typedef bf16x8 type; static constexpr int N = 8; };
template <> struct RowVec<bf16, 8> { typedef bf16x4 type; static constexpr int N = 4; };
template <> struct RowVec<float, 8> { typedef float __attribute__((ext_vector_type(2))) type; static constexpr int N = 2; };

template <typename T, int VB>
DEVI void segment_rows(const T* __restrict__ y, const int* __restrict__ perm, int a, int b, long ld, int col,
                       float* acc) {
  typedef typename RowVec<T, VB>::type V;
  constexpr int N = RowVec<T, VB>::N;
  const int lane = threadIdx.x & 63;
  for (int i = a; i < b; i += kSegU) {
    // perm entries of this step: one vector load, broadcast with readlane
    const int pe = perm ? perm[min(i + (lane & (kSegU - 1)), b - 1)] : 0;
    V r[kSegU];
#pragma unroll
    for (int u = 0; u < kSegU; ++u) {
      const long e = perm ? __builtin_amdgcn_readlane(pe, u) : min(i + u, b - 1);
      r[u] = *reinterpret_cast<const V*>(y + e * ld + col);
    }
#pragma unroll
    for (int u = 0; u < kSegU; ++u) {
      if (i + u < b) {
#pragma unroll
        for (int k = 0; k < N; ++k) acc[k] += (float)r[u][k];
      }
    }
  }
}

template <typename T, int VB>
__global__ __launch_bounds__(256) void segment_sum_rows_kernel(const T* __restrict__ y, long ld,
                                                               const int* __restrict__ perm1,
                                                               const int* __restrict__ indptr1, int off1,
                                                               const int* __restrict__ perm2,
                                                               const int* __restrict__ indptr2, int off2,
                                                               int num_nodes, int features, T* __restrict__ out) {
  typedef typename RowVec<T, VB>::type V;
  constexpr int N = RowVec<T, VB>::N;
  const int lane = threadIdx.x & 63;
  const int waves = gridDim.x * 4;
  for (int n = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); n < num_nodes; n += waves) {
    const int a1 = indptr1[n], b1 = indptr1[n + 1];
    for (int col = lane * N; col < features; col += 64 * N) {
      float acc[N];
#pragma unroll
      for (int k = 0; k < N; ++k) acc[k] = 0.f;
      segment_rows<T, VB>(y, perm1, a1, b1, ld, off1 + col, acc);
      if (indptr2) segment_rows<T, VB>(y, perm2, indptr2[n], indptr2[n + 1], ld, off2 + col, acc);
      V o;
#pragma unroll
      for (int k = 0; k < N; ++k) o[k] = (T)acc[k];
      *reinterpret_cast<V*>(out + (size_t)n * features + col) = o;
    }
  }
}

// Stream mode for one CSR whose rows are exactly one wave-load wide
// (features * sizeof(T) == 64 * VB): a wave owns `npw` consecutive nodes and
// walks their positions indptr[n0] .. indptr[n0 + npw] as one stream, U rows
// per step with the next step's loads in flight while the current step is
// added (two register buffers, so no load is waited for early).  A node's
// sum is stored when the stream crosses its end; every node still gets the
// fp32 left-to-right sum of its own rows, starting from 0.  The wave's
// indptr entries are held one per lane and read with readlane.
#ifndef ESA_STREAM_BYTES
#define ESA_STREAM_BYTES 128  // bytes in flight per lane per step
#endif
#ifndef ESA_STREAM_NODES
#define ESA_STREAM_NODES 32   // nodes per wave (at most 63)
#endif
#ifndef ESA_NODE_MODE
#define ESA_NODE_MODE 1       // canonical-order CSRs of 512 / 1024-byte rows: the node-per-wave kernel
#endif
#ifndef ESA_STREAM_NTSTORE
#define ESA_STREAM_NTSTORE 0  // nontemporal stores of the node sums
#endif
constexpr int kStreamNodes = ESA_STREAM_NODES;

template <int VB> struct StreamU { static constexpr int value = ESA_STREAM_BYTES / VB; };

template <typename T, int VB>
DEVI void stream_load(const T* __restrict__ y, const int* __restrict__ perm, int i, int iend, int col,
                      typename RowVec<T, VB>::type* r) {
  typedef typename RowVec<T, VB>::type V;
  constexpr int kStreamU = StreamU<VB>::value;
  const int lane = threadIdx.x & 63;
  const int pe = perm ? perm[min(i + (lane & (kStreamU - 1)), iend - 1)] : 0;
#pragma unroll
  for (int u = 0; u < kStreamU; ++u) {
    const long e = perm ? __builtin_amdgcn_readlane(pe, u) : min(i + u, iend - 1);
    // read once: nontemporal, so the stream does not evict reused lines from L2
    r[u] = __builtin_nontemporal_load(reinterpret_cast<const V*>(y + e * (long)(64 * RowVec<T, VB>::N) + col));
  }
}

template <typename T, int VB>
__global__ __launch_bounds__(256) void segment_sum_stream_kernel(const T* __restrict__ y,
                                                                 const int* __restrict__ perm,
                                                                 const int* __restrict__ indptr, int num_nodes,
                                                                 T* __restrict__ out) {
  typedef typename RowVec<T, VB>::type V;
  constexpr int N = RowVec<T, VB>::N;
  constexpr int F = 64 * N;
  constexpr int kStreamU = StreamU<VB>::value;
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = wave * kStreamNodes;
  if (n0 >= num_nodes) return;
  const int nn = min(kStreamNodes, num_nodes - n0);
  const int ip = indptr[n0 + min(lane, nn)];   // lanes 0..nn: indptr[n0 .. n0 + nn]
  const int col = lane * N;
  int k = 0;                                    // current node n0 + k
  int b = __builtin_amdgcn_readlane(ip, 1);     // its end
  const int iend = __builtin_amdgcn_readlane(ip, nn);
  float acc[N];
#pragma unroll
  for (int c = 0; c < N; ++c) acc[c] = 0.f;
  auto flush = [&]() {
    V o;
#pragma unroll
    for (int c = 0; c < N; ++c) { o[c] = (T)acc[c]; acc[c] = 0.f; }
#if ESA_STREAM_NTSTORE
    __builtin_nontemporal_store(o, reinterpret_cast<V*>(out + (size_t)(n0 + k) * F + col));
#else
    *reinterpret_cast<V*>(out + (size_t)(n0 + k) * F + col) = o;
#endif
    ++k;
    b = __builtin_amdgcn_readlane(ip, min(k + 1, nn));
  };
  auto consume = [&](int i, const V* r) {
#pragma unroll
    for (int u = 0; u < kStreamU; ++u) {
      const int row = i + u;
      if (row >= iend) break;
      while (row >= b) flush();
#pragma unroll
      for (int c = 0; c < N; ++c) acc[c] += (float)r[u][c];
    }
  };
  int i = __builtin_amdgcn_readlane(ip, 0);
  V ra[kStreamU], rb[kStreamU];
  if (i < iend) stream_load<T, VB>(y, perm, i, iend, col, ra);
  while (i < iend) {
    if (i + kStreamU < iend) stream_load<T, VB>(y, perm, i + kStreamU, iend, col, rb);
    consume(i, ra);
    i += kStreamU;
    if (i >= iend) break;
    if (i + kStreamU < iend) stream_load<T, VB>(y, perm, i + kStreamU, iend, col, ra);
    consume(i, rb);
    i += kStreamU;
  }
  while (k < nn) flush();
}

// Node mode for one CSR in canonical order (no perm) whose rows are 512 or
// 1024 bytes: NPW nodes per wave, 64 / NPW lanes per node, 16 bytes of every
// row per lane.  Each step has up to U rows of a node in flight (nontemporal
// loads, issued only for the node's own rows), then adds them in ascending
// position, so every lane keeps the fp32 left-to-right sum of its columns.
// A wave lives for its nodes only; occupancy hides the load latency (the
// access pattern of a plain streaming read, which reaches about 7 TB/s).
#ifndef ESA_NODE_U_F32
#define ESA_NODE_U_F32 32   // rows in flight per node and step, fp32 rows
#endif
#ifndef ESA_NODE_U_BF16
#define ESA_NODE_U_BF16 8   // bf16 rows (their conversions and the two nodes per wave cost registers)
#endif
template <typename T, int NPW, int U>
__global__ __launch_bounds__(256) void segment_sum_node_kernel(const T* __restrict__ y, const int* __restrict__ indptr,
                                                               int num_nodes, T* __restrict__ out) {
  constexpr int LPN = 64 / NPW;            // lanes per node
  constexpr int E = 16 / (int)sizeof(T);   // elements per lane per row
  constexpr int F = LPN * E;               // row elements
  const int lane = threadIdx.x & 63;
  const long n = ((long)blockIdx.x * 4 + (threadIdx.x >> 6)) * NPW + lane / LPN;
  const int l = lane % LPN;
  const bool valid = n < num_nodes;
  const int a = valid ? indptr[n] : 0, b = valid ? indptr[n + 1] : 0;
  float acc[E];
#pragma unroll
  for (int k = 0; k < E; ++k) acc[k] = 0.f;
  const u32x4* row0 = reinterpret_cast<const u32x4*>(y) + l;
  for (int i = a; __ballot(i < b); i += U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i + u < b) v[u] = __builtin_nontemporal_load(row0 + (size_t)(i + u) * (F * sizeof(T) / 16));
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (i + u < b) {
        if constexpr (sizeof(T) == 4) {
          const f32x4 f = __builtin_bit_cast(f32x4, v[u]);
#pragma unroll
          for (int k = 0; k < 4; ++k) acc[k] += f[k];
        } else {
          const bf16x8 h = __builtin_bit_cast(bf16x8, v[u]);
#pragma unroll
          for (int k = 0; k < 8; ++k) acc[k] += (float)h[k];
        }
      }
    }
  }
  if (!valid) return;
  typedef T VE __attribute__((ext_vector_type(E)));
  VE o;
#pragma unroll
  for (int k = 0; k < E; ++k) o[k] = (T)acc[k];
  __builtin_nontemporal_store(o, reinterpret_cast<VE*>(out + (size_t)n * F) + l);
}

// Element-wise fallback for feature counts that are not a multiple of 16 bytes.
template <typename T>
__global__ void segment_sum_scalar_kernel(const T* __restrict__ y, long ld, const int* __restrict__ perm1,
                                          const int* __restrict__ indptr1, int off1,
                                          const int* __restrict__ perm2, const int* __restrict__ indptr2,
                                          int off2, int num_nodes, int features, T* __restrict__ out) {
  const long total = (long)num_nodes * features;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    const int n = (int)(i / features), f = (int)(i - (long)n * features);
    float acc = 0.f;
    for (int j = indptr1[n]; j < indptr1[n + 1]; ++j) {
      const long e = perm1 ? perm1[j] : j;
      acc += (float)y[e * ld + off1 + f];
    }
    if (indptr2)
      for (int j = indptr2[n]; j < indptr2[n + 1]; ++j) {
        const long e = perm2 ? perm2[j] : j;
        acc += (float)y[e * ld + off2 + f];
      }
    out[i] = (T)acc;
  }
}

// Largest finite value of T (torch_scatter's initial value for a minimum).
template <typename T> DEVI float max_finite();
template <> DEVI float max_finite<float>() { return 3.40282347e38f; }
template <> DEVI float max_finite<bf16>() { return __uint_as_float(0x7F7F0000u); }

constexpr int kMinMaxRound = 8;   // CSR positions a lane loads per round

// Segmented minimum (MAX = false) or maximum with its argument: one lane per
// (node, feature), consecutive lanes on consecutive features of a node.  The
// running value starts at the largest finite value (the lowest for MAX) and is
// replaced only by a strictly smaller (larger) element, taken in ascending CSR
// position, so with a stable CSR a tie keeps the lowest edge id and NaN and
// values beyond the start never win; a value never replaced is written as 0
// with arg = num_edges.  Comparisons are exact (bf16 values compare as fp32).
template <typename T, bool MAX>
__global__ __launch_bounds__(256) void segment_minmax_kernel(const T* __restrict__ y, const int* __restrict__ perm,
                                                             const int* __restrict__ indptr, int num_nodes,
                                                             int features, long long num_edges, T* __restrict__ out,
                                                             long long* __restrict__ arg) {
  const long total = (long)num_nodes * features;
  const float start = MAX ? -max_finite<T>() : max_finite<T>();
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    const int n = (int)(i / features), f = (int)(i - (long)n * features);
    float best = start;
    long long at = num_edges;
    const int j1 = indptr[n + 1];
    // 8 positions per round: their edge ids and then their values load independently (a chain of two
    // dependent loads per round, not per position); the compares keep ascending position order.
    for (int j = indptr[n]; j < j1; j += kMinMaxRound) {
      long e[kMinMaxRound];
      float v[kMinMaxRound];
#pragma unroll
      for (int k = 0; k < kMinMaxRound; ++k) e[k] = j + k < j1 ? (perm ? perm[j + k] : j + k) : -1;
#pragma unroll
      for (int k = 0; k < kMinMaxRound; ++k) v[k] = e[k] >= 0 ? (float)y[e[k] * features + f] : start;
#pragma unroll
      for (int k = 0; k < kMinMaxRound; ++k)
        if (MAX ? v[k] > best : v[k] < best) {
          best = v[k];
          at = e[k];
        }
    }
    out[i] = at == num_edges ? (T)0.f : (T)best;
    if (arg) arg[i] = at;
  }
}

unsigned grid_for(long n, int block, long cap = 1L << 20) {
  long g = (n + block - 1) / block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (unsigned)g;
}

bool misaligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) != 0; }

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

int radix_blocks(int64_t num_edges) { return (int)((num_edges + kSortTile - 1) / kSortTile); }

// Passes of kRadixBits over the keys 0 .. num_nodes (num_nodes: the slot of invalid keys).
int radix_passes(int num_nodes) {
  const int bits = 32 - __builtin_clz((unsigned)num_nodes | 1u);
  return (bits + kRadixBits - 1) / kRadixBits;
}

// Workspace: hist and its chunk sums, and two buffers of E (key, id) pairs
// (pass p writes pair buffer p & 1; the last pass writes the sorted keys into
// the buffer it does not read).
struct CsrWs { size_t hist, part, pairs_a, pairs_b, total; };
CsrWs csr_ws(int64_t num_edges, int num_nodes) {
  (void)num_nodes;
  CsrWs w;
  const long nhist = (long)kRadixBins * radix_blocks(num_edges);
  const long npart = (long)kRadixBins * hist_chunks(radix_blocks(num_edges));
  size_t off = 0;
  w.hist = off; off += align256((size_t)(nhist > 0 ? nhist : 1) * 4);
  w.part = off; off += align256((size_t)(npart > 0 ? npart : 1) * 4);
  w.pairs_a = off; off += align256((size_t)num_edges * 8);
  w.pairs_b = off; off += align256((size_t)num_edges * 8);
  w.total = off;
  return w;
}

template <typename T>
int launch_segsum(const T* y, long ld, const int* perm1, const int* indptr1, int off1, const int* perm2,
                  const int* indptr2, int off2, int num_nodes, int features, T* out, hipStream_t st) {
  constexpr int V = Vec16<T>::N;
  const bool vec = features % V == 0 && ld % V == 0 && off1 % V == 0 && off2 % V == 0 && !misaligned16(y) &&
                   !misaligned16(out);
  const long row_bytes = (long)features * (long)sizeof(T);
  const bool rows_ok = !misaligned16(y) && !misaligned16(out) && (ld * (long)sizeof(T)) % 16 == 0 &&
                       (off1 * (long)sizeof(T)) % 16 == 0 && (off2 * (long)sizeof(T)) % 16 == 0;
  if (ESA_NODE_MODE && rows_ok && !perm1 && !perm2 && !indptr2 && off1 == 0 && ld == features &&
      (row_bytes == 64 * 16 || row_bytes == 32 * 16)) {
    constexpr int U = sizeof(T) == 4 ? ESA_NODE_U_F32 : ESA_NODE_U_BF16;
    if (row_bytes == 64 * 16) {
      const unsigned blocks = (unsigned)(((long)num_nodes + 3) / 4);
      ESA_TIMED(esa_profile::kSegmentSum, st,
                hipLaunchKernelGGL((segment_sum_node_kernel<T, 1, U>), dim3(blocks), dim3(256), 0, st, y, indptr1,
                                   num_nodes, out));
    } else {
      const unsigned blocks = (unsigned)(((long)num_nodes + 7) / 8);
      ESA_TIMED(esa_profile::kSegmentSum, st,
                hipLaunchKernelGGL((segment_sum_node_kernel<T, 2, U>), dim3(blocks), dim3(256), 0, st, y, indptr1,
                                   num_nodes, out));
    }
  } else if (rows_ok && !perm2 && !indptr2 && off1 == 0 && ld == features &&
             (row_bytes == 64 * 16 || row_bytes == 64 * 8)) {
    const long waves = ((long)num_nodes + kStreamNodes - 1) / kStreamNodes;
    const unsigned blocks = (unsigned)((waves + 3) / 4);
    if (row_bytes == 64 * 16)
      ESA_TIMED(esa_profile::kSegmentSum, st,
                hipLaunchKernelGGL((segment_sum_stream_kernel<T, 16>), dim3(blocks), dim3(256), 0, st, y, perm1,
                                   indptr1, num_nodes, out));
    else
      ESA_TIMED(esa_profile::kSegmentSum, st,
                hipLaunchKernelGGL((segment_sum_stream_kernel<T, 8>), dim3(blocks), dim3(256), 0, st, y, perm1,
                                   indptr1, num_nodes, out));
  } else if (rows_ok && row_bytes % (64 * 16) == 0) {
    const unsigned blocks = grid_for((long)num_nodes, 4, 1L << 18);
    ESA_TIMED(esa_profile::kSegmentSum, st,
              hipLaunchKernelGGL((segment_sum_rows_kernel<T, 16>), dim3(blocks), dim3(256), 0, st, y, ld, perm1,
                                 indptr1, off1, perm2, indptr2, off2, num_nodes, features, out));
  } else if (rows_ok && row_bytes % (64 * 8) == 0) {
    const unsigned blocks = grid_for((long)num_nodes, 4, 1L << 18);
    ESA_TIMED(esa_profile::kSegmentSum, st,
              hipLaunchKernelGGL((segment_sum_rows_kernel<T, 8>), dim3(blocks), dim3(256), 0, st, y, ld, perm1,
                                 indptr1, off1, perm2, indptr2, off2, num_nodes, features, out));
  } else if (vec) {
    const unsigned blocks = grid_for((long)num_nodes, 4, 1L << 18);
    ESA_TIMED(esa_profile::kSegmentSum, st,
              hipLaunchKernelGGL(segment_sum_kernel<T>, dim3(blocks), dim3(256), 0, st, y, ld, perm1, indptr1, off1,
                                 perm2, indptr2, off2, num_nodes, features, out));
  } else {
    hipLaunchKernelGGL(segment_sum_scalar_kernel<T>, dim3(grid_for((long)num_nodes * features, 256)), dim3(256), 0,
                       st, y, ld, perm1, indptr1, off1, perm2, indptr2, off2, num_nodes, features, out);
  }
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

}  // namespace

extern "C" {

int esa_edge_gather(const void* x, const int* src, const int* dst, int64_t num_edges, int num_nodes,
                    int features, int dtype, void* out, void* stream) {
  if (num_edges < 0 || num_nodes < 0 || features < 1) return ESA_ERR_SHAPE;
  if (dtype != ESA_F32 && dtype != ESA_BF16) return ESA_ERR_DTYPE;
  if (num_edges == 0) return ESA_OK;
  if (!x || !src || !dst || !out) return ESA_ERR_NULL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int es = dtype == ESA_F32 ? 4 : 2;
  const long row_bytes = (long)features * es;
  const long x_bytes = (long)num_nodes * row_bytes;
  const int row_chunks = (int)(row_bytes / 16);
  const int pieces = row_bytes % 16 == 0 ? 2 * row_chunks / 64 : 0;
  if (row_bytes % 512 == 0 && !misaligned16(x) && !misaligned16(out) && x_bytes <= (1L << 31) &&
      (pieces == 1 || pieces == 2 || pieces == 4)) {
    // Row mode: one step (all of a wave's gather loads in flight at once) per wave, a multiple of 8 blocks
    // (one share per XCD).
    const int epw = ESA_GATHER_LOADS / pieces * ESA_GATHER_STEPS;
    const long waves = (num_edges + epw - 1) / epw;
    const long blocks8 = ((waves + 3) / 4 + 7) / 8 * 8;
    const int per_xcd = (int)(blocks8 / 8);
    auto go = [&](auto kern) {
      ESA_TIMED(esa_profile::kEdgeGather, st,
                hipLaunchKernelGGL(kern, dim3((unsigned)blocks8), dim3(256), 0, st, x, (uint32_t)x_bytes, src, dst,
                                   (long)num_edges, num_nodes, row_chunks, epw, per_xcd, static_cast<u32x4*>(out)));
    };
    if (pieces == 1) go(edge_gather_rows_kernel<1>);
    else if (pieces == 2) go(edge_gather_rows_kernel<2>);
    else go(edge_gather_rows_kernel<4>);
  } else if (row_bytes % 16 == 0 && !misaligned16(x) && !misaligned16(out)) {
    const int chunks = (int)(row_bytes / 16);
    // About 4096 chunk moves per block.
    int epb = (int)(4096 / (2 * chunks));
    if (epb < 1) epb = 1;
    const long blocks = (num_edges + epb - 1) / epb;
    ESA_TIMED(esa_profile::kEdgeGather, st,
              hipLaunchKernelGGL(edge_gather_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                                 static_cast<const u32x4*>(x), src, dst, (long)num_edges, num_nodes, chunks, epb,
                                 static_cast<u32x4*>(out)));
  } else if (dtype == ESA_F32) {
    hipLaunchKernelGGL(edge_gather_scalar_kernel<float>, dim3(grid_for(num_edges * 2 * features, 256)), dim3(256), 0,
                       st, static_cast<const float*>(x), src, dst, (long)num_edges, num_nodes, features,
                       static_cast<float*>(out));
  } else {
    hipLaunchKernelGGL(edge_gather_scalar_kernel<bf16>, dim3(grid_for(num_edges * 2 * features, 256)), dim3(256), 0,
                       st, static_cast<const bf16*>(x), src, dst, (long)num_edges, num_nodes, features,
                       static_cast<bf16*>(out));
  }
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

int esa_edge_gather_add(const void* a, int64_t lda, const void* b, int64_t ldb, const void* bias, const int* src,
                        const int* dst, int64_t num_edges, int num_nodes, int features, int dtype, void* out,
                        void* stream) {
  if (num_edges < 0 || num_nodes < 0 || features < 1 || lda < features || ldb < features) return ESA_ERR_SHAPE;
  if (dtype != ESA_F32 && dtype != ESA_BF16) return ESA_ERR_DTYPE;
  if (num_edges == 0) return ESA_OK;
  if (!a || !b || !src || !dst || !out) return ESA_ERR_NULL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int es = dtype == ESA_F32 ? 4 : 2;
  const long row_bytes = (long)features * es;
  const int C = (int)(row_bytes / 16);
  const bool vec_ok = row_bytes % 16 == 0 && (lda * es) % 16 == 0 && (ldb * es) % 16 == 0 && !misaligned16(a) &&
                      !misaligned16(b) && !misaligned16(out) && (!bias || !misaligned16(bias));
  const bool pow2 = C > 0 && (C & (C - 1)) == 0;
  const int P = C > 64 ? C / 64 : 1;
  if (ESA_GADD_ROWS && vec_ok && C % 64 == 0 && (P == 1 || P == 2 || P == 4 || P == 8)) {
    const int epw = 32;
    const long waves = (num_edges + epw - 1) / epw;
    const long blocks8 = ((waves + 3) / 4 + 7) / 8 * 8;
    const int per_xcd = (int)(blocks8 / 8);
    auto go = [&](auto kern) {
      ESA_TIMED(esa_profile::kEdgeGatherAdd, st,
                hipLaunchKernelGGL(kern, dim3((unsigned)blocks8), dim3(256), 0, st, static_cast<const char*>(a),
                                   (long)(lda * es), static_cast<const char*>(b), (long)(ldb * es),
                                   static_cast<const u32x4*>(bias), src, dst, (long)num_edges, num_nodes, epw,
                                   per_xcd, static_cast<u32x4*>(out)));
    };
    if (dtype == ESA_F32) {
      if (P == 1) go(edge_gather_add_rows_kernel<float, 1>);
      else if (P == 2) go(edge_gather_add_rows_kernel<float, 2>);
      else if (P == 4) go(edge_gather_add_rows_kernel<float, 4>);
      else go(edge_gather_add_rows_kernel<float, 8>);
    } else {
      if (P == 1) go(edge_gather_add_rows_kernel<bf16, 1>);
      else if (P == 2) go(edge_gather_add_rows_kernel<bf16, 2>);
      else if (P == 4) go(edge_gather_add_rows_kernel<bf16, 4>);
      else go(edge_gather_add_rows_kernel<bf16, 8>);
    }
  } else if (vec_ok && ((C <= 64 && pow2) || (C % 64 == 0 && (P == 2 || P == 4 || P == 8)))) {
    const int L = C < 64 ? C : 64;
    const long per_step = (long)(8 / P) * (64 / L);
    const long steps = (num_edges + per_step - 1) / per_step;
    const long steps_per_wave = 4;
    const long waves = (steps + steps_per_wave - 1) / steps_per_wave;
    const long blocks8 = ((waves + 3) / 4 + 7) / 8 * 8;
    const int per_xcd = (int)(blocks8 / 8);
    const long lda16 = lda * es / 16, ldb16 = ldb * es / 16;
    auto go = [&](auto kern) {
      ESA_TIMED(esa_profile::kEdgeGatherAdd, st,
                hipLaunchKernelGGL(kern, dim3((unsigned)blocks8), dim3(256), 0, st, static_cast<const u32x4*>(a),
                                   lda16, static_cast<const u32x4*>(b), ldb16, static_cast<const u32x4*>(bias), src,
                                   dst, (long)num_edges, num_nodes, L, steps_per_wave, per_xcd,
                                   static_cast<u32x4*>(out)));
    };
    if (dtype == ESA_F32) {
      if (P == 1) go(edge_gather_add_kernel<float, 1>);
      else if (P == 2) go(edge_gather_add_kernel<float, 2>);
      else if (P == 4) go(edge_gather_add_kernel<float, 4>);
      else go(edge_gather_add_kernel<float, 8>);
    } else {
      if (P == 1) go(edge_gather_add_kernel<bf16, 1>);
      else if (P == 2) go(edge_gather_add_kernel<bf16, 2>);
      else if (P == 4) go(edge_gather_add_kernel<bf16, 4>);
      else go(edge_gather_add_kernel<bf16, 8>);
    }
  } else if (dtype == ESA_F32) {
    hipLaunchKernelGGL(edge_gather_add_scalar_kernel<float>, dim3(grid_for(num_edges * features, 256)), dim3(256), 0,
                       st, static_cast<const float*>(a), (long)lda, static_cast<const float*>(b), (long)ldb,
                       static_cast<const float*>(bias), src, dst, (long)num_edges, num_nodes, features,
                       static_cast<float*>(out));
  } else {
    hipLaunchKernelGGL(edge_gather_add_scalar_kernel<bf16>, dim3(grid_for(num_edges * features, 256)), dim3(256), 0,
                       st, static_cast<const bf16*>(a), (long)lda, static_cast<const bf16*>(b), (long)ldb,
                       static_cast<const bf16*>(bias), src, dst, (long)num_edges, num_nodes, features,
                       static_cast<bf16*>(out));
  }
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

int esa_csr_workspace_size(int64_t num_edges, int num_nodes, size_t* bytes) {
  if (!bytes) return ESA_ERR_NULL;
  if (num_edges < 0 || num_nodes < 0 || num_edges >= (1LL << 31)) return ESA_ERR_SHAPE;
  *bytes = csr_ws(num_edges, num_nodes).total;
  return ESA_OK;
}

int esa_csr_build(const int* keys, int64_t num_edges, int num_nodes, int* indptr, int* perm, void* workspace,
                  size_t workspace_bytes, void* stream) {
  return csr_build_impl(keys, num_edges, num_nodes, indptr, perm, workspace, workspace_bytes,
                        reinterpret_cast<hipStream_t>(stream), nullptr);
}

}  // extern "C"

int csr_build_impl(const int* keys, int64_t num_edges, int num_nodes, int* indptr, int* perm, void* workspace,
                   size_t workspace_bytes, hipStream_t st, const int* skip) {
  if (!indptr || !workspace || (num_edges > 0 && (!keys || !perm))) return ESA_ERR_NULL;
  if (num_edges < 0 || num_nodes < 0 || num_edges >= (1LL << 31)) return ESA_ERR_SHAPE;
  const CsrWs w = csr_ws(num_edges, num_nodes);
  if (workspace_bytes < w.total) return ESA_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  ESA_TIMED(esa_profile::kCsrBuild, st, {
    const int* sorted = nullptr;
    if (num_edges > 0) {
      // perm: stable radix sort of the edge ids by key
      const int ntiles = radix_blocks(num_edges), passes = radix_passes(num_nodes);
      const int nchunks = hist_chunks(ntiles);
      int* hist = reinterpret_cast<int*>(ws + w.hist);
      int* part = reinterpret_cast<int*>(ws + w.part);
      int* pairs[2] = {reinterpret_cast<int*>(ws + w.pairs_a), reinterpret_cast<int*>(ws + w.pairs_b)};
      int* skeys = pairs[(passes - 1) & 1];
      const bool vec_keys = !misaligned16(keys);
      for (int p = 0; p < passes; ++p) {
        const int shift = p * kRadixBits;
        const bool first = p == 0, last = p == passes - 1;
        const int* in = first ? keys : pairs[(p - 1) & 1];
        int* out = last ? skeys : pairs[p & 1];
        if (first)
          hipLaunchKernelGGL(radix_hist_kernel<false>, dim3(ntiles), dim3(kSortThreads), 0, st, in,
                             (long)num_edges, num_nodes, shift, vec_keys, hist, indptr, (long)num_nodes + 1, skip);
        else
          hipLaunchKernelGGL(radix_hist_kernel<true>, dim3(ntiles), dim3(kSortThreads), 0, st, in,
                             (long)num_edges, num_nodes, shift, true, hist, nullptr, 0L, skip);
        if (ntiles <= kSmallScanTiles) {
          hipLaunchKernelGGL(hist_scan_small_kernel, dim3(1), dim3(4 * kRadixBins), 0, st, hist, ntiles, skip);
        } else {
          hipLaunchKernelGGL(hist_chunk_sum_kernel, dim3(nchunks), dim3(kRadixBins), 0, st, hist, ntiles, part, skip);
          hipLaunchKernelGGL(hist_chunk_scan_kernel, dim3(1), dim3(4 * kRadixBins), 0, st, part, nchunks, skip);
          hipLaunchKernelGGL(hist_chunk_apply_kernel, dim3(nchunks), dim3(kRadixBins), 0, st, hist, ntiles,
                             part, skip);
        }
        auto scatter = first ? (last ? radix_scatter_kernel<false, false> : radix_scatter_kernel<false, true>)
                             : (last ? radix_scatter_kernel<true, false> : radix_scatter_kernel<true, true>);
        hipLaunchKernelGGL(scatter, dim3(ntiles), dim3(kSortThreads), 0, st, in, (long)num_edges, num_nodes,
                           shift, !first || vec_keys, hist, out, perm, skip);
      }
      sorted = skeys;
    }
    // indptr: the boundaries of the sorted keys' runs (set to -1 by the first histogram pass)
    if (num_edges == 0)
      hipLaunchKernelGGL(fill_int_kernel, dim3(grid_for((long)num_nodes + 1, 256, 4096)), dim3(256), 0, st, indptr,
                         (long)num_nodes + 1, -1, skip);
    hipLaunchKernelGGL(indptr_runs_kernel, dim3(grid_for(num_edges / 4 + 1, 256)), dim3(256), 0, st, sorted,
                       (long)num_edges, num_nodes, indptr, skip);
    hipLaunchKernelGGL(indptr_gap_kernel, dim3(grid_for((long)num_nodes + 1, 256, 4096)), dim3(256), 0, st,
                       sorted, (long)num_edges, num_nodes, indptr, skip);
  });
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

extern "C" {

int esa_csr_segment_sum(const void* y, const int* perm, const int* indptr, int num_nodes, int features, int dtype,
                        void* out, void* stream) {
  if (!indptr || !out || (!y && num_nodes > 0)) return ESA_ERR_NULL;
  if (num_nodes < 0 || features < 1) return ESA_ERR_SHAPE;
  if (dtype != ESA_F32 && dtype != ESA_BF16) return ESA_ERR_DTYPE;
  if (num_nodes == 0) return ESA_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == ESA_F32)
    return launch_segsum<float>(static_cast<const float*>(y), features, perm, indptr, 0, nullptr, nullptr, 0,
                                num_nodes, features, static_cast<float*>(out), st);
  return launch_segsum<bf16>(static_cast<const bf16*>(y), features, perm, indptr, 0, nullptr, nullptr, 0, num_nodes,
                             features, static_cast<bf16*>(out), st);
}

int esa_csr_segment_minmax(const void* y, const int* perm, const int* indptr, int num_nodes, int features, int dtype,
                           int is_max, int64_t num_edges, void* out, int64_t* arg, void* stream) {
  if (!indptr || !out || (!y && num_nodes > 0 && num_edges > 0)) return ESA_ERR_NULL;
  if (num_nodes < 0 || features < 1 || num_edges < 0) return ESA_ERR_SHAPE;
  if (dtype != ESA_F32 && dtype != ESA_BF16) return ESA_ERR_DTYPE;
  if (num_nodes == 0) return ESA_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const unsigned blocks = grid_for((long)num_nodes * features, 256);
  long long* a = reinterpret_cast<long long*>(arg);
  if (dtype == ESA_F32) {
    const float* yf = static_cast<const float*>(y);
    float* of = static_cast<float*>(out);
    if (is_max)
      ESA_TIMED(esa_profile::kSegmentMinMax, st,
                hipLaunchKernelGGL((segment_minmax_kernel<float, true>), dim3(blocks), dim3(256), 0, st, yf, perm,
                                   indptr, num_nodes, features, (long long)num_edges, of, a));
    else
      ESA_TIMED(esa_profile::kSegmentMinMax, st,
                hipLaunchKernelGGL((segment_minmax_kernel<float, false>), dim3(blocks), dim3(256), 0, st, yf, perm,
                                   indptr, num_nodes, features, (long long)num_edges, of, a));
  } else {
    const bf16* yb = static_cast<const bf16*>(y);
    bf16* ob = static_cast<bf16*>(out);
    if (is_max)
      ESA_TIMED(esa_profile::kSegmentMinMax, st,
                hipLaunchKernelGGL((segment_minmax_kernel<bf16, true>), dim3(blocks), dim3(256), 0, st, yb, perm,
                                   indptr, num_nodes, features, (long long)num_edges, ob, a));
    else
      ESA_TIMED(esa_profile::kSegmentMinMax, st,
                hipLaunchKernelGGL((segment_minmax_kernel<bf16, false>), dim3(blocks), dim3(256), 0, st, yb, perm,
                                   indptr, num_nodes, features, (long long)num_edges, ob, a));
  }
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

int esa_edge_gather_bwd(const void* g, const int* src_perm, const int* src_indptr, const int* dst_perm,
                        const int* dst_indptr, int num_nodes, int features, int dtype, void* gx, void* stream) {
  if (!g || !src_indptr || !dst_indptr || !gx) return ESA_ERR_NULL;
  if (num_nodes < 0 || features < 1) return ESA_ERR_SHAPE;
  if (dtype != ESA_F32 && dtype != ESA_BF16) return ESA_ERR_DTYPE;
  if (num_nodes == 0) return ESA_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const long ld = 2L * features;
  if (dtype == ESA_F32)
    return launch_segsum<float>(static_cast<const float*>(g), ld, src_perm, src_indptr, 0, dst_perm, dst_indptr,
                                features, num_nodes, features, static_cast<float*>(gx), st);
  return launch_segsum<bf16>(static_cast<const bf16*>(g), ld, src_perm, src_indptr, 0, dst_perm, dst_indptr, features,
                             num_nodes, features, static_cast<bf16*>(gx), st);
}

}  // extern "C"
