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
DEVI float4 chunk_f32(u32x4 v, int k);   // elements 4k..4k+3 of a 16-byte chunk as fp32
template <>
DEVI float4 chunk_f32<float>(u32x4 v, int k) {
  (void)k;
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
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

__global__ void zero_int_kernel(int* __restrict__ p, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) p[i] = 0;
}

__global__ void count_keys_kernel(const int* __restrict__ keys, long num_edges, int num_nodes,
                                  int* __restrict__ counts) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < num_edges; i += (long)gridDim.x * blockDim.x) {
    const int k = keys[i];
    if ((unsigned)k < (unsigned)num_nodes) atomicAdd(&counts[k], 1);
  }
}

constexpr int kScanBlock = 1024;
constexpr int kScanItems = 4;  // per thread
constexpr int kScanTile = kScanBlock * kScanItems;

// Block-wide exclusive scan of one value per thread (Hillis-Steele in LDS).
DEVI int block_exclusive_scan(int v, int* sh, int& total) {
  const int tid = threadIdx.x;
  sh[tid] = v;
  __syncthreads();
  for (int off = 1; off < kScanBlock; off <<= 1) {
    const int add = tid >= off ? sh[tid - off] : 0;
    __syncthreads();
    sh[tid] += add;
    __syncthreads();
  }
  total = sh[kScanBlock - 1];
  const int incl = sh[tid];
  __syncthreads();
  return incl - v;
}

// Pass 1: per-tile sums of counts[0..n).
__global__ __launch_bounds__(kScanBlock) void scan_reduce_kernel(const int* __restrict__ in, int n,
                                                                 int* __restrict__ tile_sums) {
  __shared__ int sh[kScanBlock];
  const int base = blockIdx.x * kScanTile + threadIdx.x * kScanItems;
  int s = 0;
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) s += base + j < n ? in[base + j] : 0;
  int total;
  block_exclusive_scan(s, sh, total);
  if (threadIdx.x == 0) tile_sums[blockIdx.x] = total;
}

// Pass 2: exclusive scan of the tile sums in one block (loops over chunks).
__global__ __launch_bounds__(kScanBlock) void scan_tiles_kernel(int* __restrict__ tile_sums, int ntiles) {
  __shared__ int sh[kScanBlock];
  int carry = 0;
  for (int base = 0; base < ntiles; base += kScanBlock) {
    const int i = base + threadIdx.x;
    const int v = i < ntiles ? tile_sums[i] : 0;
    int total;
    const int ex = block_exclusive_scan(v, sh, total);
    if (i < ntiles) tile_sums[i] = carry + ex;
    carry += total;
  }
}

// Pass 3: indptr[i] = exclusive prefix of counts, indptr[n] = total;
// cursor[i] = indptr[i] (fill cursor).
__global__ __launch_bounds__(kScanBlock) void scan_apply_kernel(const int* __restrict__ in, int n,
                                                                const int* __restrict__ tile_offsets,
                                                                int* __restrict__ indptr,
                                                                int* __restrict__ cursor) {
  __shared__ int sh[kScanBlock];
  const int base = blockIdx.x * kScanTile + threadIdx.x * kScanItems;
  int v[kScanItems];
  int s = 0;
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) { v[j] = base + j < n ? in[base + j] : 0; s += v[j]; }
  int total;
  int run = block_exclusive_scan(s, sh, total) + tile_offsets[blockIdx.x];
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) {
    if (base + j < n) { indptr[base + j] = run; cursor[base + j] = run; }
    run += v[j];
  }
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == kScanBlock - 1) indptr[n] = run;
}

// perm by a stable LSD radix sort of (key, edge id) over 8-bit digits, so
// every edge's position follows from counts alone (no atomic ordering, no
// per-segment sort): per pass, each block counts the digits of its tile of
// kSortTile consecutive edges (hist, digit-major: [digit][block]); an
// exclusive scan of hist in that (digit, block) order gives each (digit,
// block) its first output slot; the scatter pass then places element i of
// the tile at that slot + the number of earlier elements of the tile with the
// same digit.  Earlier means earlier in edge order: the tile is walked in
// rounds j of kSortThreads consecutive edges (edge base + j * 256 + tid), and
// inside a round by wave, then lane.  Each pass is therefore stable, and the
// passes over digits 0, 1, ... leave the edges sorted by key with ties in
// ascending edge id.  Keys outside [0, num_nodes) sort as num_nodes, after
// every valid key (past indptr[num_nodes]).
constexpr int kSortThreads = 256;
constexpr int kSortItems = 16;
constexpr int kSortTile = kSortThreads * kSortItems;
constexpr int kRadixBits = 8;
constexpr int kRadixBins = 1 << kRadixBits;
static_assert(kRadixBins == kSortThreads, "one digit per thread in the per-digit steps");

DEVI int sort_key(const int* __restrict__ keys, long i, int num_nodes, bool raw) {
  const int k = keys[i];
  return !raw || (unsigned)k < (unsigned)num_nodes ? k : num_nodes;
}

__global__ __launch_bounds__(kSortThreads) void radix_hist_kernel(const int* __restrict__ keys, long n, int num_nodes,
                                                                 bool raw, int shift, int nblocks,
                                                                 int* __restrict__ hist) {
  __shared__ int h[kRadixBins];
  const int tid = threadIdx.x;
  h[tid] = 0;
  __syncthreads();
  const long base = (long)blockIdx.x * kSortTile;
#pragma unroll 4
  for (int j = 0; j < kSortItems; ++j) {
    const long i = base + (long)j * kSortThreads + tid;
    if (i < n) atomicAdd(&h[(sort_key(keys, i, num_nodes, raw) >> shift) & (kRadixBins - 1)], 1);
  }
  __syncthreads();
  hist[(long)tid * nblocks + blockIdx.x] = h[tid];
}

// offsets: the exclusive scan of hist.  vals_in null: the values are the edge
// ids.  keys_out null: the last pass (only the values are needed).
__global__ __launch_bounds__(kSortThreads) void radix_scatter_kernel(const int* __restrict__ keys_in,
                                                                    const int* __restrict__ vals_in, long n,
                                                                    int num_nodes, bool raw, int shift, int nblocks,
                                                                    const int* __restrict__ offsets,
                                                                    int* __restrict__ keys_out,
                                                                    int* __restrict__ vals_out) {
  constexpr int kWaves = kSortThreads / 64;
  __shared__ int run[kRadixBins];           // next slot of each digit
  __shared__ int wcnt[kWaves][kRadixBins];  // this round's count of each digit per wave
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  run[tid] = offsets[(long)tid * nblocks + blockIdx.x];
#pragma unroll
  for (int w = 0; w < kWaves; ++w) wcnt[w][tid] = 0;
  __syncthreads();
  const long base = (long)blockIdx.x * kSortTile;
  const uint64_t below_mask = (1ull << lane) - 1;
  for (int j = 0; j < kSortItems; ++j) {
    const long i = base + (long)j * kSortThreads + tid;
    const bool valid = i < n;
    int k = 0, v = 0, d = 0;
    if (valid) {
      k = sort_key(keys_in, i, num_nodes, raw);
      v = vals_in ? vals_in[i] : (int)i;
      d = (k >> shift) & (kRadixBins - 1);
    }
    // lanes of this wave holding the same digit
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < kRadixBits; ++b) {
      const bool bit = (d >> b) & 1;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const int below = __popcll(peers & below_mask);
    if (valid && below == 0) wcnt[wave][d] = __popcll(peers);
    __syncthreads();
    if (valid) {
      int pos = run[d] + below;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) pos += w < wave ? wcnt[w][d] : 0;
      if (keys_out) keys_out[pos] = k;
      vals_out[pos] = v;
    }
    __syncthreads();
    int add = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) { add += wcnt[w][tid]; wcnt[w][tid] = 0; }
    run[tid] += add;
    __syncthreads();
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

unsigned grid_for(long n, int block, long cap = 1L << 20) {
  long g = (n + block - 1) / block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (unsigned)g;
}

bool misaligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) != 0; }

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Exclusive scan of in[0, n) into out[0, n] (out[n] = the total); in may be out.
void scan_exclusive(const int* in, int n, int* out, int* tiles, hipStream_t st) {
  const int ntiles = (n + kScanTile - 1) / kScanTile;
  hipLaunchKernelGGL(scan_reduce_kernel, dim3(ntiles), dim3(kScanBlock), 0, st, in, n, tiles);
  hipLaunchKernelGGL(scan_tiles_kernel, dim3(1), dim3(kScanBlock), 0, st, tiles, ntiles);
  hipLaunchKernelGGL(scan_apply_kernel, dim3(ntiles), dim3(kScanBlock), 0, st, in, n, tiles, out, out);
}

int radix_blocks(int64_t num_edges) { return (int)((num_edges + kSortTile - 1) / kSortTile); }

// Passes of kRadixBits over the keys 0 .. num_nodes (num_nodes: the slot of invalid keys).
int radix_passes(int num_nodes) {
  const int bits = 32 - __builtin_clz((unsigned)num_nodes | 1u);
  return (bits + kRadixBits - 1) / kRadixBits;
}

struct CsrWs { size_t counts, tiles, hist, keys_a, keys_b, vals, total; };
CsrWs csr_ws(int64_t num_edges, int num_nodes) {
  CsrWs w;
  const long nhist = (long)kRadixBins * radix_blocks(num_edges);
  const long scan_n = std::max((long)num_nodes, nhist);
  const long ntiles = (scan_n + kScanTile - 1) / kScanTile;
  size_t off = 0;
  w.counts = off; off += align256((size_t)num_nodes * 4);
  w.tiles = off; off += align256((size_t)(ntiles > 0 ? ntiles : 1) * 4);
  w.hist = off; off += align256((size_t)(nhist + 1) * 4);
  w.keys_a = off; off += align256((size_t)num_edges * 4);
  w.keys_b = off; off += align256((size_t)num_edges * 4);
  w.vals = off; off += align256((size_t)num_edges * 4);
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
  if (!indptr || !workspace || (num_edges > 0 && (!keys || !perm))) return ESA_ERR_NULL;
  if (num_edges < 0 || num_nodes < 0 || num_edges >= (1LL << 31)) return ESA_ERR_SHAPE;
  const CsrWs w = csr_ws(num_edges, num_nodes);
  if (workspace_bytes < w.total) return ESA_ERR_WORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  int* counts = reinterpret_cast<int*>(ws + w.counts);
  int* tiles = reinterpret_cast<int*>(ws + w.tiles);
  if (num_nodes == 0) {
    hipLaunchKernelGGL(zero_int_kernel, dim3(1), dim3(64), 0, st, indptr, 1L);
    ESA_LAUNCH_CHECK();
    return ESA_OK;
  }
  ESA_TIMED(esa_profile::kCsrBuild, st, {
    // indptr: key counts (order-independent) and their exclusive scan
    hipLaunchKernelGGL(zero_int_kernel, dim3(grid_for(num_nodes, 256, 4096)), dim3(256), 0, st, counts,
                       (long)num_nodes);
    if (num_edges > 0)
      hipLaunchKernelGGL(count_keys_kernel, dim3(grid_for(num_edges, 256, 8192)), dim3(256), 0, st, keys,
                         (long)num_edges, num_nodes, counts);
    scan_exclusive(counts, num_nodes, indptr, tiles, st);
    // perm: stable radix sort of the edge ids by key
    if (num_edges > 0) {
      const int nblocks = radix_blocks(num_edges), passes = radix_passes(num_nodes);
      int* hist = reinterpret_cast<int*>(ws + w.hist);
      int* kbuf[2] = {reinterpret_cast<int*>(ws + w.keys_a), reinterpret_cast<int*>(ws + w.keys_b)};
      int* vtmp = reinterpret_cast<int*>(ws + w.vals);
      const int* kin = keys;
      const int* vin = nullptr;
      for (int p = 0; p < passes; ++p) {
        const bool raw = p == 0, last = p == passes - 1;
        // values ping-pong so that the last pass writes perm
        int* vout = ((passes - 1 - p) & 1) ? vtmp : perm;
        int* kout = last ? nullptr : kbuf[p & 1];
        hipLaunchKernelGGL(radix_hist_kernel, dim3(nblocks), dim3(kSortThreads), 0, st, kin, (long)num_edges,
                           num_nodes, raw, p * kRadixBits, nblocks, hist);
        scan_exclusive(hist, kRadixBins * nblocks, hist, tiles, st);
        hipLaunchKernelGGL(radix_scatter_kernel, dim3(nblocks), dim3(kSortThreads), 0, st, kin, vin,
                           (long)num_edges, num_nodes, raw, p * kRadixBits, nblocks, hist, kout, vout);
        kin = kout;
        vin = vout;
      }
    }
  });
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

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
