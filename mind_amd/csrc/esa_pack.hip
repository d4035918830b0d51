// Token-budget batching of consecutive graphs on the device.
//
// The rule of ImprovedDynamicBatchSampler._create_batches_standard
// (data_loading/improved_dynamic_sampler.py:215-224): walk the graphs in
// order; a graph whose count would push the open batch past the budget
// closes that batch and opens the next one, unless the open batch is empty
// (an oversize graph gets a batch of its own).  Counts here are the tokens
// each graph contributes (edges for edge-set attention).
//
// The walk is sequential in the reference; on the device it is a pointer
// chase made parallel by doubling.  With P the exclusive prefix of the
// counts, a batch opened at graph i holds graphs i .. j(i) - 1 where
// j(i) = max(i + 1, (first x with P[x] > P[i] + budget) - 1), found by a
// binary search; the batch starts are the chain 0, j(0), j(j(0)), ... .
// Round r marks every start reachable from a marked one through j^(2^r) and
// squares the jump table, so after ceil(log2 G) rounds every start of the
// chain is marked (the first 2^(r+1) starts after round r; a mark seen early
// is still a start, so the racy reads only speed it up).  A scan of the marks
// then numbers the batches.  One block does all of it: graph lists are small
// (a dataset epoch) and the rounds need block-wide barriers.
#include "esa_common.h"
#include "esa_profile.h"
#include "../../include/esa_hip.h"

namespace {

constexpr int kPackThreads = 1024;
constexpr int kPackItems = 8;                       // consecutive items per thread in the scans
constexpr int kPackChunk = kPackThreads * kPackItems;

// Block-wide inclusive scan of one int64 per thread (Hillis-Steele in LDS);
// returns the inclusive value and the block total.
DEVI long long block_scan_incl(long long v, long long* sh, long long& total) {
  const int tid = threadIdx.x;
  sh[tid] = v;
  __syncthreads();
  for (int off = 1; off < kPackThreads; off <<= 1) {
    const long long add = tid >= off ? sh[tid - off] : 0;
    __syncthreads();
    sh[tid] += add;
    __syncthreads();
  }
  const long long incl = sh[tid];
  total = sh[kPackThreads - 1];
  __syncthreads();
  return incl;
}

__global__ __launch_bounds__(kPackThreads) void pack_kernel(const int* __restrict__ counts, int G, long long budget,
                                                          long long* __restrict__ prefix, int* __restrict__ jump_a,
                                                          int* __restrict__ jump_b, volatile int* flag,
                                                          int* __restrict__ batch_of_graph,
                                                          int* __restrict__ batch_start, int* __restrict__ num_batches) {
  __shared__ long long sh[kPackThreads];
  const int tid = threadIdx.x;
  // exclusive prefix P[0..G] of the counts (negative counts count as 0)
  long long carry = 0;
  for (int base = 0; base < G; base += kPackChunk) {
    const int i0 = base + tid * kPackItems;
    long long loc[kPackItems], s = 0;
#pragma unroll
    for (int j = 0; j < kPackItems; ++j) {
      loc[j] = s;
      s += i0 + j < G ? (long long)max(counts[i0 + j], 0) : 0;
    }
    long long total;
    const long long ex = block_scan_incl(s, sh, total) - s + carry;
#pragma unroll
    for (int j = 0; j < kPackItems; ++j)
      if (i0 + j < G) prefix[i0 + j] = ex + loc[j];
    carry += total;
  }
  if (tid == 0) prefix[G] = carry;
  __syncthreads();
  // jump table j(i) and the first mark
  for (int i = tid; i <= G; i += kPackThreads) {
    int nxt = G;
    if (i < G) {
      const long long lim = prefix[i] + budget;
      int lo = i + 1, hi = G + 1;   // first x in [i + 1, G + 1) with prefix[x] > lim, else G + 1
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (prefix[mid] > lim) hi = mid; else lo = mid + 1;
      }
      nxt = max(i + 1, lo - 1);
    }
    jump_a[i] = nxt;
    flag[i] = i == 0 ? 1 : 0;
  }
  __syncthreads();
  int* jump = jump_a;
  int* jump_next = jump_b;
  for (long long span = 1; span < G; span <<= 1) {
    for (int i = tid; i < G; i += kPackThreads)
      if (flag[i]) flag[jump[i]] = 1;
    __syncthreads();
    for (int i = tid; i <= G; i += kPackThreads) jump_next[i] = jump[jump[i]];
    __syncthreads();
    int* t = jump; jump = jump_next; jump_next = t;
  }
  // number the batches: inclusive scan of the marks
  carry = 0;
  for (int base = 0; base < G; base += kPackChunk) {
    const int i0 = base + tid * kPackItems;
    int f[kPackItems];
    long long s = 0;
#pragma unroll
    for (int j = 0; j < kPackItems; ++j) {
      f[j] = i0 + j < G ? flag[i0 + j] : 0;
      s += f[j];
    }
    long long total;
    long long id = block_scan_incl(s, sh, total) - s + carry;
#pragma unroll
    for (int j = 0; j < kPackItems; ++j) {
      if (i0 + j >= G) break;
      id += f[j];
      batch_of_graph[i0 + j] = (int)id - 1;
      if (f[j]) batch_start[id - 1] = i0 + j;
    }
    carry += total;
  }
  if (tid == 0) {
    batch_start[carry] = G;
    *num_batches = (int)carry;
  }
}

size_t a256(size_t x) { return (x + 255) & ~size_t(255); }

struct PackWs { size_t prefix, jump_a, jump_b, flag, total; };
PackWs pack_ws(int G) {
  PackWs w;
  size_t off = 0;
  w.prefix = off; off += a256((size_t)(G + 1) * 8);
  w.jump_a = off; off += a256((size_t)(G + 1) * 4);
  w.jump_b = off; off += a256((size_t)(G + 1) * 4);
  w.flag = off; off += a256((size_t)(G + 1) * 4);
  w.total = off;
  return w;
}

}  // namespace

extern "C" {

int esa_token_budget_pack_workspace_size(int num_graphs, size_t* bytes) {
  if (!bytes) return ESA_ERR_NULL;
  if (num_graphs < 0 || num_graphs >= (1 << 30)) return ESA_ERR_SHAPE;
  *bytes = pack_ws(num_graphs).total;
  return ESA_OK;
}

int esa_token_budget_pack(const int* counts, int num_graphs, int64_t budget, int* batch_of_graph, int* batch_start,
                          int* num_batches, void* workspace, size_t workspace_bytes, void* stream) {
  if (!batch_start || !num_batches || !workspace) return ESA_ERR_NULL;
  if (num_graphs > 0 && (!counts || !batch_of_graph)) return ESA_ERR_NULL;
  if (num_graphs < 0 || num_graphs >= (1 << 30)) return ESA_ERR_SHAPE;
  const PackWs w = pack_ws(num_graphs);
  if (workspace_bytes < w.total) return ESA_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(pack_kernel, dim3(1), dim3(kPackThreads), 0, st, counts, num_graphs, (long long)budget,
                     reinterpret_cast<long long*>(ws + w.prefix), reinterpret_cast<int*>(ws + w.jump_a),
                     reinterpret_cast<int*>(ws + w.jump_b), reinterpret_cast<volatile int*>(ws + w.flag),
                     batch_of_graph, batch_start, num_batches);
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

}  // extern "C"
