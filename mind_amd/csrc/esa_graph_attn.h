// Internal interface of the node-mode (CSR adjacency) attention kernels; the
// C ABI entry points in esa_attn.hip dispatch here for ESA_MASK_NODE.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>

constexpr int kHd16 = 16;   // head_dim of every ESA attention kernel

struct GraphAttnArgs {
  const void* q; const void* k; const void* v;
  const int* cu_q; const int* cu_k; int nseg;
  int total_q, total_k, heads;
  const int* indptr; const int* indices; int nnz;   // CSR by query: keys of each query row
  float c, scale;                                   // c = softmax_scale * log2(e)
  void* out; float* lse;                            // forward outputs
  const void* out_in; const void* dout; const float* lse_in;   // backward inputs
  void* dq; void* dk; void* dv;                     // backward outputs
  float* dsum; int* row_of; int* t_indptr; int* t_perm;         // backward workspace
};

int graph_attn_workspace_size(int total_q, int total_k, int heads, int nnz, bool backward, size_t* bytes);
int graph_attn_fwd(GraphAttnArgs a, int dtype, hipStream_t st);
int graph_attn_bwd(GraphAttnArgs a, int dtype, void* workspace, size_t workspace_bytes, hipStream_t st);
