// Internal interface of the segment-tiled dense (unmasked) bf16 attention
// kernels; the C ABI entry points in esa_attn.hip dispatch here for
// ESA_MASK_NONE with ESA_BF16.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include "esa_common.h"

struct DenseAttnCall {
  const void* q; const void* k; const void* v;
  const int* cu_q; const int* cu_k; int nseg;
  int total_q, total_k, heads, head_dim;
  float scale;
  void* out; float* lse;                             // forward outputs
  const void* out_in; const void* dout; const float* lse_in;   // backward inputs
  void* dq; void* dk; void* dv;                      // backward outputs
  DropoutCfg drop; bool dropout;                     // attention dropout (esa_common.h) when `dropout`
};

// head_dim 16 without dropout: the kernels of esa_attn_dense.hip; 24, 32, 64
// and every head dim with dropout: esa_attn_wide.hip.  The workspace size
// covers both.
int dense_attn_workspace_size(int total_q, int total_k, int heads, int head_dim, bool backward, size_t* bytes);
int dense_attn_fwd(const DenseAttnCall& c, void* workspace, size_t workspace_bytes, hipStream_t st);
int dense_attn_bwd(const DenseAttnCall& c, void* workspace, size_t workspace_bytes, hipStream_t st);

// The head-dim 32 / 64 kernels (esa_attn_wide.hip).
size_t wide_attn_workspace_size(int total_q, int total_k, int heads, int head_dim, bool backward);
int wide_attn_fwd(const DenseAttnCall& c, void* workspace, size_t workspace_bytes, hipStream_t st);
int wide_attn_bwd(const DenseAttnCall& c, void* workspace, size_t workspace_bytes, hipStream_t st);
