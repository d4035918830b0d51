// Internal interface of the node-mode (CSR adjacency) attention kernels; the
// C ABI entry points in esa_attn.hip dispatch here for ESA_MASK_NODE.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include "esa_common.h"

// Edge-mask plan sections the gather kernels read for ESA_MASK_EDGE(_PLAN) at
// head dims other than 16 (the plan's layout is esa_attn.hip's): per 32-token
// tile of direction d (0: queries, 1: keys) the partner count (-1 past the
// list capacity), kListCap partner ids and [kListCap / 32][32] mask words;
// the per-token node pairs and the flag word (1: symmetric plan, the key side
// reads direction 0).
struct GraphEdgeLists {
  const int* sym; const int2* nodes;
  const int* info[2]; const int* ids[2]; const uint32_t* bits[2];
  int cap;   // list capacity per tile
};

struct GraphAttnArgs {
  const void* q; const void* k; const void* v;
  const int* cu_q; const int* cu_k; int nseg;
  int total_q, total_k, heads, head_dim;
  const int* indptr; const int* indices; int nnz;   // CSR by query: keys of each query row
  float c, scale;                                   // c = softmax_scale * log2(e)
  void* out; float* lse;                            // forward outputs
  const void* out_in; const void* dout; const float* lse_in;   // backward inputs
  void* dq; void* dk; void* dv;                     // backward outputs
  float* dsum;                                      // backward workspace: D_i per head
  const int* t_indptr; const int* t_rows;           // transposed CSR: per key, the query rows listing it
  const int4* q_desc; const int4* k_desc;           // per-token {lo, hi, pa, pb} from a node plan, or null
  const int2* q_bounds; const int2* k_bounds;       // edge lists: per-token partner range (the plan's bounds)
  GraphEdgeLists edge;                              // edge lists (edge.ids[0] non-null): the mask's partners
  DropoutCfg drop; bool dropout;                    // attention dropout (esa_common.h) when `dropout`
};

// Head dims of the gather kernels.
inline bool graph_head_dim_ok(int hd) { return hd == 16 || hd == 24 || hd == 32 || hd == 64; }

// Edge-mask attention over a plan's lists (a.edge set, a.q_bounds / k_bounds
// the plan's bounds): the same gather kernels with the partners of a token
// read from its tile's list (mask bits) or, for a tile past the list
// capacity, from the share-an-endpoint predicate over its segment.
int graph_edge_attn_fwd(GraphAttnArgs a, int dtype, hipStream_t st);
// workspace: graph_attn_workspace_size(total_q, total_k, heads, 0, true, true).
int graph_edge_attn_bwd(GraphAttnArgs a, int dtype, void* workspace, size_t workspace_bytes, hipStream_t st);

// planned: the transposed CSR comes from a node plan (mask_b of
// ESA_MASK_NODE_PLAN) instead of being built in the workspace.
int graph_attn_workspace_size(int total_q, int total_k, int heads, int nnz, bool backward, bool planned,
                              size_t* bytes);
// plan: null, or a node plan whose query descriptors the forward reads.
int graph_attn_fwd(GraphAttnArgs a, int dtype, const void* plan, hipStream_t st);
// plan: null, or a node plan whose transposed CSR the backward reads.
int graph_attn_bwd(GraphAttnArgs a, int dtype, const void* plan, void* workspace, size_t workspace_bytes,
                   hipStream_t st);
int graph_node_plan_size(int total_q, int total_k, int nnz, size_t* bytes);
// Byte offsets of a node plan's sections: indices, t_indptr, t_rows, q_desc, k_desc.
int graph_node_plan_sections(int total_q, int total_k, int nnz, size_t offsets[5]);
int graph_node_plan_build(const int* indptr, const int* indices, const int* cu_q, const int* cu_k, int nseg,
                          int total_q, int total_k, int nnz, void* plan, size_t plan_bytes, hipStream_t st);
