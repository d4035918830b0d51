/*
 * esa_hip.h — C ABI of the MI355X (gfx950) edge-set-attention hot path.
 *
 * Conventions shared by every entry point:
 *   - Every pointer is a device pointer to a caller-allocated buffer.  The
 *     library never allocates, frees or synchronises; scratch memory is passed
 *     in as `workspace`, sized by the matching *_workspace_size() query.
 *   - Work is enqueued on `stream` (a hipStream_t passed as void*).
 *   - Return value: 0 on success, a negative ESA_ERR_* code for an argument
 *     error (nothing is launched), or a positive hipError_t from the launch.
 *   - Token tensors are packed: [total, heads, head_dim] contiguous, one
 *     segment (graph) after another, with int32 cu_seqlens [batch + 1].
 *   - Features are bf16 (ESA_BF16) or fp32 (ESA_F32) as each entry point says;
 *     indices and offsets are int32.
 */
#ifndef ESA_HIP_H
#define ESA_HIP_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define ESA_API __attribute__((visibility("default")))
#else
#define ESA_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define ESA_OK 0
#define ESA_ERR_NULL (-1)       /* a required pointer is null */
#define ESA_ERR_SHAPE (-2)      /* a size or count is out of range */
#define ESA_ERR_HEAD_DIM (-3)   /* head_dim other than 16, 24, 32 or 64 */
#define ESA_ERR_WORKSPACE (-4)  /* workspace smaller than the query says */
#define ESA_ERR_DTYPE (-5)      /* unsupported dtype code */
#define ESA_ERR_ALIGN (-6)      /* pointer not 16-byte aligned */
#define ESA_ERR_MASK (-7)       /* unknown mask kind, or the edge mask without total_q == total_k */
#define ESA_ERR_SCRATCH (-8)    /* the call needs more scratch than esa_noalloc_scratch_bytes() */
#define ESA_ERR_DROPOUT (-9)    /* dropout_p outside [0, 1) */

#define ESA_F32 0
#define ESA_BF16 1

/* Attention mask kinds (see esa_varlen_attn_fwd). */
#define ESA_MASK_NONE 0
#define ESA_MASK_EDGE 1
#define ESA_MASK_NODE 2
#define ESA_MASK_EDGE_PLAN 3
#define ESA_MASK_NODE_PLAN 4

/* Library version and build target, e.g. "esa_hip 0.1 gfx950". */
ESA_API const char* esa_version(void);

/* ------------------------------------------------------------------------ */
/* Varlen attention over packed segments.                                    */
/*                                                                           */
/* Replaces flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k,      */
/* max_seqlen_q, max_seqlen_k, dropout_p, softmax_scale, causal=False)       */
/* called at esa/mha_flash_varlen.py:177-184, and the per-graph attention of */
/* memory_efficient_attention / SDPA at esa/mha.py:76 and :80-83.            */
/*                                                                           */
/* q [total_q, heads, head_dim], k and v [total_k, heads, head_dim], out     */
/* like q, all of `dtype`: ESA_BF16 (bf16 MFMA, fp32 softmax; the bf16-mixed */
/* training path) or ESA_F32 (fp32 throughout; the reference's fp32          */
/* modules).  head_dim is 16, 24, 32 or 64 (dim / num_heads of every MIND    */
/* configuration, esa/mha.py:50-52).                                         */
/*                                                                           */
/* mask_kind ESA_MASK_EDGE: mask_a / mask_b are the per-token endpoint node  */
/* ids src / dst [total_q] (self-attention, total_q == total_k, same         */
/* cu_seqlens); query token i attends to key token j of the same segment iff */
/* i != j and {src_i, dst_i} and {src_j, dst_j} share a node — the predicate */
/* of create_edge_adjacency_mask (esa/masked_layers.py:121-142) that          */
/* get_adj_mask_from_edge_index_edge (:217-268) turns into a 0 / -99999      */
/* bias.  No E x E mask is stored: the call builds an edge-mask plan (below) */
/* in its workspace.  n_mask_edges is unused.                                */
/*                                                                           */
/* mask_kind ESA_MASK_EDGE_PLAN: the same mask from a plan built once by     */
/* esa_edge_plan_build with the same cu_seqlens pointers; mask_a = the plan */
/* (cast), mask_b unused.  ESA_MASK_NONE: mask_a, mask_b unused.             */
/*                                                                           */
/* mask_kind ESA_MASK_NODE: a CSR adjacency by query, mask_a = indptr        */
/* [total_q + 1], mask_b = indices [n_mask_edges] (key token ids); query i   */
/* attends to keys mask_b[mask_a[i] .. mask_a[i+1]) — the mask               */
/* get_adj_mask_from_edge_index_node (esa/masked_layers.py:79-118) encodes   */
/* as bias[b, src, dst] = 0 per edge src -> dst (query = src).  Each row     */
/* lists its keys in ascending order; an entry equal to its predecessor      */
/* counts once (a repeated edge); entries outside the query's segment are    */
/* ignored.  Work is O(n_mask_edges * heads * head_dim).                     */
/*                                                                           */
/* mask_kind ESA_MASK_NODE_PLAN: the same mask with mask_b = a node plan     */
/* built once by esa_node_plan_build from (mask_a, indices): its first       */
/* n_mask_edges ints are a copy of the indices, followed by the transposed   */
/* CSR the backward reads, so the backward does not rebuild it per call.     */
/*                                                                           */
/* A query with no admissible key gets output 0 and lse = -inf.              */
/*                                                                           */
/* max_seqlen_q / max_seqlen_k never change a result.  max_seqlen_q selects */
/* a route: unmasked ESA_F32 calls with 1 <= max_seqlen_q <= 4 (the PMA's   */
/* seeds) take kernels with one wave per (segment, query, head) that walk   */
/* every query of a segment whatever the value, so a value below the true   */
/* maximum costs time, not correctness.                                     */
/*                                                                           */
/* dropout_p in [0, 1): attention dropout on the softmax probabilities, as   */
/* the reference's p / dropout_p in training (esa/mha.py:76,82): out =       */
/* (P o Z s) V with the keep mask Z a counter-based hash of (dropout_seed,   */
/* head, query token, key token) — query q keeps key k in head h iff         */
/* half(fmix32(row(q, h) ^ col(k)), k mod 2) >= thr, row(q, h) =             */
/* fmix32(s0 ^ fmix32(q heads + h)), col(k) = fmix32(s1 ^ fmix32(k / 2))     */
/* (integer division: keys 2i and 2i + 1 share one hash), half(x, 0) / (x, 1) */
/* its low / high 16 bits, thr = round(dropout_p 2^16) capped at 2^16 - 1,   */
/* s = 2^16 / (2^16 - thr) (1 / (1 - dropout_p) with dropout_p quantised to  */
/* 2^-16), s0 / s1 the seed's low / high words (s1 xor 0x9E3779B9), fmix32   */
/* MurmurHash3's 32-bit finalizer, q and k the global token indices.         */
/* softmax_lse is that of the undropped scores.  The backward takes the same */
/* dropout_p and seed.  0 disables dropout (the seed is then unused).        */
/*                                                                           */
/* softmax_lse is [heads, total_q] fp32 (natural log), as flash-attn's.      */
/* ------------------------------------------------------------------------ */
/* ------------------------------------------------------------------------ */
/* Edge-mask plan: the per-batch data of the ESA_MASK_EDGE mask (packed node */
/* pairs, per-tile node metadata, per-token segment bounds, and per 32-token */
/* tile the union of its admissible partners with one mask bit per token and */
/* partner), built once and read by every attention call over the same       */
/* tokens and segments.  It replaces the [B, N, N] bias that                 */
/* get_adj_mask_from_edge_index_edge (esa/masked_layers.py:217-268) builds   */
/* once per batch and every masked layer reads (esa/masked_layers.py:849-    */
/* 936).  `symmetric`: the attention calls pass one pointer as both          */
/* cu_seqlens (self-attention over one segment array); otherwise the plan   */
/* also holds the key tiles' lists.  The build uses the pointer equality of  */
/* its own cu_seqlens arguments; later calls must pass the same arrays.      */
/* The plan stays valid while tok_src / tok_dst / cu_seqlens are unchanged.  */
/* ------------------------------------------------------------------------ */
ESA_API int esa_edge_plan_size(int total_q, int total_k, int symmetric, size_t* bytes);
ESA_API int esa_edge_plan_build(const int* tok_src, const int* tok_dst,
                        const int* cu_seqlens_q, const int* cu_seqlens_k,
                        int batch, int total_q, int total_k,
                        void* plan, size_t plan_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Node-mode plan: the per-batch data of the ESA_MASK_NODE mask, i.e. a copy */
/* of the CSR's indices and the transposed CSR (per key token, the query     */
/* rows that list it, in ascending position) that the backward's dK / dV    */
/* pass gathers over, and per query and key token its partner range and row */
/* bounds (from cu_seqlens).  Built once per batch and read by every        */
/* attention call over the same adjacency, as the reference builds its       */
/* [B, 1, N, N]                                                              */
/* node bias once per batch (get_adj_mask_from_edge_index_node,             */
/* esa/masked_layers.py:79-118) for all its layers (:849-936).  The plan's   */
/* tail is the build's scratch.  It stays valid while indptr / indices and   */
/* the cu_seqlens are unchanged; calls pass the same indptr as mask_a, the   */
/* same cu_seqlens, and the total_q, total_k and n_mask_edges it was built   */
/* with (the call locates the plan's sections from them; the plan is not     */
/* read back to check).  With one cu_seqlens pointer for queries and keys    */
/* and total_q == total_k, a CSR that is its own transpose (ascending rows,  */
/* each entry (i, j) matched by as many (j, i); undirected graphs) is found  */
/* so on the device and copied instead of sorted: the same plan, fewer       */
/* cycles.                                                                   */
/* ------------------------------------------------------------------------ */
ESA_API int esa_node_plan_size(int total_q, int total_k, int n_mask_edges, size_t* bytes);
ESA_API int esa_node_plan_build(const int* indptr, const int* indices,
                        const int* cu_seqlens_q, const int* cu_seqlens_k, int batch,
                        int total_q, int total_k, int n_mask_edges,
                        void* plan, size_t plan_bytes, void* stream);

ESA_API int esa_varlen_attn_workspace_size(int total_q, int total_k, int heads,
                                   int head_dim, int dtype, int mask_kind,
                                   int n_mask_edges, int backward,
                                   size_t* bytes);

ESA_API int esa_varlen_attn_fwd(const void* q, const void* k, const void* v,
                        const int* cu_seqlens_q, const int* cu_seqlens_k,
                        int batch, int total_q, int total_k,
                        int max_seqlen_q, int max_seqlen_k,
                        int heads, int head_dim, int dtype, float softmax_scale,
                        float dropout_p, unsigned long long dropout_seed,
                        int mask_kind, const int* mask_a, const int* mask_b,
                        int n_mask_edges,
                        void* out, float* softmax_lse,
                        void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* No-allocation forward.  No counterpart in the reference: it is for        */
/* callers that cannot allocate device memory (code under HIP graph capture, */
/* tight serving loops, harnesses that forbid hipMalloc).  Same arguments     */
/* and results as esa_varlen_attn_fwd without the workspace: the scratch is  */
/* a static device array of esa_noalloc_scratch_bytes() (16 MiB) per GPU,    */
/* held until the process ends, enough for every ESA shape up to 131,072      */
/* tokens x 32 heads (any mask kind).  A call needing more returns            */
/* ESA_ERR_SCRATCH and launches nothing.  The caller still passes the inputs */
/* and outputs; nothing is allocated or freed.  All calls on one GPU share   */
/* that GPU's scratch: calls that overlap in time on one GPU (other streams, */
/* other host threads without ordering) race and must be serialised by the  */
/* caller.                                                                   */
/* ------------------------------------------------------------------------ */
ESA_API size_t esa_noalloc_scratch_bytes(void);
ESA_API int esa_varlen_attn_fwd_noalloc(const void* q, const void* k, const void* v,
                        const int* cu_seqlens_q, const int* cu_seqlens_k,
                        int batch, int total_q, int total_k,
                        int max_seqlen_q, int max_seqlen_k,
                        int heads, int head_dim, int dtype, float softmax_scale,
                        float dropout_p, unsigned long long dropout_seed,
                        int mask_kind, const int* mask_a, const int* mask_b,
                        int n_mask_edges,
                        void* out, float* softmax_lse, void* stream);

/* Gradients of esa_varlen_attn_fwd; replaces flash-attn's varlen backward. */
ESA_API int esa_varlen_attn_bwd(const void* dout, const void* q, const void* k,
                        const void* v, const void* out,
                        const float* softmax_lse,
                        const int* cu_seqlens_q, const int* cu_seqlens_k,
                        int batch, int total_q, int total_k,
                        int max_seqlen_q, int max_seqlen_k,
                        int heads, int head_dim, int dtype, float softmax_scale,
                        float dropout_p, unsigned long long dropout_seed,
                        int mask_kind, const int* mask_a, const int* mask_b,
                        int n_mask_edges,
                        void* dq, void* dk, void* dv,
                        void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* PMA seed pooling: PMA.forward = MAB(S.repeat(B, 1, 1), X) (esa/mha.py:   */
/* 101-109; PMAFlashVarlen, esa/mha_flash_varlen.py:233-248) over packed     */
/* sets.  q [k_seeds, H, head_dim] holds the projected seeds fc_q(S), shared */
/* by all batch sets; k, v [total_k, H, head_dim] with cu_seqlens_k          */
/* [batch + 1].  out is [batch * k_seeds, H, head_dim] set-major,            */
/* softmax_lse [H][batch * k_seeds].  The backward's dq [k_seeds, H,         */
/* head_dim] sums the sets' seed gradients in set order (deterministic).     */
/* Workspace size from esa_pma_workspace_size.  dropout_p / dropout_seed as  */
/* esa_varlen_attn_fwd's, over the expanded queries (query b * k_seeds + s   */
/* is seed s of set b).                                                      */
/* ------------------------------------------------------------------------ */
ESA_API int esa_pma_workspace_size(int batch, int k_seeds, int total_k, int heads,
                           int head_dim, int dtype, int backward, size_t* bytes);
ESA_API int esa_pma_fwd(const void* q, const void* k, const void* v, const int* cu_seqlens_k,
                int batch, int k_seeds, int total_k, int max_seqlen_k, int heads,
                int head_dim, int dtype, float softmax_scale,
                float dropout_p, unsigned long long dropout_seed, void* out,
                float* softmax_lse, void* workspace, size_t workspace_bytes,
                void* stream);
ESA_API int esa_pma_bwd(const void* dout, const void* q, const void* k, const void* v,
                const void* out, const float* softmax_lse, const int* cu_seqlens_k,
                int batch, int k_seeds, int total_k, int max_seqlen_k, int heads,
                int head_dim, int dtype, float softmax_scale,
                float dropout_p, unsigned long long dropout_seed, void* dq, void* dk,
                void* dv, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Debug decode of an edge-mask plan (tests and debugging): the admissible   */
/* partners of every outer token, read from the plan the way the attention   */
/* kernels read it — per 32-token tile the partner list entries whose mask  */
/* bit is set, or, for a tile whose group overflowed the lists, the walk     */
/* kernels' predicate over its partner range if the group is on the plan's   */
/* overflow list.  The result is the mask that get_adj_mask_from_edge_index_ */
/* edge (esa/masked_layers.py:217-268) encodes as 0 entries of its bias,     */
/* row by row, as a CSR over the packed tokens.                              */
/* direction 0: the query tiles (forward and dQ passes); 1: what the dK/dV   */
/* passes read (the key tiles' lists, or the query tiles' lists when the     */
/* plan was built symmetric).  Two calls: with indptr NULL, out[t] (total_q  */
/* ints) receives outer token t's partner count; with indptr = the counts'   */
/* exclusive scan [total_q + 1], out[indptr[t] .. indptr[t+1]) receives its  */
/* partner token ids in ascending order.  Sizes as the plan was built with.  */
/* ------------------------------------------------------------------------ */
ESA_API int esa_edge_plan_decode(const void* plan, int total_q, int total_k, int direction,
                         const int* indptr, int* out, void* stream);

/* Byte offsets in a node plan (esa_node_plan_build) of its sections, for   */
/* tests and debugging: offsets[0] the copy of the indices [n_mask_edges],  */
/* [1] t_indptr [total_k + 1] and [2] t_rows [n_mask_edges] (the transposed */
/* CSR: per key token the query rows listing it, in ascending entry         */
/* position; keys outside [0, total_k) after t_indptr[total_k]), [3] the    */
/* query descriptors int4 [total_q] and [4] the key descriptors int4        */
/* [total_k] ({partner range lo, hi, row begin, row end}, the row emptied   */
/* when the range is).  No device access.                                    */
ESA_API int esa_node_plan_sections(int total_q, int total_k, int n_mask_edges, size_t* offsets);

/* Materialises the edge-adjacency mask of each segment as a padded
 * [batch, max_items, max_items] uint8 array (1 = attend), the same entries
 * get_adj_mask_from_edge_index_edge (esa/masked_layers.py:217-268) sets to 0
 * in its bias.  For tests and debugging on small inputs only. */
ESA_API int esa_edge_mask_dense(const int* tok_src, const int* tok_dst,
                        const int* cu_seqlens, int batch, int total,
                        int max_items, uint8_t* mask_out, void* stream);

/* ------------------------------------------------------------------------ */
/* Edge-token gather: out[e] = [x[src[e]] || x[dst[e]]], out is [E, 2F].     */
/* Replaces the gather + torch.cat at core/pretraining_model.py:153-155 and  */
/* esa/models.py:307-309.  dtype is ESA_F32 or ESA_BF16; bit-exact copy.     */
/* ------------------------------------------------------------------------ */
ESA_API int esa_edge_gather(const void* x, const int* src, const int* dst,
                    int64_t num_edges, int num_nodes, int features, int dtype,
                    void* out, void* stream);

/* ------------------------------------------------------------------------ */
/* Fused edge-token projection: out[e] = a[src[e]] + b[dst[e]] + bias, out   */
/* is [E, F] (contiguous), a and b are node rows lda / ldb elements apart,  */
/* bias is [F] or NULL.  With a = x W_s^T and b = x W_d^T (node-level GEMMs  */
/* of the two input halves of a Linear(2F', F) weight W = [W_s | W_d]) this  */
/* is Linear(cat(x[src], x[dst])) (core/pretraining_model.py:153-198,        */
/* esa/mlp_utils.py:28-32) without the [E, 2F'] intermediate.  Sums in fp32  */
/* in the order (a + b) + bias, rounded once; dtype ESA_F32 or ESA_BF16;     */
/* a node id outside [0, num_nodes) contributes zeros.                       */
/* ------------------------------------------------------------------------ */
ESA_API int esa_edge_gather_add(const void* a, int64_t lda, const void* b, int64_t ldb,
                        const void* bias, const int* src, const int* dst,
                        int64_t num_edges, int num_nodes, int features, int dtype,
                        void* out, void* stream);

/* ------------------------------------------------------------------------ */
/* CSR construction by a key array (e.g. dst): indptr[N+1] and perm[E], perm */
/* listing edge ids grouped by key in ascending edge order (a stable sort).  */
/* The layout torch_scatter's segment_*_csr consumes                        */
/* (GET/utils/sorted_segment_ops.py:17-41).                                  */
/* ------------------------------------------------------------------------ */
ESA_API int esa_csr_workspace_size(int64_t num_edges, int num_nodes, size_t* bytes);

ESA_API int esa_csr_build(const int* keys, int64_t num_edges, int num_nodes,
                  int* indptr, int* perm,
                  void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Token-budget batching: the greedy rule of                                */
/* ImprovedDynamicBatchSampler._create_batches_standard                     */
/* (data_loading/improved_dynamic_sampler.py:215-224) over graphs in order,  */
/* on the device.  counts [num_graphs] (int32, device; negative counts as 0) */
/* are the tokens each graph contributes; a graph that would push the open   */
/* batch past `budget` opens the next batch, unless the open batch is empty. */
/* Writes batch_of_graph [num_graphs] (batch id of each graph, consecutive   */
/* from 0), batch_start [num_graphs + 1] (first graph of each batch, then    */
/* num_graphs after the last; entries past it unused) and *num_batches (a    */
/* device int).  One block; no host synchronisation.                         */
/* ------------------------------------------------------------------------ */
ESA_API int esa_token_budget_pack_workspace_size(int num_graphs, size_t* bytes);
ESA_API int esa_token_budget_pack(const int* counts, int num_graphs, int64_t budget,
                          int* batch_of_graph, int* batch_start, int* num_batches,
                          void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Deterministic segmented sum: out[n] = sum_{i in [indptr[n], indptr[n+1])} */
/* y[perm ? perm[i] : i], accumulated in fp32 in ascending i and rounded     */
/* once.  y is [E, F], out is [N, F], both of `dtype`.  Replaces the atomic  */
/* scatter_add edge->node reductions (core/molecular_encoder.py:241-242)     */
/* with the CSR semantics of GET/utils/sorted_segment_ops.py:40-41.          */
/* ------------------------------------------------------------------------ */
ESA_API int esa_csr_segment_sum(const void* y, const int* perm, const int* indptr,
                        int num_nodes, int features, int dtype, void* out,
                        void* stream);

/* ------------------------------------------------------------------------ */
/* Deterministic segmented minimum / maximum with argument: torch_scatter's  */
/* scatter_min / scatter_max over dim 0 without `out` (torch_scatter 2.1,    */
/* pyg::pytorch-scatter in GET/env.yml), as the encoder takes each node's    */
/* closest close-range neighbour distance (core/molecular_encoder.py:214,    */
/* `scatter_min(close_dists, close_src, dim=0, dim_size=num_nodes)`).  For   */
/* node n and feature f the value starts at the largest finite value of      */
/* `dtype` (the lowest when is_max) and, over i in [indptr[n], indptr[n+1])  */
/* in ascending i with e = perm ? perm[i] : i, is replaced by y[e, f] when   */
/* that is strictly smaller (larger), arg[n, f] = e; a value never replaced  */
/* (empty segment, or only NaN / values beyond the start) is written as 0    */
/* with arg[n, f] = num_edges.  With the stable CSR of esa_csr_build a tie   */
/* keeps the lowest edge id (torch_scatter's CPU order; its GPU kernel keeps */
/* any tied edge).  y is [num_edges, F], out [N, F] of `dtype` (ESA_F32 or   */
/* ESA_BF16), arg [N, F] int64 or NULL.                                      */
/* ------------------------------------------------------------------------ */
ESA_API int esa_csr_segment_minmax(const void* y, const int* perm, const int* indptr,
                           int num_nodes, int features, int dtype, int is_max,
                           int64_t num_edges, void* out, int64_t* arg,
                           void* stream);

/* Backward of esa_edge_gather: gx[n] = sum over edges with src == n of
 * g[e, :F] + sum over edges with dst == n of g[e, F:], via two CSRs, each
 * accumulated in fp32 in ascending edge order (deterministic). */
ESA_API int esa_edge_gather_bwd(const void* g, const int* src_perm,
                        const int* src_indptr, const int* dst_perm,
                        const int* dst_indptr, int num_nodes, int features,
                        int dtype, void* gx, void* stream);

/* ------------------------------------------------------------------------ */
/* Block epilogue: y = mish(z) (+ residual), elementwise over n values of    */
/* `dtype` (ESA_F32 or ESA_BF16), evaluated in fp32 and rounded once.        */
/* With residual = the MAB's attention output O and z = fc_o(O) this is      */
/* `out + F.mish(fc_o(out))` (esa/mha.py:87, esa/mha_flash_varlen.py:195);  */
/* with residual NULL it is the MLP activation nn.Mish                        */
/* (esa/mlp_utils.py:24-37).  residual may be NULL; y may alias z or residual. */
/* ------------------------------------------------------------------------ */
ESA_API int esa_mish_fwd(const void* z, const void* residual, int64_t n, int dtype,
                 void* y, void* stream);

/* Backward of esa_mish_fwd: dz = grad * mish'(z) (the residual's gradient is */
/* grad itself).  dz may alias z or grad.                                     */
ESA_API int esa_mish_bwd(const void* z, const void* grad, int64_t n, int dtype,
                 void* dz, void* stream);

/* ------------------------------------------------------------------------ */
/* The block residual over the MAB epilogue: y = x + r(o + mish(z)), x and y */
/* fp32 [n] (the pre-norm block's residual stream, esa/masked_layers.py:    */
/* 471-472), z = fc_o(o) and o of `dtype` (esa/mha.py:87), r() the rounding */
/* to dtype that the MAB output gets.  Backward from g (fp32): g_o = r(g)   */
/* (o's gradient through the residual) and dz = r(g_o * mish'(z)); x's      */
/* gradient is g.                                                            */
/* ------------------------------------------------------------------------ */
ESA_API int esa_mab_residual_fwd(const void* z, const void* o, const float* x, int64_t n,
                         int dtype, float* y, void* stream);
ESA_API int esa_mab_residual_bwd(const void* z, const float* g, int64_t n, int dtype,
                         void* dz, void* g_o, void* stream);

/* ------------------------------------------------------------------------ */
/* Pre-norm LayerNorm over the last dimension of [rows, features] (features */
/* a multiple of 4, at most 2048): nn.LayerNorm(features, eps) as the ESA    */
/* blocks apply it (esa/utils/norm_layers.py:36; esa/masked_layers.py:418-  */
/* 419, 478-483), fp32 statistics, y = (x - mean) rstd weight + bias with    */
/* rstd = 1/sqrt(biased var + eps).  x is ESA_F32 or ESA_BF16; weight and    */
/* bias are fp32 [features] or NULL (1 and 0).  Writes y (y_dtype) and/or    */
/* its bf16 copy y_lp (either may be NULL, not both) and the per-row mean    */
/* and rstd [rows] that the backward takes.  Pointers 16-byte aligned.       */
/* ------------------------------------------------------------------------ */
ESA_API int esa_layer_norm_fwd(const void* x, int x_dtype, const float* weight,
                       const float* bias, int64_t rows, int features, float eps,
                       void* y, int y_dtype, void* y_lp, float* mean, float* rstd,
                       void* stream);

ESA_API int esa_layer_norm_bwd_workspace_size(int64_t rows, int features, size_t* bytes);

/* Backward: with g = dy + dy_lp (dy of dy_dtype and/or the bf16 gradient of */
/* y_lp; NULL = zero, not both), dx (x_dtype) = rstd (g w - mean(g w) -      */
/* xhat mean(g w xhat)) + dx_add and, when dweight / dbias are given, the    */
/* fp32 column sums of g xhat / g, reduced in a fixed order (deterministic). */
/* dx_add (x_dtype, NULL = none, must not overlap dx) is the gradient of x   */
/* from its other uses, e.g. a residual add: autograd would otherwise sum    */
/* the two in a separate pass.  The workspace (size from the query) is       */
/* needed only for dweight / dbias.                                          */
ESA_API int esa_layer_norm_bwd(const void* x, int x_dtype, const float* weight,
                       const float* mean, const float* rstd, const void* dy,
                       int dy_dtype, const void* dy_lp, const void* dx_add,
                       int64_t rows, int features, void* dx, float* dweight,
                       float* dbias, void* workspace, size_t workspace_bytes,
                       void* stream);

/* ------------------------------------------------------------------------ */
/* Column sums out[c] = sum_r x[r][c] (fp32, [cols]) of x [rows, cols]      */
/* (ESA_F32 or ESA_BF16; cols a multiple of 4): the bias gradient of the    */
/* blocks' nn.Linear layers over packed tokens (their autograd in the       */
/* reference, esa/mha.py:12-15, esa/mlp_utils.py:18-37).  Fixed summation   */
/* order (deterministic); workspace size from the query.                    */
/* ------------------------------------------------------------------------ */
ESA_API int esa_column_sum_workspace_size(int64_t rows, int cols, size_t* bytes);
ESA_API int esa_column_sum(const void* x, int dtype, int64_t rows, int cols, float* out,
                   void* workspace, size_t workspace_bytes, void* stream);

/* Mish backward with the bias gradient of the Linear that produced z (an   */
/* MLP's Linear -> Mish, esa/mlp_utils.py:18-37; autograd of nn.Linear's     */
/* bias, esa/mlp_utils.py:28-32): dz (dtype) as esa_mish_bwd writes it over  */
/* a [rows, cols] tensor, and dbias = the fp32 column sums of dz, equal to   */
/* esa_column_sum over dz, in one pass.  Workspace size from                 */
/* esa_column_sum_workspace_size(rows, cols).  cols % 4 == 0; 16-byte        */
/* aligned pointers.                                                         */
ESA_API int esa_mish_bwd_colsum(const void* z, const void* grad, int64_t rows, int cols,
                        int dtype, void* dz, float* dbias, void* workspace,
                        size_t workspace_bytes, void* stream);

/* fp32 Linear layers of the blocks: y_i = x W_i^T + b_i for i < n_out      */
/* (1-3) weights over one input, as nn.Linear computes them in fp32         */
/* (fc_q / fc_k / fc_v share their input, esa/mha.py:54-56; fc_o and the    */
/* MLP Linears take one, esa/mha.py:87, esa/mlp_utils.py:18-37).  Replaces  */
/* F.linear for fp32 device tensors of these shapes; the modules call it    */
/* for two or three weights over one input (one launch instead of several;  */
/* a single weight runs as fast in the library GEMM).  x [rows, K], W_i     */
/* [N_i, K], b_i [N_i] (or null), y_i [rows, N_i], all fp32, row-major and  */
/* contiguous; K % 16 == 0, N_i % 64 == 0; x, W_i, y_i 16-byte aligned.     */
/* weight, bias, y and out_features are host arrays of n_out entries.       */
/* fp32 products accumulated in fp32 (an order of its own: results agree    */
/* with a library GEMM to fp32 rounding, not bit for bit).  One launch;     */
/* rows == 0 launches nothing (then x, W_i and y_i may be null).            */
ESA_API int esa_linear_f32(const float* x, int rows, int in_features, int n_out,
                   const float* const* weight, const float* const* bias, float* const* y,
                   const int* out_features, void* stream);

/* ------------------------------------------------------------------------ */
/* Profiling hook (no counterpart in the reference; used by the benchmark).  */
/* While enabled, every kernel launch of the entry points above is           */
/* bracketed by hipEvents on its stream.  esa_profile_collect waits for the  */
/* recorded events (it synchronises), returns the summed milliseconds and    */
/* launch count per kernel id (capacity >= ESA_PROFILE_KERNELS) and clears   */
/* the record.  Not for concurrent use from several threads.                 */
/* ------------------------------------------------------------------------ */
#define ESA_PROFILE_KERNELS 23
ESA_API int esa_profile_enable(int on);
ESA_API int esa_profile_collect(float* total_ms, int* launches, int capacity);
ESA_API const char* esa_profile_kernel_name(int kernel);

#ifdef __cplusplus
}
#endif

#endif /* ESA_HIP_H */
