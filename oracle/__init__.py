"""CPU oracle for the ESA hot path — TEST INFRASTRUCTURE ONLY.

A plain restatement of the reference's arithmetic, used as the checker in
``tests/``, in ``__graft_entry__.smoke()`` and as the ``cpu_baseline`` leg of
``bench.py``.  Nothing in ``mind_amd`` imports it; the product path never runs
on it.

Each function cites the reference file:line it restates.  How each one is
pinned (the reference holds no golden vectors, tests or fixtures for this
path, and its Python cannot be imported here: xformers, flash_attn,
torch_geometric and torch_scatter are absent):

  packing.cu_seqlens / positions / to_dense_batch
      closed form pos = index - graph start; hypothesis round trips.
  mask.edge_adjacency_global / edge_bias_padded
      brute force vs an independent set-intersection loop on tiny graphs;
      invariants: symmetric, zero diagonal, (u->v) ~ (v->u), no cross-graph
      pairs; nnz closed form sum_v c_v(c_v-1) - sum_{u<v} m_uv(m_uv-1).
  mask.node_adjacency_segment / node_bias_padded
      node_bias_padded restates esa/masked_layers.py:79-118 from edge_index;
      the CSR blocks equal its zero entries per graph, and both agree with a
      plain loop over the edges (repeated edges and self-loops included).
  attention.varlen_attention (fwd, lse)
      torch.nn.functional.scaled_dot_product_attention (math backend, fp64)
      per segment; special cases L=1 (out = v), q = 0 (out = mean v), a
      single admissible key (out = that v), -inf bias == -99999 bias.
  attention.varlen_attention_bwd
      torch.autograd through the fp64 forward and central finite differences.
  dropout.fmix32 / keep_mask, attention with dropout=(p, seed)
      fmix32 inside the whole MurmurHash3_x86_32 equals scikit-learn's
      murmurhash3_32 on random keys and seeds, and the hash's published
      test vectors hold; the two 16-bit halves a key pair shares are
      independent (correlation, joint keep rate); keep rate 1 - p within
      binomial bounds, no correlation between neighbouring queries / keys /
      heads or seeds; p = 0 equals the plain oracle; the forward is the
      definition (P o Z / (1 - p)) V, its mean over seeds tends to P V; the
      backward equals torch.autograd through a dense fp64 forward with the
      same materialised Z.
  edges.edge_gather / csr_build / segment_sum
      bitwise copy identities; numpy stable argsort + bincount; constant rows
      give degree * value exactly; fp64 index_add agrees to rounding.
  edges.scatter_minmax (torch_scatter 2.1's scatter_min / scatter_max)
      the literal sequential update and the vectorised form agree bit for
      bit (ties, NaN, +-inf, the largest finite value, -0, dropped indices);
      values equal torch.scatter_reduce amin / amax; args by brute force;
      the scatter_max example of torch_scatter's documentation.
  modules (MAB / MABFlashVarlen / SAB / PMA / SmallMLP / LN / blocks)
      closed forms: fc_q = 0 gives uniform attention, whose output is the
      key-mean of V = fc_v(K) (esa/mha.py:55) or fc_v(fc_k(K))
      (esa/mha_flash_varlen.py:155-156); identity fc_o with zero bias gives
      out = O + mish(O).
"""
