"""Packed token bookkeeping on the device.

The reference pads every graph's edge tokens to ``num_max_items`` with
``to_dense_batch`` (core/pretraining_model.py:211, esa/models.py:317) and
builds a dense [B, 1, N, N] adjacency bias over the whole batch
(esa/masked_layers.py:79-118 node mode, :217-268 edge mode).  Here a batch is
described once by a ``PackedSets`` descriptor: int32 ``cu_seqlens``, each
token's slot in the padded [B, N] layout and the mask in O(tokens + edges)
memory — per-token endpoint ids (``EdgeAdjacency``, whose edge-mask plan of
per-tile partner lists is built once on first use and shared by every masked
layer) or a CSR adjacency (``NodeAdjacency``).
It is passed where the reference passes ``adj_mask``.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import ctypes

import torch

from .. import _lib


def nearest_multiple_of_8(n: int) -> int:
    """core/molecular_encoder.py:15."""
    return ((int(n) + 7) // 8) * 8


def token_budget_batches(counts: torch.Tensor, budget: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Greedy token-budget batching of graphs in order, on the device (esa_token_budget_pack).

    The rule of ImprovedDynamicBatchSampler (data_loading/improved_dynamic_sampler.py:215-224) with
    ``counts`` [G] the tokens of each graph (edge counts for edge-set attention): a graph that would push
    the open batch past ``budget`` opens the next batch, unless the open batch is empty.  Returns device
    tensors (batch_of_graph [G] int32, batch_start [G + 1] int32, num_batches int32 scalar): batch b holds
    graphs batch_start[b] .. batch_start[b + 1] - 1 for b < num_batches.  Nothing synchronises with the host.
    """
    _lib.require_gpu(counts)
    if counts.dim() != 1:
        raise ValueError("counts must be 1-D")
    counts = counts.to(torch.int32).contiguous()
    g = counts.numel()
    lib = _lib.load()
    nbytes = ctypes.c_size_t(0)
    _lib.check(lib.esa_token_budget_pack_workspace_size(g, ctypes.byref(nbytes)), "esa_token_budget_pack_workspace_size")
    ws = torch.empty(max(int(nbytes.value), 256), dtype=torch.uint8, device=counts.device)
    batch_of_graph = torch.empty(g, dtype=torch.int32, device=counts.device)
    batch_start = torch.empty(g + 1, dtype=torch.int32, device=counts.device)
    num = torch.empty((), dtype=torch.int32, device=counts.device)
    _lib.check(lib.esa_token_budget_pack(counts.data_ptr(), g, int(budget), batch_of_graph.data_ptr(),
                                         batch_start.data_ptr(), num.data_ptr(), ws.data_ptr(), ws.numel(),
                                         _lib.stream_of(counts)), "esa_token_budget_pack")
    return batch_of_graph, batch_start, num


def cu_seqlens_from_counts(counts: torch.Tensor) -> torch.Tensor:
    """[0, cumsum(counts)] as int32 (the flash-attn varlen offsets)."""
    cu = torch.zeros(counts.numel() + 1, dtype=torch.int32, device=counts.device)
    cu[1:] = torch.cumsum(counts, 0).to(torch.int32)
    return cu


@dataclass
class PackedSets:
    """Tokens of a batch packed graph after graph, and their slots in the padded [B, N] layout.

    graph              : int64 [T] graph of each token
    position           : int64 [T] slot of the token inside its graph
    cu_seqlens         : int32 [B+1] token offsets per graph
    batch_size, max_items : the padded layout [B, N] the reference uses
    """

    graph: torch.Tensor
    position: torch.Tensor
    cu_seqlens: torch.Tensor
    batch_size: int
    max_items: int

    @property
    def num_tokens(self) -> int:
        return int(self.graph.numel())

    @property
    def padded_index(self) -> torch.Tensor:
        """Flat index of each token in the padded [B * N] layout."""
        return self.graph * self.max_items + self.position

    def unpad(self, x: torch.Tensor) -> torch.Tensor:
        """[B, N, ...] -> [T, ...] (the valid tokens, in token order)."""
        b, n = x.shape[0], x.shape[1]
        if b != self.batch_size or n != self.max_items:
            raise ValueError(f"padded input is [{b}, {n}], descriptor is [{self.batch_size}, {self.max_items}]")
        return x.reshape(b * n, *x.shape[2:]).index_select(0, self.padded_index)

    def pad(self, y: torch.Tensor) -> torch.Tensor:
        """[T, ...] -> [B, N, ...] with zeros at padding (flash-attn's pad_input)."""
        out = y.new_zeros((self.batch_size * self.max_items,) + tuple(y.shape[1:]))
        out = out.index_copy(0, self.padded_index, y)
        return out.view(self.batch_size, self.max_items, *y.shape[1:])

    def kernel_mask(self, padded: bool) -> dict:
        """Keyword arguments of ``varlen_attention`` that apply this mask, for packed tokens or for the
        padded [B * N] token layout."""
        raise NotImplementedError


def _positions(graph: torch.Tensor, batch_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """cu_seqlens [B+1] and each token's slot in its graph, for tokens grouped by graph in ascending order
    (a PyG batch; to_dense_batch makes the same assumption).  Binary searches over the sorted graph ids,
    so no host synchronisation: graph ids outside [0, B) clamp to the nearest graph."""
    dev = graph.device
    bounds = torch.arange(batch_size + 1, device=dev, dtype=graph.dtype)
    cu = torch.searchsorted(graph, bounds).to(torch.int32)
    g = graph.clamp(0, max(batch_size - 1, 0))
    position = torch.arange(graph.numel(), device=dev, dtype=torch.int64) - cu[:-1].to(torch.int64)[g]
    return cu, position


@dataclass
class EdgeAdjacency(PackedSets):
    """Edge tokens of a batch and their share-an-endpoint mask, unmaterialised.

    edge_src, edge_dst : int32 [T] endpoint node ids of each token (global ids:
                          different graphs never share a node)
    """

    edge_src: torch.Tensor = None
    edge_dst: torch.Tensor = None
    _plan: torch.Tensor | None = field(default=None, repr=False, compare=False)

    @classmethod
    def from_edge_index(cls, edge_index: torch.Tensor, batch_mapping: torch.Tensor, batch_size: int,
                        max_items: int) -> "EdgeAdjacency":
        """Tokens = edges in edge_index order, grouped by graph (a PyG batch).

        The graph of an edge is the graph of its source node
        (core/pretraining_model.py:202, esa/models.py:316); its slot is its
        rank among the graph's edges, as in to_dense_batch.
        """
        src, dst = edge_index[0], edge_index[1]
        graph = batch_mapping.index_select(0, src).to(torch.int64)
        cu, position = _positions(graph, batch_size)
        return cls(graph=graph, position=position, cu_seqlens=cu, batch_size=int(batch_size),
                   max_items=int(max_items), edge_src=src.to(torch.int32).contiguous(),
                   edge_dst=dst.to(torch.int32).contiguous())

    def padded_nodes(self) -> tuple[torch.Tensor, torch.Tensor]:
        """Endpoint ids in the padded layout; padding slots get ids that match nothing."""
        n = self.batch_size * self.max_items
        dev = self.edge_src.device
        # distinct negative ids per padding slot: no two padding slots share a node
        fill = -1 - torch.arange(n, device=dev, dtype=torch.int32)
        src = fill.clone().index_copy(0, self.padded_index, self.edge_src)
        dst = (fill - n).index_copy(0, self.padded_index, self.edge_dst)
        return src, dst

    def plan(self) -> torch.Tensor:
        """The batch's edge-mask plan over the packed tokens and ``cu_seqlens`` (esa_edge_plan_build), built on
        first use and reused by every masked layer's forward and backward, as the reference builds its mask
        once per batch (esa/masked_layers.py:849-936)."""
        if self._plan is None:
            from .attention import edge_plan
            self._plan = edge_plan(self.edge_src, self.edge_dst, self.cu_seqlens)
        return self._plan

    def kernel_mask(self, padded: bool) -> dict:
        if padded:
            src, dst = self.padded_nodes()
            return {"edge_src": src, "edge_dst": dst}
        return {"edge_plan": self.plan()}


@dataclass
class NodeAdjacency(PackedSets):
    """Node tokens of a batch and the node-mode mask (query src attends to key dst per edge).

    The mask get_adj_mask_from_edge_index_node (esa/masked_layers.py:79-118)
    writes into a [B, 1, N, N] bias, kept here as a CSR by query over packed
    token ids: row t lists the dst nodes of t's out-edges in ascending order
    (a repeated edge appears twice and counts once).

    indptr  : int32 [T+1]
    indices : int32 [nnz]
    """

    indptr: torch.Tensor = None
    indices: torch.Tensor = None
    _plan: torch.Tensor | None = field(default=None, repr=False, compare=False)

    @classmethod
    def from_edge_index(cls, edge_index: torch.Tensor, batch_mapping: torch.Tensor, batch_size: int,
                        max_items: int) -> "NodeAdjacency":
        """Tokens = nodes in node order (a PyG batch: graphs contiguous and ascending), slot = node id
        minus the graph's first node, as to_dense_batch and unbatch_edge_index number them."""
        graph = batch_mapping.to(torch.int64)
        cu, position = _positions(graph, batch_size)
        nodes = graph.numel()
        src, dst = edge_index[0].to(torch.int64), edge_index[1].to(torch.int64)
        key = torch.sort(src * max(nodes, 1) + dst).values
        s_sorted = torch.div(key, max(nodes, 1), rounding_mode="floor")
        # row starts by binary search over the sorted query ids (no host synchronisation)
        indptr = torch.searchsorted(s_sorted, torch.arange(nodes + 1, device=key.device, dtype=key.dtype))
        indptr = indptr.to(torch.int32)
        indices = (key - s_sorted * max(nodes, 1)).to(torch.int32).contiguous()
        return cls(graph=graph, position=position, cu_seqlens=cu, batch_size=int(batch_size),
                   max_items=int(max_items), indptr=indptr, indices=indices)

    def padded_csr(self) -> tuple[torch.Tensor, torch.Tensor]:
        """The same CSR over the padded [B * N] token layout (padding rows are empty)."""
        pidx = self.padded_index
        deg = (self.indptr[1:] - self.indptr[:-1]).to(torch.int64)
        counts = torch.zeros(self.batch_size * self.max_items, dtype=torch.int64, device=deg.device)
        counts.index_copy_(0, pidx, deg)
        return cu_seqlens_from_counts(counts), pidx.index_select(0, self.indices.to(torch.int64)).to(torch.int32)

    def plan(self) -> torch.Tensor:
        """The batch's node plan (esa_node_plan_build: the CSR's transpose by key), built on first use and
        reused by every node-mode layer's backward, as the reference builds its node bias once per batch
        (esa/masked_layers.py:849-936)."""
        if self._plan is None:
            from .attention import node_plan
            self._plan = node_plan(self.indptr, self.indices, self.cu_seqlens)
        return self._plan

    def kernel_mask(self, padded: bool) -> dict:
        if padded:
            ip, ix = self.padded_csr()
            return {"adj_indptr": ip, "adj_indices": ix}
        return {"adj_indptr": self.indptr, "adj_indices": self.indices, "adj_plan": self.plan()}
