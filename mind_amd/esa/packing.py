"""Packed edge-token bookkeeping on the device (no host synchronisation).

The reference pads every graph's edge tokens to ``num_max_items`` with
``to_dense_batch`` (core/pretraining_model.py:211, esa/models.py:317) and
builds a dense [B, 1, N, N] edge-adjacency bias over the whole batch
(esa/masked_layers.py:217-268).  Here a batch is described once by an
``EdgeAdjacency``: per-token endpoint ids, int32 ``cu_seqlens`` and each
token's slot in the padded [B, N] layout.  It is passed where the reference
passes ``adj_mask``; the attention kernels evaluate the mask from it on the fly.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


def nearest_multiple_of_8(n: int) -> int:
    """core/molecular_encoder.py:15."""
    return ((int(n) + 7) // 8) * 8


def cu_seqlens_from_counts(counts: torch.Tensor) -> torch.Tensor:
    """[0, cumsum(counts)] as int32 (the flash-attn varlen offsets)."""
    cu = torch.zeros(counts.numel() + 1, dtype=torch.int32, device=counts.device)
    cu[1:] = torch.cumsum(counts, 0).to(torch.int32)
    return cu


@dataclass
class EdgeAdjacency:
    """Edge tokens of a batch and their share-an-endpoint mask, unmaterialised.

    edge_src, edge_dst : int32 [T] endpoint node ids of each token (global ids:
                          different graphs never share a node)
    graph              : int64 [T] graph of each token
    position           : int64 [T] slot of the token inside its graph
    cu_seqlens         : int32 [B+1] token offsets per graph
    batch_size, max_items : the padded layout [B, N] the reference uses
    """

    edge_src: torch.Tensor
    edge_dst: torch.Tensor
    graph: torch.Tensor
    position: torch.Tensor
    cu_seqlens: torch.Tensor
    batch_size: int
    max_items: int

    @property
    def num_tokens(self) -> int:
        return int(self.edge_src.numel())

    @property
    def padded_index(self) -> torch.Tensor:
        """Flat index of each token in the padded [B * N] layout."""
        return self.graph * self.max_items + self.position

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
        counts = torch.bincount(graph, minlength=batch_size)
        cu = cu_seqlens_from_counts(counts)
        position = torch.arange(graph.numel(), device=graph.device, dtype=torch.int64) - cu[:-1].to(torch.int64)[graph]
        return cls(src.to(torch.int32).contiguous(), dst.to(torch.int32).contiguous(), graph, position, cu,
                   int(batch_size), int(max_items))

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

    def padded_nodes(self) -> tuple[torch.Tensor, torch.Tensor]:
        """Endpoint ids in the padded layout; padding slots get ids that match nothing."""
        n = self.batch_size * self.max_items
        dev = self.edge_src.device
        # distinct negative ids per padding slot: no two padding slots share a node
        fill = -1 - torch.arange(n, device=dev, dtype=torch.int32)
        src = fill.clone().index_copy(0, self.padded_index, self.edge_src)
        dst = (fill - n).index_copy(0, self.padded_index, self.edge_dst)
        return src, dst
