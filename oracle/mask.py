"""Edge-adjacency and node masks (test infrastructure; see oracle/__init__.py)."""
from __future__ import annotations

import numpy as np
import torch

from .packing import positions

MASK_FILL = -99999.0  # esa/masked_layers.py:229 (empty_mask_fill_value)


def edge_adjacency_global(src: np.ndarray, dst: np.ndarray) -> np.ndarray:
    """E x E bool: edges share an endpoint, diagonal excluded.

    Restates create_edge_adjacency_mask (esa/masked_layers.py:121-142): the
    four endpoint comparisons OR-ed, then fill_diagonal_(0).
    """
    s = np.asarray(src)[:, None]
    d = np.asarray(dst)[:, None]
    m = (s == s.T) | (d == d.T) | (s == d.T) | (d == s.T)
    np.fill_diagonal(m, False)
    return m


def edge_adjacency_segment(src: np.ndarray, dst: np.ndarray, start: int, stop: int) -> np.ndarray:
    """The [L, L] block of one segment (tokens start..stop-1)."""
    return edge_adjacency_global(np.asarray(src)[start:stop], np.asarray(dst)[start:stop])


def edge_bias_padded(edge_index: np.ndarray, graph_of_edge: np.ndarray, batch_size: int, max_items: int,
                     dtype=torch.float32, fill: float = MASK_FILL) -> torch.Tensor:
    """[B, 1, N, N] additive bias: 0 where edges i, j of graph b share a node.

    Restates get_adj_mask_from_edge_index_edge (esa/masked_layers.py:217-268)
    for the xformers / fp path: full of -99999, the global E x E adjacency's
    nonzeros mapped to (graph, local i, local j) and set to 0.
    """
    src, dst = np.asarray(edge_index[0]), np.asarray(edge_index[1])
    adj = edge_adjacency_global(src, dst)
    pos = positions(graph_of_edge)
    bias = torch.full((batch_size, max_items, max_items), fill, dtype=dtype)
    i, j = np.nonzero(adj)
    g = np.asarray(graph_of_edge)
    bias[torch.as_tensor(g[i]), torch.as_tensor(pos[i]), torch.as_tensor(pos[j])] = 0.0
    return bias.unsqueeze(1)


def node_bias_padded(edge_index: np.ndarray, batch_mapping: np.ndarray, batch_size: int, max_items: int,
                     dtype=torch.float32, fill: float = MASK_FILL) -> torch.Tensor:
    """[B, 1, N, N] node-mode bias: 0 at (graph, local src, local dst) of each edge.

    Restates get_adj_mask_from_edge_index_node (esa/masked_layers.py:79-118):
    local ids from unbatch_edge_index (node id - first node of its graph).
    """
    bm = np.asarray(batch_mapping)
    first = {}
    for n, b in enumerate(bm):
        first.setdefault(int(b), n)
    src, dst = np.asarray(edge_index[0]), np.asarray(edge_index[1])
    g = bm[src]
    ls = src - np.array([first[int(b)] for b in g], dtype=np.int64)
    ld = dst - np.array([first[int(b)] for b in g], dtype=np.int64)
    bias = torch.full((batch_size, max_items, max_items), fill, dtype=dtype)
    bias[torch.as_tensor(g), torch.as_tensor(ls), torch.as_tensor(ld)] = 0.0
    return bias.unsqueeze(1)


def node_adjacency_segment(indptr: np.ndarray, indices: np.ndarray, qs: int, qe: int, ks: int,
                           ke: int) -> np.ndarray:
    """[Lq, Lk] bool block of a CSR adjacency: query i attends to key j iff j is listed in row i.

    The per-graph block of get_adj_mask_from_edge_index_node
    (esa/masked_layers.py:110-112): 0 (attend) at (src_local, dst_local) of
    every edge; repeated edges set the same entry again.
    """
    indptr = np.asarray(indptr, dtype=np.int64)
    indices = np.asarray(indices, dtype=np.int64)
    m = np.zeros((qe - qs, ke - ks), dtype=bool)
    for i in range(qs, qe):
        js = indices[indptr[i]:indptr[i + 1]]
        js = js[(js >= ks) & (js < ke)]
        m[i - qs, js - ks] = True
    return m


def edge_mask_nnz(src: np.ndarray, dst: np.ndarray) -> int:
    """Closed-form count of true entries of edge_adjacency_global.

    Pairs (i, j), i != j, sharing a node = sum over nodes v of c_v (c_v - 1)
    (ordered pairs of edge-incidences at v) minus the double count of pairs
    sharing both endpoints: for each unordered node pair {u, v} joined by m_uv
    edges, those m_uv (m_uv - 1) ordered pairs were counted at u and at v.
    Self-loops (u == v) are incident twice to one node; they are not produced
    by radius graphs and are excluded here.
    """
    src = np.asarray(src, dtype=np.int64)
    dst = np.asarray(dst, dtype=np.int64)
    assert not np.any(src == dst), "closed form assumes no self-loops"
    _, c = np.unique(np.concatenate([src, dst]), return_counts=True)
    total = int((c * (c - 1)).sum())
    lo, hi = np.minimum(src, dst), np.maximum(src, dst)
    _, m = np.unique(np.stack([lo, hi], 1), axis=0, return_counts=True)
    return total - int((m * (m - 1)).sum())
