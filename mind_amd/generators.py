"""Seeded synthetic inputs for the benchmark configurations.

No dataset or network is available, so each configuration is generated from
its written description (the five ``configs`` of the benchmark definition).
Edges follow ``radius_graph(pos, r, loop=False)`` conventions
(data_loading/cache_to_pyg.py:546-550): edge ``j -> i`` for every neighbour
``j`` of centre ``i`` within ``r``, so ``edge_index[0]`` is the neighbour
(source) and ``edge_index[1]`` the centre (target).  Edges are ordered by
target, then source, within each graph, and graphs are concatenated with node
offsets, as a PyG ``Batch`` does.  Every generator is a pure function of its
seed (numpy PCG64), so the CPU oracle and the GPU see identical integers.

Choices the configuration text leaves open:
  * random-walk direction jitter: d_i = normalise(d_{i-1} + N(0, sigma^2 I));
  * neighbour cap: keep the ``cap`` nearest neighbours of each centre, ties
    broken by the lower node index;
  * token-budget packing: greedy, a new batch starts when the next graph
    would exceed the budget (data_loading/improved_dynamic_sampler.py:215-224),
    counting edges (the attention tokens) rather than atoms.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class GraphBatch:
    """A packed batch of graphs in PyG layout plus the edge-token packing."""

    pos: np.ndarray            # [N, 3] float32
    batch: np.ndarray          # [N] int64 graph id per node
    edge_index: np.ndarray     # [2, E] int64, global node ids, grouped by graph
    node_counts: np.ndarray    # [B] nodes per graph
    edge_counts: np.ndarray    # [B] edges (= tokens) per graph
    meta: dict = field(default_factory=dict)

    @property
    def num_graphs(self) -> int:
        return int(self.node_counts.shape[0])

    @property
    def num_tokens(self) -> int:
        return int(self.edge_index.shape[1])

    @property
    def cu_seqlens(self) -> np.ndarray:
        return np.concatenate([[0], np.cumsum(self.edge_counts)]).astype(np.int32)

    @property
    def max_seqlen(self) -> int:
        return int(self.edge_counts.max()) if self.edge_counts.size else 0

    @property
    def sum_sq(self) -> int:
        """Sum of squared segment lengths: the dense attention pair count."""
        return int((self.edge_counts.astype(np.int64) ** 2).sum())


def radius_edges(pos: np.ndarray, r: float, cap: int | None = None) -> np.ndarray:
    """Directed radius-graph edges of one graph, ``[2, E]`` (source, target).

    Pair (j, i), j != i, is an edge iff |pos_j - pos_i| <= r; with ``cap``, only
    the ``cap`` nearest sources per target are kept (ties: lower index).
    Sorted by target, then source.
    """
    n = pos.shape[0]
    if n == 0:
        return np.zeros((2, 0), dtype=np.int64)
    d2 = ((pos[:, None, :].astype(np.float64) - pos[None, :, :].astype(np.float64)) ** 2).sum(-1)
    within = d2 <= r * r
    np.fill_diagonal(within, False)
    if cap is not None:
        # rank sources of each target by (distance, index); keep the first `cap`
        order = np.lexsort((np.broadcast_to(np.arange(n), (n, n)), d2), axis=1)  # per row i: sources sorted
        keep = np.zeros_like(within)
        sorted_within = np.take_along_axis(within, order, axis=1)
        rank = np.cumsum(sorted_within, axis=1)
        sel = sorted_within & (rank <= cap)
        np.put_along_axis(keep, order, sel, axis=1)
        within = keep
    tgt, src = np.nonzero(within)  # row-major: sorted by target, then source
    return np.stack([src, tgt]).astype(np.int64)


def _assemble(graph_pos: list[np.ndarray], r: float, cap: int | None, meta: dict) -> GraphBatch:
    pos_all, batch_all, edges_all, ncount, ecount = [], [], [], [], []
    offset = 0
    for b, p in enumerate(graph_pos):
        e = radius_edges(p, r, cap)
        pos_all.append(p.astype(np.float32))
        batch_all.append(np.full(p.shape[0], b, dtype=np.int64))
        edges_all.append(e + offset)
        ncount.append(p.shape[0])
        ecount.append(e.shape[1])
        offset += p.shape[0]
    return GraphBatch(
        pos=np.concatenate(pos_all) if pos_all else np.zeros((0, 3), np.float32),
        batch=np.concatenate(batch_all) if batch_all else np.zeros(0, np.int64),
        edge_index=np.concatenate(edges_all, axis=1) if edges_all else np.zeros((2, 0), np.int64),
        node_counts=np.asarray(ncount, dtype=np.int64),
        edge_counts=np.asarray(ecount, dtype=np.int64),
        meta=meta,
    )


def random_walk(rng: np.random.Generator, n: int, step: float = 3.8, sigma: float = 0.5) -> np.ndarray:
    """Chain of ``n`` points: unit direction d_i = normalise(d_{i-1} + N(0, sigma^2 I)), step length ``step``."""
    d = rng.normal(size=3)
    d /= np.linalg.norm(d)
    pts = np.zeros((n, 3))
    for i in range(1, n):
        d = d + rng.normal(scale=sigma, size=3)
        d /= np.linalg.norm(d)
        pts[i] = pts[i - 1] + step * d
    return pts


def small_molecules(seed: int = 0, num_graphs: int = 64, n_min: int = 9, n_max: int = 29,
                    sigma: float = 1.5, r: float = 5.0, num_types: int = 16) -> tuple[GraphBatch, np.ndarray]:
    """Config 0 (CPU-runnable ESA block): returns the batch and node types U{0..num_types-1}."""
    rng = np.random.default_rng(seed)
    sizes = rng.integers(n_min, n_max + 1, size=num_graphs)
    graphs = [rng.normal(scale=sigma, size=(int(n), 3)) for n in sizes]
    gb = _assemble(graphs, r, None, {"generator": "small_molecules", "seed": seed, "r": r})
    types = rng.integers(0, num_types, size=int(sizes.sum()))
    return gb, types


def protein_like(seed: int = 0, num_graphs: int = 32, n_min: int = 64, n_max: int = 512,
                 r: float = 8.0, cap: int = 16) -> GraphBatch:
    """Config 1 (varlen attention): node counts U{n_min..n_max}, random-walk chains."""
    rng = np.random.default_rng(seed)
    sizes = rng.integers(n_min, n_max + 1, size=num_graphs)
    graphs = [random_walk(rng, int(n)) for n in sizes]
    return _assemble(graphs, r, cap, {"generator": "protein_like", "seed": seed, "r": r, "cap": cap})


def protein_budget(seed: int = 0, token_budget: int = 65536, mu: float = 5.5, sigma: float = 0.5,
                   n_min: int = 32, n_max: int = 1024, r: float = 8.0, cap: int = 16,
                   count: str = "edges") -> GraphBatch:
    """Config 2 (masked MAB): lognormal node counts, greedy packing to a token budget.

    Graphs are drawn until the next one would push the batch past
    ``token_budget`` tokens; that graph is not included (it would open the
    next batch).  ``count``: "edges" (edge tokens, edge mode) or "nodes" (node
    tokens, node mode).
    """
    if count not in ("edges", "nodes"):
        raise ValueError("count is 'edges' or 'nodes'")
    rng = np.random.default_rng(seed)
    graphs, total = [], 0
    while True:
        n = int(np.clip(round(rng.lognormal(mu, sigma)), n_min, n_max))
        p = random_walk(rng, n)
        ne = radius_edges(p, r, cap).shape[1] if count == "edges" else n
        if total + ne > token_budget and graphs:
            break
        graphs.append(p)
        total += ne
        if total >= token_budget:
            break
    meta = {"generator": "protein_budget", "seed": seed, "budget": token_budget, "r": r, "cap": cap}
    if count != "edges":
        meta["count"] = count
    return _assemble(graphs, r, cap, meta)


def block_local_edges(seed: int = 0, num_nodes: int = 1 << 21, num_edges: int = 1 << 25,
                      block: int = 512) -> tuple[np.ndarray, np.ndarray]:
    """Config 3 (gather-scatter): src ~ U{0..N-1}; dst in src's block of ``block`` nodes.

    Returns int32 ``(src, dst)`` in generation order.
    """
    rng = np.random.default_rng(seed)
    src = rng.integers(0, num_nodes, size=num_edges, dtype=np.int64)
    dst = (src // block) * block + rng.integers(0, block, size=num_edges, dtype=np.int64)
    dst = np.minimum(dst, num_nodes - 1)
    return src.astype(np.int32), dst.astype(np.int32)
