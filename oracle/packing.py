"""Segment bookkeeping (test infrastructure; see oracle/__init__.py)."""
from __future__ import annotations

import numpy as np
import torch


def nearest_multiple_of_8(n: int) -> int:
    """core/molecular_encoder.py:15 (used for num_max_items, esa/models.py:417-418)."""
    return int(np.ceil(n / 8) * 8)


def cu_seqlens(counts) -> np.ndarray:
    """[0, cumsum(counts)] int32 — the cu_seqlens flash-attn's unpad_input builds
    (esa/mha_flash_varlen.py:168-170)."""
    counts = np.asarray(counts, dtype=np.int64)
    return np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)


def positions(graph_of_token: np.ndarray) -> np.ndarray:
    """Position of each token inside its graph, tokens grouped by graph.

    Restates edge_batch_index_to_original_index (esa/masked_layers.py:247-249,
    get_first_unique_index :145-155 + generate_consecutive_tensor :158-171)
    and the slot to_dense_batch assigns (esa/models.py:317).
    """
    g = np.asarray(graph_of_token)
    pos = np.zeros(g.shape[0], dtype=np.int64)
    for i in range(1, g.shape[0]):
        pos[i] = pos[i - 1] + 1 if g[i] == g[i - 1] else 0
    return pos


def to_dense_batch(x: torch.Tensor, graph_of_token: np.ndarray, batch_size: int, max_items: int,
                   fill: float = 0.0) -> tuple[torch.Tensor, torch.Tensor]:
    """torch_geometric.utils.to_dense_batch as called at core/pretraining_model.py:211."""
    pos = positions(graph_of_token)
    out = torch.full((batch_size, max_items) + tuple(x.shape[1:]), fill, dtype=x.dtype)
    mask = torch.zeros(batch_size, max_items, dtype=torch.bool)
    g = torch.as_tensor(np.asarray(graph_of_token), dtype=torch.long)
    p = torch.as_tensor(pos, dtype=torch.long)
    out[g, p] = x
    mask[g, p] = True
    return out, mask


def token_budget_batches(counts, budget: int) -> list[list[int]]:
    """Greedy batching of graphs in order under a token budget: the rule of
    ImprovedDynamicBatchSampler._create_batches_standard (data_loading/improved_dynamic_sampler.py:215-224),
    graph i counting ``counts[i]`` tokens.  Returns the batches as lists of graph indices."""
    batches, current, tokens = [], [], 0
    for i, c in enumerate(counts):
        c = max(int(c), 0)
        if tokens + c > budget and current:
            batches.append(current)
            current, tokens = [i], c
        else:
            current.append(i)
            tokens += c
    if current:
        batches.append(current)
    return batches
