"""Edge-token gather, CSR build and segmented sums (test infrastructure; see oracle/__init__.py)."""
from __future__ import annotations

import numpy as np
import torch


def edge_gather(x: np.ndarray, src: np.ndarray, dst: np.ndarray) -> np.ndarray:
    """[x[src] || x[dst]] — core/pretraining_model.py:153-155, esa/models.py:307-309."""
    return np.concatenate([x[src], x[dst]], axis=1)


def edge_token_linear(x: np.ndarray, src: np.ndarray, dst: np.ndarray, weight: np.ndarray,
                      bias: np.ndarray | None = None, edge_attr: np.ndarray | None = None) -> np.ndarray:
    """Linear over the edge tokens: [x[src] || x[dst] (|| edge_attr)] @ weight^T + bias, in float64 —
    core/pretraining_model.py:153-198 (edge attributes appended at :157-159) with the MLP's first Linear
    (esa/mlp_utils.py:28-32)."""
    h = edge_gather(np.asarray(x, np.float64), src, dst)
    if edge_attr is not None:
        h = np.concatenate([h, np.asarray(edge_attr, np.float64)], axis=1)
    h = h @ np.asarray(weight, np.float64).T
    return h if bias is None else h + np.asarray(bias, np.float64)


def csr_build(keys: np.ndarray, num_nodes: int) -> tuple[np.ndarray, np.ndarray]:
    """indptr [N+1] and perm [E] (edge ids grouped by key, ascending id within a key).

    The CSR layout segment_*_csr consumes (GET/utils/sorted_segment_ops.py:17-41).
    """
    keys = np.asarray(keys, dtype=np.int64)
    counts = np.bincount(keys, minlength=num_nodes)
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    perm = np.argsort(keys, kind="stable").astype(np.int32)
    return indptr, perm


def segment_sum_sequential(y: np.ndarray, perm: np.ndarray | None, indptr: np.ndarray,
                           acc_dtype=np.float32) -> np.ndarray:
    """out[n] = y[perm[a]] + y[perm[a+1]] + ... accumulated left to right in ``acc_dtype``.

    The summation order is fixed (ascending segment position), so the fp32
    result is a deterministic function of the input; vectorised over nodes,
    sequential over the position inside each segment.
    """
    indptr = np.asarray(indptr, dtype=np.int64)
    n = indptr.shape[0] - 1
    deg = indptr[1:] - indptr[:-1]
    out = np.zeros((n,) + y.shape[1:], dtype=acc_dtype)
    maxdeg = int(deg.max()) if n else 0
    for j in range(maxdeg):
        rows = np.nonzero(deg > j)[0]
        idx = indptr[rows] + j
        e = perm[idx] if perm is not None else idx
        out[rows] += y[e].astype(acc_dtype)
    return out


def segment_sum_f64(y: np.ndarray, keys: np.ndarray, num_nodes: int) -> np.ndarray:
    """fp64 scatter-add by key (the math of scatter_add, core/molecular_encoder.py:241-242)."""
    out = np.zeros((num_nodes,) + y.shape[1:], dtype=np.float64)
    np.add.at(out, np.asarray(keys, dtype=np.int64), y.astype(np.float64))
    return out


def edge_gather_torch(x: torch.Tensor, src: torch.Tensor, dst: torch.Tensor) -> torch.Tensor:
    """The reference's own expression on torch tensors, torch.cat((x[src], x[dst]), 1)
    (core/pretraining_model.py:153-155): the CPU baseline of the gather (multi-threaded in torch)."""
    return torch.cat((x[src], x[dst]), 1)


def scatter_sum_torch(y: torch.Tensor, index: torch.Tensor, num_nodes: int) -> torch.Tensor:
    """scatter_add of edge rows to nodes (core/molecular_encoder.py:241-242) as torch's index_add_ on the
    CPU: the CPU baseline of the segment sum."""
    return y.new_zeros((num_nodes,) + tuple(y.shape[1:])).index_add_(0, index, y)
