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


def scatter_min_torch(y: torch.Tensor, index: torch.Tensor, num_nodes: int) -> torch.Tensor:
    """The values of scatter_min(y, index, dim=0, dim_size=num_nodes) (core/molecular_encoder.py:214) for
    finite y as torch's scatter_reduce('amin') on the CPU (nodes without edges 0): the CPU baseline of the
    segmented minimum."""
    return y.new_zeros(num_nodes).scatter_reduce_(0, index, y, "amin", include_self=False)


def scatter_sum_torch(y: torch.Tensor, index: torch.Tensor, num_nodes: int) -> torch.Tensor:
    """scatter_add of edge rows to nodes (core/molecular_encoder.py:241-242) as torch's index_add_ on the
    CPU: the CPU baseline of the segment sum."""
    return y.new_zeros((num_nodes,) + tuple(y.shape[1:])).index_add_(0, index, y)


# torch_scatter's scatter_min / scatter_max (core/molecular_encoder.py:6,214; GET/get_clean/tools.py:110) --
# torch_scatter is absent here and unpinned by the reference (GET/env.yml: pyg::pytorch-scatter beside
# pytorch 1.13.1, the 2.1 series).  Its published CPU algorithm for dim 0 without `out`: out filled with the
# reduction's start value (numeric_limits::max() for the minimum, lowest() for the maximum) and arg with
# src.size(0); elements visited in ascending index, each replacing out[index[e]] and arg[index[e]] when
# strictly smaller (larger); finally out == start is set to 0.  Its CUDA kernel computes the same out by
# atomics and sets arg to any e whose value equals out.
def _rows(y) -> np.ndarray:
    y = np.asarray(y, np.float32)
    return y.reshape(-1, 1) if y.ndim == 1 else y.reshape(y.shape[0], int(np.prod(y.shape[1:])))


_START = {"float32": float(np.finfo(np.float32).max), "bfloat16": float(np.uint32(0x7F7F0000).view(np.float32))}


def scatter_minmax_loop(y: np.ndarray, index: np.ndarray, dim_size: int, maximum: bool = False,
                        dtype: str = "float32") -> tuple[np.ndarray, np.ndarray]:
    """The CPU algorithm above, literally, on [E] or [E, F] values (small inputs): (out, arg).
    Indices outside [0, dim_size) are skipped (the library drops them)."""
    y2 = _rows(y)
    e_n, f_n = y2.shape
    start = -_START[dtype] if maximum else _START[dtype]
    out = np.full((dim_size, f_n), start, np.float32)
    arg = np.full((dim_size, f_n), e_n, np.int64)
    for e in range(e_n):
        n = int(index[e])
        if not 0 <= n < dim_size:
            continue
        for f in range(f_n):
            v = y2[e, f]
            if (v > out[n, f]) if maximum else (v < out[n, f]):
                out[n, f] = v
                arg[n, f] = e
    out[out == np.float32(start)] = 0.0
    return out, arg


def scatter_minmax(y: np.ndarray, index: np.ndarray, dim_size: int, maximum: bool = False,
                   dtype: str = "float32") -> tuple[np.ndarray, np.ndarray]:
    """scatter_minmax_loop vectorised (any size): per (node, feature) the first edge, in ascending e, of
    those with the extreme value among the values strictly below (above) the start -- the element the
    sequential strict update keeps; NaN never compares below the start.  out is that edge's value."""
    y2 = _rows(y)
    e_n, f_n = y2.shape
    idx = np.asarray(index, np.int64)
    start = np.float32(-_START[dtype] if maximum else _START[dtype])
    out = np.zeros((dim_size, f_n), np.float32)
    arg = np.full((dim_size, f_n), e_n, np.int64)
    valid = (idx >= 0) & (idx < dim_size)
    for f in range(f_n):
        v = y2[:, f]
        ok = valid & ((v > start) if maximum else (v < start))
        e_ok = np.nonzero(ok)[0]
        if e_ok.size == 0:
            continue
        n_ok, v_ok = idx[e_ok], v[e_ok]
        order = np.lexsort((e_ok, -v_ok if maximum else v_ok, n_ok))
        n_sorted = n_ok[order]
        first = order[np.concatenate([[True], n_sorted[1:] != n_sorted[:-1]])]
        arg[n_ok[first], f] = e_ok[first]
        out[n_ok[first], f] = v_ok[first]
    return out, arg
