"""Edge-token gather, deterministic CSR segmented sums and scatter_add on the gfx950 kernels.

``edge_gather(x, src, dst)`` builds the edge tokens ``[x[src] || x[dst]]`` of
core/pretraining_model.py:153-155 and esa/models.py:307-309 in one pass (no
intermediate ``x[src]`` / ``x[dst]`` tensors); its backward is two CSR
segmented sums (by src and by dst), accumulated in a fixed order, so the
gradient is bitwise reproducible — unlike the atomic scatter_add of the
reference's edge->node reductions (core/molecular_encoder.py:241-242).
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.ESA_F32, torch.bfloat16: _lib.ESA_BF16}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; use float32 or bfloat16") from None


def _as_index(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"{name} must be an integer tensor")
    return t.to(torch.int32).contiguous()


class CSR:
    """CSR grouping of ``num_edges`` items by an int key in [0, num_nodes).

    ``indptr`` [N+1] int32 and ``perm`` [E] int32: the edge ids of key n are
    ``perm[indptr[n]:indptr[n+1]]`` in ascending order (a stable sort).
    """

    def __init__(self, indptr: torch.Tensor, perm: torch.Tensor, num_nodes: int):
        self.indptr, self.perm, self.num_nodes = indptr, perm, num_nodes

    @classmethod
    def build(cls, keys: torch.Tensor, num_nodes: int) -> "CSR":
        keys = _as_index(keys, "keys")
        _lib.require_gpu(keys)
        lib = _lib.load()
        e = keys.numel()
        nbytes = ctypes.c_size_t(0)
        _lib.check(lib.esa_csr_workspace_size(e, num_nodes, ctypes.byref(nbytes)), "esa_csr_workspace_size")
        ws = torch.empty(max(int(nbytes.value), 256), dtype=torch.uint8, device=keys.device)
        indptr = torch.empty(num_nodes + 1, dtype=torch.int32, device=keys.device)
        perm = torch.empty(e, dtype=torch.int32, device=keys.device)
        _lib.check(lib.esa_csr_build(keys.data_ptr(), e, num_nodes, indptr.data_ptr(), perm.data_ptr(),
                                     ws.data_ptr(), ws.numel(), _lib.stream_of(keys)), "esa_csr_build")
        return cls(indptr, perm, num_nodes)


def segment_sum_csr(y: torch.Tensor, indptr: torch.Tensor, perm: torch.Tensor | None = None,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """out[n] = sum of rows y[perm[i]] (or y[i]) for i in [indptr[n], indptr[n+1]).

    fp32 accumulation in ascending i, one rounding at the end: deterministic.
    ``out`` ([N, F], dtype of y, contiguous) is written in place when given.
    """
    _lib.require_gpu(y, indptr, perm)
    if y.dim() != 2:
        raise ValueError("y must be [E, F]")
    y = y.contiguous()
    indptr = _as_index(indptr, "indptr")
    perm = None if perm is None else _as_index(perm, "perm")
    n = indptr.numel() - 1
    out = _output(out, (n, y.shape[1]), y)
    rc = _lib.load().esa_csr_segment_sum(y.data_ptr(), _lib.ptr(perm), indptr.data_ptr(), n, y.shape[1],
                                         _dtype_code(y), out.data_ptr(), _lib.stream_of(y))
    _lib.check(rc, "esa_csr_segment_sum")
    return out


def _output(out: torch.Tensor | None, shape: tuple, like: torch.Tensor) -> torch.Tensor:
    if out is None:
        return torch.empty(shape, dtype=like.dtype, device=like.device)
    if tuple(out.shape) != tuple(shape) or out.dtype != like.dtype or out.device != like.device \
            or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous {like.dtype} tensor of shape {tuple(shape)} on {like.device}")
    return out


def _gather_raw(x: torch.Tensor, src: torch.Tensor, dst: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    _lib.require_gpu(x, src, dst)
    x = x.contiguous()
    e = src.numel()
    out = _output(out, (e, 2 * x.shape[1]), x)
    rc = _lib.load().esa_edge_gather(x.data_ptr(), src.data_ptr(), dst.data_ptr(), e, x.shape[0], x.shape[1],
                                     _dtype_code(x), out.data_ptr(), _lib.stream_of(x))
    _lib.check(rc, "esa_edge_gather")
    return out


def _gather_bwd_raw(g: torch.Tensor, src_csr: CSR, dst_csr: CSR, num_nodes: int, features: int) -> torch.Tensor:
    g = g.contiguous()
    gx = torch.empty((num_nodes, features), dtype=g.dtype, device=g.device)
    rc = _lib.load().esa_edge_gather_bwd(g.data_ptr(), src_csr.perm.data_ptr(), src_csr.indptr.data_ptr(),
                                         dst_csr.perm.data_ptr(), dst_csr.indptr.data_ptr(), num_nodes, features,
                                         _dtype_code(g), gx.data_ptr(), _lib.stream_of(g))
    _lib.check(rc, "esa_edge_gather_bwd")
    return gx


# ---- torch.library registration of the gather / CSR entry points (torch.ops.esa_hip.*), with fake (shape)
# implementations for torch.compile / export.

@torch.library.custom_op("esa_hip::edge_gather", mutates_args=())
def _op_edge_gather(x: torch.Tensor, src: torch.Tensor, dst: torch.Tensor) -> torch.Tensor:
    return _gather_raw(x, src, dst)


@_op_edge_gather.register_fake
def _(x, src, dst):
    return x.new_empty((src.shape[0], 2 * x.shape[1]))


@torch.library.custom_op("esa_hip::csr_segment_sum", mutates_args=())
def _op_segment_sum(y: torch.Tensor, indptr: torch.Tensor, perm: Optional[torch.Tensor]) -> torch.Tensor:
    return segment_sum_csr(y, indptr, perm)


@_op_segment_sum.register_fake
def _(y, indptr, perm):
    return y.new_empty((indptr.shape[0] - 1, y.shape[1]))


@torch.library.custom_op("esa_hip::csr_build", mutates_args=())
def _op_csr_build(keys: torch.Tensor, num_nodes: int) -> tuple[torch.Tensor, torch.Tensor]:
    c = CSR.build(keys, num_nodes)
    return c.indptr, c.perm


@_op_csr_build.register_fake
def _(keys, num_nodes):
    return keys.new_empty((num_nodes + 1,), dtype=torch.int32), keys.new_empty((keys.shape[0],), dtype=torch.int32)


class _EdgeGather(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, src, dst, src_csr, dst_csr):
        ctx.save_for_backward(src, dst)
        ctx.csrs = (src_csr, dst_csr)
        ctx.shape = x.shape
        return torch.ops.esa_hip.edge_gather(x, src, dst)

    @staticmethod
    def backward(ctx, g):
        src, dst = ctx.saved_tensors
        src_csr, dst_csr = ctx.csrs
        n, f = ctx.shape
        if src_csr is None:
            src_csr = CSR.build(src, n)
        if dst_csr is None:
            dst_csr = CSR.build(dst, n)
        return _gather_bwd_raw(g, src_csr, dst_csr, n, f), None, None, None, None


def edge_gather(x: torch.Tensor, src: torch.Tensor, dst: torch.Tensor, src_csr: CSR | None = None,
                dst_csr: CSR | None = None) -> torch.Tensor:
    """Edge tokens ``[x[src] || x[dst]]`` ([E, 2F], dtype of x: float32 or bfloat16).

    Indices outside [0, N) produce zero rows.  The CSRs used by the backward
    are built on demand unless given (reuse them across layers of one batch).
    """
    if x.dim() != 2:
        raise ValueError("x must be [N, F]")
    src = _as_index(src, "src")
    dst = _as_index(dst, "dst")
    if src.shape != dst.shape or src.dim() != 1:
        raise ValueError("src and dst must be 1-D and of equal length")
    return _EdgeGather.apply(x, src, dst, src_csr, dst_csr)


# ---------------------------------------------------------------- fused edge-token projection

def gather_add(a: torch.Tensor, b: torch.Tensor, src: torch.Tensor, dst: torch.Tensor,
               bias: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """out[e] = a[src[e]] + b[dst[e]] + bias ([E, F], dtype of a), fp32 sums in that order, rounded once.

    a and b are [N, F] with unit column stride (row strides may differ, e.g. the two column halves of one
    [N, 2F] GEMM output).  Node ids outside [0, N) contribute zeros.
    """
    _lib.require_gpu(a, b, src, dst, bias)
    if a.dim() != 2 or b.shape != a.shape:
        raise ValueError("a and b must be [N, F] of equal shape")
    if a.dtype != b.dtype or (bias is not None and bias.dtype != a.dtype):
        raise TypeError("a, b and bias must share one dtype")
    for t, name in ((a, "a"), (b, "b")):
        if t.stride(1) != 1:
            raise ValueError(f"{name} needs unit column stride")
    src = _as_index(src, "src")
    dst = _as_index(dst, "dst")
    if bias is not None:
        bias = bias.contiguous()
    n, f = a.shape
    e = src.numel()
    out = _output(out, (e, f), a)
    rc = _lib.load().esa_edge_gather_add(a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0), _lib.ptr(bias),
                                         src.data_ptr(), dst.data_ptr(), e, n, f, _dtype_code(a), out.data_ptr(),
                                         _lib.stream_of(a))
    _lib.check(rc, "esa_edge_gather_add")
    return out


class _ScatterAdd(torch.autograd.Function):
    @staticmethod
    def forward(ctx, src, index, dim_size, csr):
        y = src.reshape(src.shape[0], math.prod(src.shape[1:]))
        out = segment_sum_csr(y, csr.indptr, csr.perm)
        ctx.save_for_backward(index)
        ctx.dim_size = dim_size
        return out.reshape((dim_size,) + tuple(src.shape[1:]))

    @staticmethod
    def backward(ctx, g):
        (index,) = ctx.saved_tensors
        idx = index.to(torch.int64)
        valid = (idx >= 0) & (idx < ctx.dim_size)
        grad = g.reshape(ctx.dim_size, math.prod(g.shape[1:])).index_select(0, idx.clamp(0, max(ctx.dim_size - 1, 0)))
        grad = grad.masked_fill(~valid.unsqueeze(1), 0)   # dropped edges: exactly 0, even beside Inf / NaN
        return grad.reshape((idx.numel(),) + tuple(g.shape[1:])), None, None, None


def scatter_add(src: torch.Tensor, index: torch.Tensor, dim: int = 0, dim_size: int | None = None,
                csr: CSR | None = None) -> torch.Tensor:
    """``torch_scatter.scatter_add(src, index, dim=0, dim_size)`` as the reference's encoder calls it
    (core/molecular_encoder.py:195-200, 213-215, 241-242): out[n] = sum of src[e] over edges with
    index[e] == n, on the deterministic CSR segment sum (fp32, ascending e, one rounding; the reference's
    atomic scatter sums in arbitrary order).  src is [E] or [E, ...] float32 / bfloat16 on the device;
    entries with an index outside [0, dim_size) are dropped.  ``csr`` (CSR.build(index, dim_size)) may be
    passed to reuse one grouping for several sums.  Differentiable in src (the gradient is a row gather)."""
    if dim != 0:
        raise NotImplementedError("scatter_add: only dim=0 (edge -> node rows) is on the reference path")
    index = _as_index(index, "index")
    if index.dim() != 1 or index.numel() != src.shape[0]:
        raise ValueError("index must be 1-D with one entry per row of src")
    if dim_size is None:
        dim_size = int(index.max()) + 1 if index.numel() else 0
    if csr is None:
        csr = CSR.build(index, dim_size)
    elif csr.num_nodes != dim_size:
        raise ValueError("csr was built for another dim_size")
    return _ScatterAdd.apply(src, index, dim_size, csr)


def segment_minmax_csr(y: torch.Tensor, indptr: torch.Tensor, perm: torch.Tensor | None = None,
                       maximum: bool = False, num_edges: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(out [N, F], arg [N, F] int64): per CSR segment the minimum (``maximum``: the maximum) of the rows
    y[perm[indptr[n]:indptr[n+1]]] with the edge id attaining it, the semantics of torch_scatter's
    scatter_min / scatter_max (no ``out``): strict comparison in ascending CSR position from the dtype's
    largest finite value (lowest for the maximum), so a tie keeps the first (lowest, with a stable CSR)
    edge id; a segment with nothing smaller (larger) than that start gives 0 and arg = num_edges
    (default: y's row count)."""
    _lib.require_gpu(y, indptr, perm)
    if y.dim() != 2:
        raise ValueError("y must be [E, F]")
    y = y.contiguous()
    indptr = _as_index(indptr, "indptr")
    perm = None if perm is None else _as_index(perm, "perm")
    n = indptr.numel() - 1
    e = y.shape[0] if num_edges is None else int(num_edges)
    out = torch.empty((n, y.shape[1]), dtype=y.dtype, device=y.device)
    arg = torch.empty((n, y.shape[1]), dtype=torch.int64, device=y.device)
    rc = _lib.load().esa_csr_segment_minmax(y.data_ptr(), _lib.ptr(perm), indptr.data_ptr(), n, y.shape[1],
                                           _dtype_code(y), int(maximum), e, out.data_ptr(), arg.data_ptr(),
                                           _lib.stream_of(y))
    _lib.check(rc, "esa_csr_segment_minmax")
    return out, arg


class _ScatterMinMax(torch.autograd.Function):
    @staticmethod
    def forward(ctx, src, dim_size, csr, maximum):
        y = src.reshape(src.shape[0], math.prod(src.shape[1:]))
        out, arg = segment_minmax_csr(y, csr.indptr, csr.perm, maximum)
        ctx.save_for_backward(arg)
        ctx.src_shape = tuple(src.shape)
        ctx.mark_non_differentiable(arg)
        tail = tuple(src.shape[1:])
        return out.reshape((dim_size,) + tail), arg.reshape((dim_size,) + tail)

    @staticmethod
    def backward(ctx, g, _g_arg):
        # torch_scatter's rule: the output's gradient goes to the element that attained it; untouched
        # outputs (arg = E) send theirs to a row past the end, which is cut off.  Every edge belongs to one
        # segment, so no two outputs of a feature share a target: the scatter is a permutation.
        (arg,) = ctx.saved_tensors
        e = ctx.src_shape[0]
        g2 = g.reshape(g.shape[0], math.prod(g.shape[1:]))
        grad = torch.zeros((e + 1, g2.shape[1]), dtype=g.dtype, device=g.device)
        grad.scatter_(0, arg.reshape(g2.shape), g2)
        return grad[:e].reshape(ctx.src_shape), None, None, None


def _scatter_minmax(src, index, dim, out, dim_size, csr, maximum, name):
    if out is not None:
        raise NotImplementedError(f"{name}: `out` is not on the reference path (core/molecular_encoder.py:214)")
    if dim not in (0, -src.dim()):
        raise NotImplementedError(f"{name}: only dim=0 (edge -> node rows) is on the reference path")
    index = _as_index(index, "index")
    if index.dim() != 1 or index.numel() != src.shape[0]:
        raise ValueError("index must be 1-D with one entry per row of src")
    if dim_size is None:
        dim_size = int(index.max()) + 1 if index.numel() else 0
    if csr is None:
        csr = CSR.build(index, dim_size)
    elif csr.num_nodes != dim_size:
        raise ValueError("csr was built for another dim_size")
    return _ScatterMinMax.apply(src, dim_size, csr, maximum)


def scatter_min(src: torch.Tensor, index: torch.Tensor, dim: int = 0, out: torch.Tensor | None = None,
                dim_size: int | None = None, csr: CSR | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """``torch_scatter.scatter_min(src, index, dim=0, dim_size=...)`` -> (out, argmin), as the encoder takes
    each node's closest close-range neighbour distance (core/molecular_encoder.py:214): out[n] = the minimum
    of src[e] over edges with index[e] == n, argmin[n] the edge attaining it (the lowest edge id on a tie;
    the reference's GPU kernel keeps any tied edge), 0 and src.shape[0] where no edge of n has a value below
    the dtype's largest finite value (torch_scatter's start).  On the deterministic CSR; src is [E] or
    [E, ...] float32 / bfloat16 on the device; edges with an index outside [0, dim_size) are dropped.
    Differentiable in src: the gradient of out[n] goes to src[argmin[n]]."""
    return _scatter_minmax(src, index, dim, out, dim_size, csr, False, "scatter_min")


def scatter_max(src: torch.Tensor, index: torch.Tensor, dim: int = 0, out: torch.Tensor | None = None,
                dim_size: int | None = None, csr: CSR | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """``torch_scatter.scatter_max`` -> (out, argmax): :func:`scatter_min` with the maximum (start: the
    dtype's lowest finite value)."""
    return _scatter_minmax(src, index, dim, out, dim_size, csr, True, "scatter_max")


class _EdgeTokenLinear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, src, dst, src_csr, dst_csr, edge_attr):
        n, f = x.shape
        d = weight.shape[0]
        w2 = torch.cat((weight[:, :f], weight[:, f:2 * f]), 0)   # [W_s ; W_d], [2D, F]
        pq = x @ w2.t()                                             # node-level projections [N, 2D]
        out = gather_add(pq[:, :d], pq[:, d:], src, dst, bias)
        w_e = None
        if edge_attr is not None:                                   # the edge-attribute block W_e, [D, F_e]
            w_e = weight[:, 2 * f:]
            out.add_(edge_attr @ w_e.t())
        ctx.save_for_backward(x, w2, src, dst, edge_attr, w_e)
        ctx.csrs = (src_csr, dst_csr)
        ctx.has_bias = bias is not None
        return out

    @staticmethod
    def backward(ctx, g):
        from .esa.linear import column_sum, weight_grad
        x, w2, src, dst, edge_attr, w_e = ctx.saved_tensors
        src_csr, dst_csr = ctx.csrs
        n, f = x.shape
        d = w2.shape[0] // 2
        g = g.contiguous()
        if src_csr is None:
            src_csr = CSR.build(src, n)
        if dst_csr is None:
            dst_csr = CSR.build(dst, n)
        # d(a[src] + b[dst]) / d(a, b): per-node sums of the edge gradients, in ascending edge order
        dpq = torch.cat((segment_sum_csr(g, src_csr.indptr, src_csr.perm),
                         segment_sum_csr(g, dst_csr.indptr, dst_csr.perm)), 1)   # [N, 2D]
        dx = dpq @ w2 if ctx.needs_input_grad[0] else None
        dweight = None
        if ctx.needs_input_grad[1]:
            dw2 = weight_grad(dpq, x).to(w2.dtype)                # [2D, F]
            parts = [dw2[:d], dw2[d:]]
            if edge_attr is not None:
                parts.append(weight_grad(g, edge_attr).to(w2.dtype))   # [D, F_e]
            dweight = torch.cat(parts, 1)                          # [D, 2F (+ F_e)]
        dbias = column_sum(g).to(g.dtype) if ctx.has_bias and ctx.needs_input_grad[2] else None
        dattr = g @ w_e if edge_attr is not None and ctx.needs_input_grad[7] else None
        return dx, dweight, dbias, None, None, None, None, dattr


def edge_token_linear(x: torch.Tensor, src: torch.Tensor, dst: torch.Tensor, weight: torch.Tensor,
                      bias: torch.Tensor | None = None, src_csr: CSR | None = None,
                      dst_csr: CSR | None = None, edge_attr: torch.Tensor | None = None) -> torch.Tensor:
    """``F.linear(torch.cat((x[src], x[dst](, edge_attr)), 1), weight, bias)`` without the [E, 2F] edge tokens.

    The Linear over concatenated endpoint features (core/pretraining_model.py:153-198, with the edge
    attributes appended when the batch has them, :157-159; the first layer of the edge MLP,
    esa/mlp_utils.py:28-32) splits by input block, W = [W_s | W_d (| W_e)]: one node-level GEMM
    x [W_s ; W_d]^T gives both endpoint projections, and the gather-add kernel writes
    out[e] = (x W_s^T)[src e] + (x W_d^T)[dst e] + bias; edge attributes add edge_attr W_e^T (one GEMM over
    the edges).  The backward sums the edge gradients per node through two CSRs (deterministic) and finishes
    with GEMMs (split-K weight gradients, a deterministic bias gradient).  Computes in the dtype of x
    (float32 or bfloat16); weight, bias and edge_attr must share it.  Mathematically equal to the
    reference; results differ from it only by summation order.
    """
    if x.dim() != 2:
        raise ValueError("x must be [N, F]")
    fe = 0 if edge_attr is None else edge_attr.shape[-1]
    if weight.dim() != 2 or weight.shape[1] != 2 * x.shape[1] + fe:
        raise ValueError("weight must be [D, 2F + F_e]")
    if (weight.dtype != x.dtype or (bias is not None and bias.dtype != x.dtype)
            or (edge_attr is not None and edge_attr.dtype != x.dtype)):
        raise TypeError("x, weight, bias and edge_attr must share one dtype")
    src = _as_index(src, "src")
    dst = _as_index(dst, "dst")
    if src.shape != dst.shape or src.dim() != 1:
        raise ValueError("src and dst must be 1-D and of equal length")
    if edge_attr is not None and (edge_attr.dim() != 2 or edge_attr.shape[0] != src.shape[0]):
        raise ValueError("edge_attr must be [E, F_e]")
    return _EdgeTokenLinear.apply(x, weight, bias, src, dst, src_csr, dst_csr,
                                  None if edge_attr is None else edge_attr.contiguous())


class EdgeTokenLinear(torch.nn.Module):
    """Drop-in for the ``nn.Linear(2F (+ F_e), D)`` applied to ``torch.cat((x[src], x[dst](, edge_attr)), 1)``:
    same parameter names and shapes (a reference state_dict loads), forward(x, src, dst, edge_attr=None) via
    ``edge_token_linear``."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True, edge_features: int = 0):
        super().__init__()
        lin = torch.nn.Linear(2 * in_features + edge_features, out_features, bias=bias)
        self.weight = lin.weight
        self.bias = lin.bias
        self.in_features, self.out_features, self.edge_features = in_features, out_features, edge_features

    def forward(self, x: torch.Tensor, src: torch.Tensor, dst: torch.Tensor, src_csr: CSR | None = None,
                dst_csr: CSR | None = None, edge_attr: torch.Tensor | None = None) -> torch.Tensor:
        if (edge_attr is None) != (self.edge_features == 0):
            raise ValueError(f"this layer takes {self.edge_features} edge features; got "
                             f"{'none' if edge_attr is None else edge_attr.shape[-1]}")
        return edge_token_linear(x, src, dst, self.weight, self.bias, src_csr, dst_csr, edge_attr)
