"""Varlen attention over packed edge-token segments, on the gfx950 kernels.

``varlen_attention`` is the drop-in for ``flash_attn_varlen_func`` as the
reference calls it (esa/mha_flash_varlen.py:177-184: causal=False, dropout_p
in training, ``softmax_scale=None`` meaning 1/sqrt(head_dim)), extended with the
edge-adjacency mask of esa/masked_layers.py:121-142 evaluated on the fly from
per-token ``(src, dst)`` node ids.  Tensors are packed ``[total, heads,
head_dim]`` (head_dim 16, 24, 32 or 64: ESA's dim / heads) bf16 (MFMA kernels, fp32
softmax) or float32 (fp32 throughout) with int32 ``cu_seqlens``.  Backward is
deterministic.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from .. import _lib

HEAD_DIMS = (16, 24, 32, 64)   # head dims the kernels take
_SEED_MASK = (1 << 63) - 1


def _check_dropout(p: float) -> float:
    p = float(p)
    if not 0.0 <= p < 1.0:
        raise ValueError(f"dropout_p must be in [0, 1) (got {p})")
    return p


def draw_dropout_seed() -> int:
    """A fresh 62-bit dropout seed from torch's default CPU generator (so ``torch.manual_seed`` reproduces the
    keep masks of a run)."""
    return int(torch.randint(0, 1 << 62, (), dtype=torch.int64))


_DTYPES = {torch.bfloat16: _lib.ESA_BF16, torch.float32: _lib.ESA_F32}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"attention tensors must be bfloat16 or float32 (got {t.dtype})") from None


def _workspace(device: torch.device, total_q: int, total_k: int, heads: int, head_dim: int, dtype: int,
               mask_kind: int, nnz: int, backward: bool):
    lib = _lib.load()
    n = _lib.ctypes.c_size_t(0)
    _lib.check(lib.esa_varlen_attn_workspace_size(total_q, total_k, heads, head_dim, dtype, mask_kind, nnz,
                                                  int(backward), _lib.ctypes.byref(n)),
               "esa_varlen_attn_workspace_size")
    return torch.empty(max(int(n.value), 256), dtype=torch.uint8, device=device)


def _check_tokens(name: str, t: torch.Tensor, heads: int | None = None, dtype: torch.dtype | None = None,
                  head_dim: int | None = None) -> None:
    _dtype_code(t)
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} is {t.dtype}; all attention tensors must share one dtype ({dtype})")
    if t.dim() != 3 or t.shape[2] not in HEAD_DIMS:
        raise ValueError(f"{name} must be [total, heads, head_dim] with head_dim in {HEAD_DIMS} "
                         f"(got {tuple(t.shape)})")
    if head_dim is not None and t.shape[2] != head_dim:
        raise ValueError(f"{name} has head_dim {t.shape[2]}, expected {head_dim}")
    if heads is not None and t.shape[1] != heads:
        raise ValueError(f"{name} has {t.shape[1]} heads, expected {heads}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _check_index(name: str, t: torch.Tensor | None, n: int | None = None) -> None:
    if t is None:
        return
    if t.dtype != torch.int32 or t.dim() != 1 or not t.is_contiguous():
        raise TypeError(f"{name} must be a contiguous 1-D int32 tensor (got {t.dtype}, {tuple(t.shape)})")
    if n is not None and t.numel() != n:
        raise ValueError(f"{name} has {t.numel()} entries, expected {n}")


def edge_plan(edge_src, edge_dst, cu_seqlens_q, cu_seqlens_k=None) -> torch.Tensor:
    """The edge-mask plan of a batch (esa_edge_plan_build): a uint8 device tensor holding the share-an-endpoint
    mask of the edge tokens with node ids ``edge_src`` / ``edge_dst`` (int32 [T]) over the segments
    ``cu_seqlens_q`` / ``cu_seqlens_k`` (``cu_seqlens_k`` defaults to the same tensor: self-attention, a
    symmetric mask).  Built once per batch and passed as ``edge_plan=`` to every attention call over those
    tokens, as the reference builds its [B, N, N] mask once per batch (get_adj_mask_from_edge_index_edge,
    esa/masked_layers.py:217-268) for all masked layers.  Later calls must pass the same cu_seqlens tensors."""
    cu_k = cu_seqlens_q if cu_seqlens_k is None else cu_seqlens_k
    _lib.require_gpu(edge_src, edge_dst, cu_seqlens_q, cu_k)
    t = edge_src.numel()
    _check_index("edge_src", edge_src, t)
    _check_index("edge_dst", edge_dst, t)
    _check_index("cu_seqlens_q", cu_seqlens_q)
    batch = cu_seqlens_q.numel() - 1
    _check_index("cu_seqlens_k", cu_k, batch + 1)
    lib = _lib.load()
    n = _lib.ctypes.c_size_t(0)
    sym = cu_k.data_ptr() == cu_seqlens_q.data_ptr()
    _lib.check(lib.esa_edge_plan_size(t, t, int(sym), _lib.ctypes.byref(n)), "esa_edge_plan_size")
    plan = torch.empty(max(int(n.value), 256), dtype=torch.uint8, device=edge_src.device)
    rc = lib.esa_edge_plan_build(edge_src.data_ptr(), edge_dst.data_ptr(), cu_seqlens_q.data_ptr(), cu_k.data_ptr(),
                                 batch, t, t, plan.data_ptr(), plan.numel(), _lib.stream_of(edge_src))
    _lib.check(rc, "esa_edge_plan_build")
    return plan


def node_plan(adj_indptr, adj_indices, cu_seqlens_q, cu_seqlens_k=None, total_k: int | None = None) -> torch.Tensor:
    """The node-mode plan of a batch (esa_node_plan_build): a uint8 device tensor holding a copy of the CSR's
    indices, its transpose (per key token, the query rows that list it) and per query and key token its
    partner range and row bounds over the segments ``cu_seqlens_q`` / ``cu_seqlens_k`` (``cu_seqlens_k``
    defaults to the same tensor and ``total_k`` to the number of queries: self-attention; with distinct key
    segments ``total_k`` is required).  Built once per batch
    and passed as ``adj_plan=`` (with the same ``adj_indptr`` / ``adj_indices`` and cu_seqlens) to every
    attention call over that adjacency, so no call rebuilds it, as the reference builds its node bias once per
    batch (get_adj_mask_from_edge_index_node, esa/masked_layers.py:79-118) for all layers."""
    if cu_seqlens_k is not None and total_k is None:
        raise ValueError("node_plan over distinct key segments needs total_k (the number of key tokens)")
    cu_k = cu_seqlens_q if cu_seqlens_k is None else cu_seqlens_k
    _lib.require_gpu(adj_indptr, adj_indices, cu_seqlens_q, cu_k)
    _check_index("adj_indptr", adj_indptr)
    _check_index("adj_indices", adj_indices)
    _check_index("cu_seqlens_q", cu_seqlens_q)
    batch = cu_seqlens_q.numel() - 1
    _check_index("cu_seqlens_k", cu_k, batch + 1)
    tq, nnz = adj_indptr.numel() - 1, adj_indices.numel()
    tk = tq if total_k is None else int(total_k)
    lib = _lib.load()
    n = _lib.ctypes.c_size_t(0)
    _lib.check(lib.esa_node_plan_size(tq, tk, nnz, _lib.ctypes.byref(n)), "esa_node_plan_size")
    plan = torch.empty(max(int(n.value), 256), dtype=torch.uint8, device=adj_indptr.device)
    rc = lib.esa_node_plan_build(adj_indptr.data_ptr(), adj_indices.data_ptr(), cu_seqlens_q.data_ptr(),
                                 cu_k.data_ptr(), batch, tq, tk, nnz, plan.data_ptr(), plan.numel(),
                                 _lib.stream_of(adj_indptr))
    _lib.check(rc, "esa_node_plan_build")
    return plan


def edge_plan_bytes(total: int, symmetric: bool) -> int:
    """Bytes of an edge-mask plan over ``total`` tokens (esa_edge_plan_size); ``symmetric``: one cu_seqlens
    array for queries and keys (the plan then holds no key-tile lists)."""
    n = _lib.ctypes.c_size_t(0)
    _lib.check(_lib.load().esa_edge_plan_size(total, total, int(symmetric), _lib.ctypes.byref(n)),
               "esa_edge_plan_size")
    return int(n.value)


def node_plan_bytes(total_q: int, total_k: int, nnz: int) -> int:
    """Bytes of a node plan (esa_node_plan_size)."""
    n = _lib.ctypes.c_size_t(0)
    _lib.check(_lib.load().esa_node_plan_size(total_q, total_k, nnz, _lib.ctypes.byref(n)), "esa_node_plan_size")
    return int(n.value)


def _mask_args(tq: int, edge_src, edge_dst, adj_indptr, adj_indices, edge_plan=None, adj_plan=None, tk=None,
               symmetric=True):
    """(mask_kind, mask_a, mask_b, n_mask_edges) of the C ABI for the given mask tensors.

    The C ABI takes a plan without its size and reads it at the offsets the call's token counts give, so a
    plan smaller than those sizes need (one built for another batch) is refused here, before any launch."""
    if sum(x is not None for x in (edge_src, adj_indptr, edge_plan)) > 1:
        raise ValueError("give one mask: the edge mask (edge_src / edge_dst), its plan, or the node adjacency")
    tk = tq if tk is None else tk
    if adj_plan is not None:
        if adj_indptr is None or adj_indices is None:
            raise ValueError("adj_plan goes with the adj_indptr / adj_indices it was built from")
        _check_index("adj_indptr", adj_indptr, tq + 1)
        _check_index("adj_indices", adj_indices)
        need = node_plan_bytes(tq, tk, adj_indices.numel())
        if adj_plan.numel() < need:
            raise ValueError(f"adj_plan holds {adj_plan.numel()} bytes; a node plan over {tq} queries, {tk} keys "
                             f"and {adj_indices.numel()} entries needs {need} (built for another batch?)")
        if adj_plan.dtype != torch.uint8 or not adj_plan.is_cuda:
            raise ValueError("adj_plan must be the uint8 device tensor node_plan() returns")
        return _lib.ESA_MASK_NODE_PLAN, adj_indptr, adj_plan, adj_indices.numel()
    if edge_plan is not None:
        need = edge_plan_bytes(tq, symmetric)
        if edge_plan.numel() < need:
            raise ValueError(f"edge_plan holds {edge_plan.numel()} bytes; a plan over {tq} tokens"
                             f"{'' if symmetric else ' with distinct key segments'} needs {need} "
                             "(built for another batch?)")
        if edge_plan.dtype != torch.uint8 or not edge_plan.is_cuda:
            raise ValueError("edge_plan must be the uint8 device tensor edge_plan() returns")
        return _lib.ESA_MASK_EDGE_PLAN, edge_plan, None, 0
    if edge_src is not None:
        _check_index("edge_src", edge_src, tq)
        _check_index("edge_dst", edge_dst, tq)
        return _lib.ESA_MASK_EDGE, edge_src, edge_dst, 0
    if adj_indptr is not None:
        _check_index("adj_indptr", adj_indptr, tq + 1)
        _check_index("adj_indices", adj_indices)
        return _lib.ESA_MASK_NODE, adj_indptr, adj_indices, adj_indices.numel()
    return _lib.ESA_MASK_NONE, None, None, 0


def attn_fwd(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale,
             edge_src=None, edge_dst=None, adj_indptr=None, adj_indices=None, edge_plan=None, adj_plan=None,
             dropout_p=0.0, dropout_seed=0):
    """Raw forward: returns ``(out [Tq,H,hd] (dtype of q), softmax_lse [H,Tq] fp32)``.  With ``dropout_p`` > 0
    the keep mask is the hash of ``(dropout_seed, head, q, k)`` the C ABI defines; the backward must get the same
    ``dropout_p`` and seed."""
    dropout_p = _check_dropout(dropout_p)
    _lib.require_gpu(q, k, v, cu_seqlens_q, cu_seqlens_k, edge_src, edge_dst, adj_indptr, adj_indices, edge_plan,
                     adj_plan)
    heads, hd = q.shape[1], q.shape[-1]
    _check_tokens("q", q)
    _check_tokens("k", k, heads, q.dtype, hd)
    _check_tokens("v", v, heads, q.dtype, hd)
    if k.shape[0] != v.shape[0]:
        raise ValueError("k and v must have the same number of tokens")
    batch = cu_seqlens_q.numel() - 1
    _check_index("cu_seqlens_q", cu_seqlens_q)
    _check_index("cu_seqlens_k", cu_seqlens_k, batch + 1)
    tq, tk = q.shape[0], k.shape[0]
    mask_kind, mask_a, mask_b, nnz = _mask_args(tq, edge_src, edge_dst, adj_indptr, adj_indices, edge_plan, adj_plan,
                                             tk, cu_seqlens_k.data_ptr() == cu_seqlens_q.data_ptr())
    dt = _dtype_code(q)
    out = torch.empty_like(q)
    lse = torch.empty((heads, tq), dtype=torch.float32, device=q.device)
    ws = _workspace(q.device, tq, tk, heads, hd, dt, mask_kind, nnz, False)
    lib = _lib.load()
    rc = lib.esa_varlen_attn_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(), batch, tq, tk,
        int(max_seqlen_q), int(max_seqlen_k), heads, hd, dt, float(softmax_scale), dropout_p,
        int(dropout_seed) & _SEED_MASK, mask_kind, _lib.ptr(mask_a), _lib.ptr(mask_b), nnz, out.data_ptr(),
        lse.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(q))
    _lib.check(rc, "esa_varlen_attn_fwd")
    return out, lse


def attn_fwd_noalloc(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, out, lse,
                     edge_src=None, edge_dst=None, adj_indptr=None, adj_indices=None, edge_plan=None, adj_plan=None,
                     dropout_p=0.0, dropout_seed=0):
    """``attn_fwd`` into caller-provided ``out`` [Tq,H,hd] and ``lse`` [H,Tq] fp32 through
    esa_varlen_attn_fwd_noalloc: no workspace, no device allocation (the library's static per-GPU scratch;
    calls that overlap on one GPU race).  Raises EsaError (ESA_ERR_SCRATCH) for shapes beyond that scratch."""
    _lib.require_gpu(q, k, v, cu_seqlens_q, cu_seqlens_k, edge_src, edge_dst, adj_indptr, adj_indices, out, lse,
                     edge_plan, adj_plan)
    heads, hd = q.shape[1], q.shape[-1]
    _check_tokens("q", q)
    _check_tokens("k", k, heads, q.dtype, hd)
    _check_tokens("v", v, heads, q.dtype, hd)
    _check_tokens("out", out, heads, q.dtype, hd)
    if out.shape != q.shape:
        raise ValueError("out must have the shape of q")
    if lse.dtype != torch.float32 or tuple(lse.shape) != (heads, q.shape[0]) or not lse.is_contiguous():
        raise ValueError(f"lse must be a contiguous float32 [{heads}, {q.shape[0]}] tensor")
    batch = cu_seqlens_q.numel() - 1
    _check_index("cu_seqlens_q", cu_seqlens_q)
    _check_index("cu_seqlens_k", cu_seqlens_k, batch + 1)
    tq, tk = q.shape[0], k.shape[0]
    mask_kind, mask_a, mask_b, nnz = _mask_args(tq, edge_src, edge_dst, adj_indptr, adj_indices, edge_plan, adj_plan,
                                             tk, cu_seqlens_k.data_ptr() == cu_seqlens_q.data_ptr())
    rc = _lib.load().esa_varlen_attn_fwd_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(), batch, tq, tk,
        int(max_seqlen_q), int(max_seqlen_k), heads, hd, _dtype_code(q), float(softmax_scale),
        _check_dropout(dropout_p), int(dropout_seed) & _SEED_MASK, mask_kind, _lib.ptr(mask_a), _lib.ptr(mask_b), nnz, out.data_ptr(), lse.data_ptr(), _lib.stream_of(q))
    _lib.check(rc, "esa_varlen_attn_fwd_noalloc")
    return out, lse


def attn_bwd(dout, q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale,
             edge_src=None, edge_dst=None, adj_indptr=None, adj_indices=None, edge_plan=None, adj_plan=None,
             dropout_p=0.0, dropout_seed=0):
    """Raw backward: returns ``(dq, dk, dv)`` (dtype and shapes of q, k, v)."""
    dropout_p = _check_dropout(dropout_p)
    _lib.require_gpu(dout, q, k, v, out, lse)
    heads, hd = q.shape[1], q.shape[-1]
    _check_tokens("q", q)
    for name, t in (("dout", dout), ("k", k), ("v", v), ("out", out)):
        _check_tokens(name, t, heads, q.dtype, hd)
    if dout.shape != q.shape or out.shape != q.shape:
        raise ValueError("dout and out must have the shape of q")
    batch = cu_seqlens_q.numel() - 1
    tq, tk = q.shape[0], k.shape[0]
    mask_kind, mask_a, mask_b, nnz = _mask_args(tq, edge_src, edge_dst, adj_indptr, adj_indices, edge_plan, adj_plan,
                                             tk, cu_seqlens_k.data_ptr() == cu_seqlens_q.data_ptr())
    dt = _dtype_code(q)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = _workspace(q.device, tq, tk, heads, hd, dt, mask_kind, nnz, True)
    lib = _lib.load()
    rc = lib.esa_varlen_attn_bwd(
        dout.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
        cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(), batch, tq, tk, int(max_seqlen_q), int(max_seqlen_k),
        heads, hd, dt, float(softmax_scale), dropout_p, int(dropout_seed) & _SEED_MASK, mask_kind,
        _lib.ptr(mask_a), _lib.ptr(mask_b), nnz, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(),
        ws.numel(), _lib.stream_of(q))
    _lib.check(rc, "esa_varlen_attn_bwd")
    return dq, dk, dv


# ---- torch.library registration: the C-ABI entry points as torch operators (torch.ops.esa_hip.*), with
# fake (shape) implementations, so torch.compile / export see them as opaque ops, and autograd on the
# forward op.

@torch.library.custom_op("esa_hip::varlen_attn_fwd", mutates_args=())
def _op_varlen_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_q: torch.Tensor,
                   cu_seqlens_k: torch.Tensor, max_seqlen_q: int, max_seqlen_k: int, softmax_scale: float,
                   edge_src: Optional[torch.Tensor], edge_dst: Optional[torch.Tensor],
                   adj_indptr: Optional[torch.Tensor], adj_indices: Optional[torch.Tensor],
                   edge_plan: Optional[torch.Tensor] = None,
                   adj_plan: Optional[torch.Tensor] = None, dropout_p: float = 0.0,
                   dropout_seed: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    return attn_fwd(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, edge_src,
                    edge_dst, adj_indptr, adj_indices, edge_plan, adj_plan, dropout_p, dropout_seed)


@_op_varlen_fwd.register_fake
def _(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, edge_src, edge_dst,
      adj_indptr, adj_indices, edge_plan=None, adj_plan=None, dropout_p=0.0, dropout_seed=0):
    return torch.empty_like(q), q.new_empty((q.shape[1], q.shape[0]), dtype=torch.float32)


@torch.library.custom_op("esa_hip::varlen_attn_bwd", mutates_args=())
def _op_varlen_bwd(dout: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
                   lse: torch.Tensor, cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, max_seqlen_q: int,
                   max_seqlen_k: int, softmax_scale: float, edge_src: Optional[torch.Tensor],
                   edge_dst: Optional[torch.Tensor], adj_indptr: Optional[torch.Tensor],
                   adj_indices: Optional[torch.Tensor],
                   edge_plan: Optional[torch.Tensor] = None,
                   adj_plan: Optional[torch.Tensor] = None, dropout_p: float = 0.0,
                   dropout_seed: int = 0) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return attn_bwd(dout, q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale,
                    edge_src, edge_dst, adj_indptr, adj_indices, edge_plan, adj_plan, dropout_p, dropout_seed)


@_op_varlen_bwd.register_fake
def _(dout, q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, edge_src,
      edge_dst, adj_indptr, adj_indices, edge_plan=None, adj_plan=None, dropout_p=0.0, dropout_seed=0):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


def _varlen_setup(ctx, inputs, output):
    (q, k, v, cu_q, cu_k, max_q, max_k, scale, edge_src, edge_dst, adj_indptr, adj_indices, edge_plan, adj_plan,
     dropout_p, dropout_seed) = inputs
    out, lse = output
    ctx.save_for_backward(q, k, v, out, lse, cu_q, cu_k, edge_src, edge_dst, adj_indptr, adj_indices, edge_plan,
                          adj_plan)
    ctx.meta = (max_q, max_k, scale, dropout_p, dropout_seed)


def _varlen_backward(ctx, dout, _dlse):
    q, k, v, out, lse, cu_q, cu_k, edge_src, edge_dst, adj_indptr, adj_indices, edge_plan, adj_plan = ctx.saved_tensors
    max_q, max_k, scale, dropout_p, dropout_seed = ctx.meta
    dq, dk, dv = torch.ops.esa_hip.varlen_attn_bwd(dout.contiguous(), q, k, v, out, lse, cu_q, cu_k, max_q, max_k,
                                                   scale, edge_src, edge_dst, adj_indptr, adj_indices, edge_plan,
                                                   adj_plan, dropout_p, dropout_seed)
    return (dq, dk, dv) + (None,) * 13


torch.library.register_autograd("esa_hip::varlen_attn_fwd", _varlen_backward, setup_context=_varlen_setup)


def varlen_attention(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, dropout_p=0.0,
                     softmax_scale=None, causal=False, edge_src=None, edge_dst=None, return_lse=False,
                     adj_indptr=None, adj_indices=None, edge_plan=None, adj_plan=None, dropout_seed=None):
    """``flash_attn_varlen_func``-compatible entry (plus the ESA masks).

    q: [Tq, H, hd]; k, v: [Tk, H, hd] (hd 16, 24, 32 or 64), all bfloat16 or all float32;
    cu_seqlens_*: int32 [B+1].
    edge_src / edge_dst: optional int32 [Tq] node ids per token (self-attention
    only); token i then attends to token j of its segment iff i != j and the
    two edges share an endpoint (edge mode).
    edge_plan: optional, the same edge mask prebuilt by ``edge_plan()`` (instead of
    edge_src / edge_dst) and shared by every call over the batch.
    adj_indptr [Tq+1] / adj_indices [nnz]: optional int32 CSR adjacency (node
    mode): token i attends to the keys listed in its row, ascending, a
    repeated entry counting once.  adj_plan: optional, the node plan of that
    CSR from ``node_plan()``, shared by every call over the batch (the
    backward then reads its transpose).  With return_lse, also returns the
    (non-differentiable) softmax log-sum-exp [H, Tq]; -inf marks a query with
    no admissible key (its output is 0).
    dropout_p: attention dropout on the softmax probabilities (the reference's
    training-time p, esa/mha.py:76,82); the keep mask is a hash of
    (dropout_seed, head, query, key), the seed drawn from torch's CPU generator
    when None.  The lse is that of the undropped scores.
    """
    if causal:
        raise NotImplementedError("causal attention is not on the ESA path (the reference uses causal=False)")
    dropout_p = _check_dropout(dropout_p)
    if dropout_p > 0.0 and dropout_seed is None:
        dropout_seed = draw_dropout_seed()
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    if (edge_src is None) != (edge_dst is None):
        raise ValueError("edge_src and edge_dst must be given together")
    if (adj_indptr is None) != (adj_indices is None):
        raise ValueError("adj_indptr and adj_indices must be given together")
    out, lse = torch.ops.esa_hip.varlen_attn_fwd(q, k, v, cu_seqlens_q, cu_seqlens_k, int(max_seqlen_q),
                                                 int(max_seqlen_k), float(softmax_scale), edge_src, edge_dst,
                                                 adj_indptr, adj_indices, edge_plan, adj_plan, dropout_p,
                                                 int(dropout_seed or 0) & _SEED_MASK)
    return (out, lse) if return_lse else out


def _pma_workspace(device, batch, k_seeds, total_k, heads, head_dim, dtype, backward):
    lib = _lib.load()
    n = _lib.ctypes.c_size_t(0)
    _lib.check(lib.esa_pma_workspace_size(batch, k_seeds, total_k, heads, head_dim, dtype, int(backward),
                                          _lib.ctypes.byref(n)), "esa_pma_workspace_size")
    return torch.empty(max(int(n.value), 256), dtype=torch.uint8, device=device)


class _PMAAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, cu_k, max_k, scale, dropout_p, dropout_seed):
        batch, k_seeds, heads, hd = cu_k.numel() - 1, q.shape[0], q.shape[1], q.shape[2]
        dt = _dtype_code(q)
        out = torch.empty((batch * k_seeds, heads, hd), dtype=q.dtype, device=q.device)
        lse = torch.empty((heads, batch * k_seeds), dtype=torch.float32, device=q.device)
        ws = _pma_workspace(q.device, batch, k_seeds, k.shape[0], heads, hd, dt, False)
        rc = _lib.load().esa_pma_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), cu_k.data_ptr(), batch, k_seeds,
                                     k.shape[0], int(max_k), heads, hd, dt, float(scale), dropout_p, dropout_seed,
                                     out.data_ptr(), lse.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(q))
        _lib.check(rc, "esa_pma_fwd")
        ctx.save_for_backward(q, k, v, out, lse, cu_k)
        ctx.meta = (max_k, scale, dropout_p, dropout_seed)
        return out

    @staticmethod
    def backward(ctx, g):
        q, k, v, out, lse, cu_k = ctx.saved_tensors
        max_k, scale, dropout_p, dropout_seed = ctx.meta
        batch, k_seeds, heads, hd = cu_k.numel() - 1, q.shape[0], q.shape[1], q.shape[2]
        dt = _dtype_code(q)
        g = g.to(q.dtype).contiguous()
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        ws = _pma_workspace(q.device, batch, k_seeds, k.shape[0], heads, hd, dt, True)
        rc = _lib.load().esa_pma_bwd(g.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                     lse.data_ptr(), cu_k.data_ptr(), batch, k_seeds, k.shape[0], int(max_k), heads,
                                     hd, dt, float(scale), dropout_p, dropout_seed, dq.data_ptr(), dk.data_ptr(),
                                     dv.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(q))
        _lib.check(rc, "esa_pma_bwd")
        return dq, dk, dv, None, None, None, None, None


def pma_attention(q, k, v, cu_seqlens_k, max_seqlen_k, softmax_scale=None, dropout_p=0.0, dropout_seed=None):
    """Seed pooling of PMA (esa/mha.py:101-109): the k seed queries q [k, H, hd] (fc_q(S), shared by every
    set) attend over each set's keys k, v [Tk, H, hd] (sets by cu_seqlens_k [B+1], int32) -> [B * k, H, hd],
    set-major.  Equals varlen attention with the seeds repeated per set; q's gradient sums the sets'.
    dropout_p / dropout_seed as ``varlen_attention``'s, over the repeated seeds (query b * k + s)."""
    _lib.require_gpu(q, k, v, cu_seqlens_k)
    heads, hd = q.shape[1], q.shape[-1]
    _check_tokens("q", q)
    _check_tokens("k", k, heads, q.dtype, hd)
    _check_tokens("v", v, heads, q.dtype, hd)
    if k.shape[0] != v.shape[0]:
        raise ValueError("k and v must have the same number of tokens")
    _check_index("cu_seqlens_k", cu_seqlens_k)
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    dropout_p = _check_dropout(dropout_p)
    if dropout_p > 0.0 and dropout_seed is None:
        dropout_seed = draw_dropout_seed()
    return _PMAAttention.apply(q, k, v, cu_seqlens_k, max_seqlen_k, float(softmax_scale), dropout_p,
                               int(dropout_seed or 0) & _SEED_MASK)


def edge_mask_dense(edge_src, edge_dst, cu_seqlens, max_items):
    """Debug materialisation of the edge mask: uint8 [B, max_items, max_items]."""
    _lib.require_gpu(edge_src, edge_dst, cu_seqlens)
    _check_index("edge_src", edge_src)
    _check_index("edge_dst", edge_dst, edge_src.numel())
    _check_index("cu_seqlens", cu_seqlens)
    batch = cu_seqlens.numel() - 1
    out = torch.empty((batch, max_items, max_items), dtype=torch.uint8, device=edge_src.device)
    rc = _lib.load().esa_edge_mask_dense(edge_src.data_ptr(), edge_dst.data_ptr(), cu_seqlens.data_ptr(), batch,
                                         edge_src.numel(), int(max_items), out.data_ptr(), _lib.stream_of(edge_src))
    _lib.check(rc, "esa_edge_mask_dense")
    return out


def edge_plan_decode(plan: torch.Tensor, total: int, direction: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """Debug decode of an edge-mask plan (esa_edge_plan_decode): the admissible partners of every token as the
    attention kernels read them from ``plan`` (direction 0: the forward and dQ passes; 1: the dK/dV passes),
    as a CSR ``(indptr [total + 1], indices)`` of int32 device tensors, each row ascending."""
    _lib.require_gpu(plan)
    if plan.dtype != torch.uint8 or plan.numel() < edge_plan_bytes(total, True):
        raise ValueError("plan must be the uint8 device tensor edge_plan() returns for these tokens")
    lib = _lib.load()
    counts = torch.empty(max(total, 1), dtype=torch.int32, device=plan.device)
    st = _lib.stream_of(plan)
    _lib.check(lib.esa_edge_plan_decode(plan.data_ptr(), total, total, int(direction), None, counts.data_ptr(), st),
               "esa_edge_plan_decode")
    indptr = torch.zeros(total + 1, dtype=torch.int32, device=plan.device)
    indptr[1:] = torch.cumsum(counts[:total], 0)
    indices = torch.empty(max(int(indptr[-1]), 1), dtype=torch.int32, device=plan.device)
    _lib.check(lib.esa_edge_plan_decode(plan.data_ptr(), total, total, int(direction), indptr.data_ptr(),
                                        indices.data_ptr(), st), "esa_edge_plan_decode")
    return indptr, indices[: int(indptr[-1])]


def node_plan_sections(plan: torch.Tensor, total_q: int, total_k: int, nnz: int) -> dict[str, torch.Tensor]:
    """Views of a node plan's sections (esa_node_plan_sections): ``indices`` [nnz] (the CSR's copy),
    ``t_indptr`` [total_k + 1] and ``t_rows`` [nnz] (the transposed CSR the dK/dV pass reads), ``q_desc``
    [total_q, 4] and ``k_desc`` [total_k, 4] (per token: partner range lo, hi and row begin, end)."""
    if plan.dtype != torch.uint8 or plan.numel() < node_plan_bytes(total_q, total_k, nnz):
        raise ValueError("plan must be the uint8 tensor node_plan() returns for these sizes")
    off = (_lib.ctypes.c_size_t * 5)()
    _lib.check(_lib.load().esa_node_plan_sections(total_q, total_k, nnz, off), "esa_node_plan_sections")

    def ints(i, n):
        return plan[off[i]: off[i] + 4 * n].view(torch.int32)

    return {"indices": ints(0, nnz), "t_indptr": ints(1, total_k + 1), "t_rows": ints(2, nnz),
            "q_desc": ints(3, 4 * total_q).view(total_q, 4), "k_desc": ints(4, 4 * total_k).view(total_k, 4)}
