"""Textbook per-segment softmax attention (test infrastructure; see oracle/__init__.py).

Restates what the reference's attention calls compute on each graph:
flash_attn_varlen_func over cu_seqlens (esa/mha_flash_varlen.py:177-184),
memory_efficient_attention / SDPA with the additive edge bias (esa/mha.py:76,
:80-83), with softmax_scale = 1/sqrt(head_dim) by default.  A masked entry
is -inf here; the reference's -99999 bias gives the same probabilities
whenever a row has an admissible key (exp(-99999 + s - max) underflows to 0).
A row with no admissible key returns 0 and lse = -inf.

``dropout=(p, seed)``: attention dropout on the probabilities, out =
(P o Z / (1 - p)) V with the keep mask Z of oracle/dropout.py (the reference's
training-time p, esa/mha.py:76,82); lse is that of the undropped scores.
``dropout=(p, seed, q_ids, k_ids)``: the same with the tokens' global indices
(the mask's q and k) given per query / key row, for a subset of a batch.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import dropout as _drop
from .mask import edge_adjacency_segment, node_adjacency_segment


def _dropout_ids(dropout, tq, tk):
    """(p, seed, global query ids [tq], global key ids [tk]) of a dropout argument."""
    p, seed = dropout[0], dropout[1]
    q_ids = np.arange(tq) if len(dropout) < 3 else np.asarray(dropout[2], dtype=np.int64)
    k_ids = np.arange(tk) if len(dropout) < 4 else np.asarray(dropout[3], dtype=np.int64)
    return p, seed, q_ids, k_ids


def _dropout_scale(dropout, heads, qs, qe, ks, ke, h0, h1, dtype, tq=None, tk=None):
    """Z / (1 - p) as a [h1 - h0, Lq, Lk] tensor for the query / key rows qs..qe, ks..ke, or None."""
    if dropout is None or dropout[0] == 0:
        return None
    p, seed, q_ids, k_ids = _dropout_ids(dropout, max(qe, tq or 0), max(ke, tk or 0))
    z = _drop.keep_mask(p, seed, heads, q_ids[qs:qe], k_ids[ks:ke], h0, h1)
    return torch.as_tensor(z).to(dtype) * _drop.params(p, seed)[3]


def _segment_mask(edge_src, edge_dst, qs, qe, ks, ke, adj=None):
    if adj is not None:
        return torch.as_tensor(node_adjacency_segment(adj[0], adj[1], qs, qe, ks, ke))
    if edge_src is None:
        return None
    assert (qs, qe) == (ks, ke), "the edge mask is self-attention only"
    m = edge_adjacency_segment(np.asarray(edge_src), np.asarray(edge_dst), qs, qe)
    return torch.as_tensor(m)


def _head_chunks(h, lq, lk, budget=1 << 26):
    """Head ranges whose [heads, Lq, Lk] score block stays within ``budget`` elements (bounded memory)."""
    step = max(1, min(h, budget // max(1, lq * lk)))
    return [(a, min(h, a + step)) for a in range(0, h, step)]


def varlen_attention(q, k, v, cu_q, cu_k, scale, edge_src=None, edge_dst=None, dtype=torch.float64, adj=None,
                     dropout=None):
    """q [Tq,H,D], k/v [Tk,H,D] -> (out [Tq,H,D], lse [H,Tq]) in ``dtype``.

    ``edge_src`` / ``edge_dst``: edge-mode mask; ``adj`` = (indptr, indices):
    node-mode CSR adjacency (query i attends to the keys of row i).
    """
    q, k, v = (torch.as_tensor(t).cpu().to(dtype) for t in (q, k, v))
    cu_q = np.asarray(cu_q, dtype=np.int64)
    cu_k = np.asarray(cu_k, dtype=np.int64)
    tq, h, d = q.shape
    outs, lses = [], []
    for b in range(len(cu_q) - 1):
        qs, qe, ks, ke = int(cu_q[b]), int(cu_q[b + 1]), int(cu_k[b]), int(cu_k[b + 1])
        if qe == qs:
            continue
        if ke == ks:
            outs.append(torch.zeros(qe - qs, h, d, dtype=dtype))
            lses.append(torch.full((h, qe - qs), float("-inf"), dtype=dtype))
            continue
        m = _segment_mask(edge_src, edge_dst, qs, qe, ks, ke, adj)
        ob, lb = [], []
        for h0, h1 in _head_chunks(h, qe - qs, ke - ks):
            qb = q[qs:qe, h0:h1].permute(1, 0, 2)           # [h, Lq, D]
            kb = k[ks:ke, h0:h1].permute(1, 2, 0)           # [h, D, Lk]
            vb = v[ks:ke, h0:h1].permute(1, 0, 2)           # [h, Lk, D]
            s = torch.matmul(qb, kb) * scale                # [h, Lq, Lk]
            if m is not None:
                s = s.masked_fill(~m, float("-inf"))
            l = torch.logsumexp(s, dim=-1)                  # [h, Lq]
            # rows with no admissible key: every s is -inf; keep p = 0 without NaN
            p = torch.exp(s - torch.where(torch.isfinite(l), l, torch.zeros_like(l))[..., None])
            zs = _dropout_scale(dropout, h, qs, qe, ks, ke, h0, h1, dtype, tq, k.shape[0])
            if zs is not None:
                p = p * zs
            ob.append(torch.matmul(p, vb).permute(1, 0, 2))
            lb.append(l)
        outs.append(torch.cat(ob, 1))
        lses.append(torch.cat(lb, 0))
    out = torch.cat(outs, 0) if outs else torch.zeros(0, h, d, dtype=dtype)
    lse = torch.cat(lses, 1) if lses else torch.zeros(h, 0, dtype=dtype)
    return out, lse


def varlen_attention_bwd(dout, q, k, v, cu_q, cu_k, scale, edge_src=None, edge_dst=None, dtype=torch.float64,
                         adj=None, dropout=None):
    """Analytic gradients of ``varlen_attention``: (dq, dk, dv).

    With P = softmax(scale Q K^T + mask), O = P V, D = rowsum(dO * O):
    dV = P^T dO, dP = dO V^T, dS = P * (dP - D), dQ = scale dS K,
    dK = scale dS^T Q.  With dropout, W = Z / (1 - p): O = (P o W) V,
    dV = (P o W)^T dO, dS = P * (dP o W - D) (D = rowsum(dO * O) still,
    since sum_j P_ij W_ij dP_ij = dO_i . O_i).
    """
    dout, q, k, v = (torch.as_tensor(t).detach().cpu().to(dtype) for t in (dout, q, k, v))
    cu_q = np.asarray(cu_q, dtype=np.int64)
    cu_k = np.asarray(cu_k, dtype=np.int64)
    dq, dk, dv = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
    h = q.shape[1]
    for b in range(len(cu_q) - 1):
        qs, qe, ks, ke = int(cu_q[b]), int(cu_q[b + 1]), int(cu_k[b]), int(cu_k[b + 1])
        if qe == qs or ke == ks:
            continue
        m = _segment_mask(edge_src, edge_dst, qs, qe, ks, ke, adj)
        for h0, h1 in _head_chunks(h, qe - qs, ke - ks):
            qb = q[qs:qe, h0:h1].permute(1, 0, 2).contiguous()
            kb = k[ks:ke, h0:h1].permute(1, 0, 2).contiguous()
            vb = v[ks:ke, h0:h1].permute(1, 0, 2).contiguous()
            gb = dout[qs:qe, h0:h1].permute(1, 0, 2).contiguous()
            s = torch.matmul(qb, kb.transpose(1, 2).contiguous()) * scale
            if m is not None:
                s = s.masked_fill(~m, float("-inf"))
            l = torch.logsumexp(s, dim=-1)
            p = torch.exp(s - torch.where(torch.isfinite(l), l, torch.zeros_like(l))[..., None])
            zs = _dropout_scale(dropout, h, qs, qe, ks, ke, h0, h1, dtype, q.shape[0], k.shape[0])
            pw = p if zs is None else p * zs
            o = torch.matmul(pw, vb)
            dvb = torch.matmul(pw.transpose(1, 2).contiguous(), gb)
            dp = torch.matmul(gb, vb.transpose(1, 2).contiguous())
            if zs is not None:
                dp = dp * zs
            drow = (gb * o).sum(-1, keepdim=True)
            ds = p * (dp - drow)
            dq[qs:qe, h0:h1] = (torch.matmul(ds, kb) * scale).permute(1, 0, 2)
            dk[ks:ke, h0:h1] = (torch.matmul(ds.transpose(1, 2).contiguous(), qb) * scale).permute(1, 0, 2)
            dv[ks:ke, h0:h1] = dvb.permute(1, 0, 2)
    return dq, dk, dv


class _VarlenAttentionFn(torch.autograd.Function):
    """varlen_attention with the analytic backward above: saves only q, k, v (bounded memory for long
    segments; the backward recomputes the scores head chunk by head chunk)."""

    @staticmethod
    def forward(ctx, q, k, v, cu_q, cu_k, scale, edge_src, edge_dst, adj, dropout=None):
        out, _ = varlen_attention(q, k, v, cu_q, cu_k, scale, edge_src, edge_dst, dtype=q.dtype, adj=adj,
                                  dropout=dropout)
        ctx.save_for_backward(q, k, v)
        ctx.meta = (cu_q, cu_k, scale, edge_src, edge_dst, adj, dropout)
        return out

    @staticmethod
    def backward(ctx, g):
        q, k, v = ctx.saved_tensors
        cu_q, cu_k, scale, edge_src, edge_dst, adj, dropout = ctx.meta
        dq, dk, dv = varlen_attention_bwd(g, q, k, v, cu_q, cu_k, scale, edge_src, edge_dst, dtype=q.dtype, adj=adj,
                                          dropout=dropout)
        return dq, dk, dv, None, None, None, None, None, None, None


def masked_attention_pairs(q, k, v, cu_q, cu_k, scale, edge_src=None, edge_dst=None, adj=None, dropout=None):
    """The masked case of ``varlen_attention`` over the admissible (query, key) pairs only, as gathers and
    scatters that torch autograd differentiates: s_ij = scale q_i . k_j per head for the mask's pairs of each
    segment, softmax per query row (a row without pairs gives 0), out_i = sum_j p_ij v_j (p_ij Z_ij / (1 - p)
    with dropout).  Work and memory follow the mask's nonzeros, not L^2 (the protein-like edge masks are about
    1 % dense)."""
    cu_q = np.asarray(cu_q, dtype=np.int64)
    cu_k = np.asarray(cu_k, dtype=np.int64)
    rows, cols = [], []
    for b in range(len(cu_q) - 1):
        qs, qe, ks, ke = int(cu_q[b]), int(cu_q[b + 1]), int(cu_k[b]), int(cu_k[b + 1])
        if qe == qs or ke == ks:
            continue
        i, j = np.nonzero(np.asarray(_segment_mask(edge_src, edge_dst, qs, qe, ks, ke, adj)))
        rows.append(i + qs)
        cols.append(j + ks)
    tq, h, d = q.shape
    if not rows or sum(r.size for r in rows) == 0:
        return q.new_zeros(tq, h, d)
    r = torch.as_tensor(np.concatenate(rows))
    c = torch.as_tensor(np.concatenate(cols))
    sc = (q.index_select(0, r) * k.index_select(0, c)).sum(-1) * scale          # [P, H]
    mx = torch.full((tq, h), float("-inf"), dtype=q.dtype).scatter_reduce(
        0, r[:, None].expand(-1, h), sc.detach(), "amax", include_self=True)
    e = torch.exp(sc - mx.index_select(0, r))
    den = q.new_zeros(tq, h).index_add(0, r, e)
    p = e / den.index_select(0, r)
    if dropout is not None and dropout[0] > 0:
        pd, seed, q_ids, k_ids = _dropout_ids(dropout, tq, k.shape[0])
        z = _drop.keep_pairs(pd, seed, h, q_ids[r.numpy()], k_ids[c.numpy()])              # [H, P]
        p = p * torch.as_tensor(z.T).to(p.dtype) * _drop.params(pd, seed)[3]
    return q.new_zeros(tq, h, d).index_add(0, r, p[..., None] * v.index_select(0, c))


def varlen_attention_diff(q, k, v, cu_q, cu_k, scale, edge_src=None, edge_dst=None, adj=None, dropout=None):
    """``varlen_attention``'s output, differentiable in q, k, v: through ``varlen_attention_bwd`` without a
    mask, through ``masked_attention_pairs`` with one."""
    if edge_src is not None or adj is not None:
        return masked_attention_pairs(q, k, v, cu_q, cu_k, scale, edge_src, edge_dst, adj, dropout)
    return _VarlenAttentionFn.apply(q, k, v, cu_q, cu_k, scale, edge_src, edge_dst, adj, dropout)


def padded_sdpa(q, k, v, cu_q, cu_k, n, scale, pair_bias=None, graphs_per_call=4):
    """The reference's padded fallback on the CPU: MABFlashVarlen._forward_padded (esa/mha_flash_varlen.py:
    81-126) pads every set to ``n`` positions, [B, H, n, D], and calls torch's
    scaled_dot_product_attention with the key-padding mask (:112-117) -- here a few sets per call, which
    changes nothing per set.  ``pair_bias(b)`` may give set b's additive [Lq, Lk] bias (the masked layers'
    0 / -99999 bias of esa/mha.py:73-77).  Returns the valid query rows [Tq, H, D] (differentiable in q, k,
    v); padded query rows are computed and dropped, as the reference's unpad does."""
    cu_q = np.asarray(cu_q, dtype=np.int64)
    cu_k = np.asarray(cu_k, dtype=np.int64)
    tq, h, d = q.shape
    outs = []
    for b0 in range(0, len(cu_q) - 1, graphs_per_call):
        bb = list(range(b0, min(b0 + graphs_per_call, len(cu_q) - 1)))
        qp = q.new_zeros(len(bb), h, n, d)
        kp = k.new_zeros(len(bb), h, n, d)
        vp = v.new_zeros(len(bb), h, n, d)
        mask = torch.full((len(bb), 1, n, n), float("-inf"), dtype=q.dtype)
        for j, b in enumerate(bb):
            lq, lk = int(cu_q[b + 1] - cu_q[b]), int(cu_k[b + 1] - cu_k[b])
            qp[j, :, :lq] = q[cu_q[b]:cu_q[b + 1]].transpose(0, 1)
            kp[j, :, :lk] = k[cu_k[b]:cu_k[b + 1]].transpose(0, 1)
            vp[j, :, :lk] = v[cu_k[b]:cu_k[b + 1]].transpose(0, 1)
            mask[j, 0, :, :lk] = 0.0
            if pair_bias is not None:
                mask[j, 0, :lq, :lk] = pair_bias(b).to(q.dtype)
            mask[j, 0, lq:, :] = 0.0     # padded query rows: any finite row (dropped below)
        o = F.scaled_dot_product_attention(qp, kp, vp, attn_mask=mask, scale=scale)
        for j, b in enumerate(bb):
            outs.append(o[j, :, : int(cu_q[b + 1] - cu_q[b])].transpose(0, 1))
    return torch.cat(outs, 0) if outs else q.new_zeros(0, h, d)


def padded_attention(q, k, v, scale, bias=None, dtype=torch.float64):
    """Dense [B, N, H, D] attention with an optional additive bias [B, 1|H, Nq, Nk].

    Restates memory_efficient_attention(Q, K, V, attn_bias) at esa/mha.py:76
    (BMHK layout), which attends to every position including padding.
    """
    q, k, v = (torch.as_tensor(t).cpu().to(dtype) for t in (q, k, v))
    qb = q.permute(0, 2, 1, 3).contiguous()
    kb = k.permute(0, 2, 3, 1).contiguous()
    vb = v.permute(0, 2, 1, 3).contiguous()
    s = torch.matmul(qb, kb) * scale
    if bias is not None:
        s = s + torch.as_tensor(bias).cpu().to(dtype)
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, vb).permute(0, 2, 1, 3)
