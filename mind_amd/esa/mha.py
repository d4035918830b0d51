"""MAB / SAB / PMA with the signatures of esa/mha.py, on the gfx950 kernels.

Constructors, parameter names (``fc_q``, ``fc_k``, ``fc_v``, ``fc_o``, ``S``,
``mab``) and the forward signatures match esa/mha.py:9-109, so existing
state_dicts load.  Attention semantics by ``adj_mask``:

  None            every query attends to every one of the N positions of its
                  batch element, padding included — what memory_efficient_attention
                  and SDPA compute at esa/mha.py:76 and :80-83 without a bias.
  EdgeAdjacency   the edge-adjacency mask of esa/masked_layers.py:121-142,
                  evaluated on the fly in the kernel (no [B, 1, N, N] bias).
  NodeAdjacency   the node-mode mask of esa/masked_layers.py:79-118 (query
                  src attends to key dst per edge) as a CSR adjacency.
                  For either descriptor ``xformers_or_torch_attn`` picks the semantics:
                    "hip"                 packed valid tokens only; a query with
                                          no admissible key gets 0;
                    "xformers" / "torch"  the reference's padded semantics
                                          exactly: a row whose bias is -99999
                                          everywhere (padding, an edge sharing no
                                          node, a node without out-edges) softmaxes
                                          over all N keys, as
                                          a constant bias shift leaves softmax
                                          unchanged.  (The "torch" backend's
                                          inverted bool mask, esa/masked_layers.py:
                                          264-265, is a reference defect and is
                                          not reproduced.)
  a tensor        the reference's own mask tensors: an additive float bias
                  [B, 1 | H, Nq, Nk] of 0 (attend) and -99999 (or any value
                  <= -1e4), as get_adj_mask_from_edge_index_* build it for
                  memory_efficient_attention (esa/mha.py:70-77), or a bool mask
                  (True = attend) as SDPA takes it (:79-84).  It becomes a CSR
                  adjacency over the padded [B * N] tokens (the node-mode
                  kernels); a row with no admissible key softmaxes over all Nk
                  keys, as the -99999 bias does.  Other bias values (a general
                  additive bias) and masks that differ between heads raise.

float32 inputs run the fp32 kernels; any other dtype runs the bf16 kernels with
fp32 softmax statistics, as the reference's bf16-mixed training does.

Attention dropout: ``dropout_p`` applies to the softmax probabilities in
training and not in eval, as ``p=self.dropout_p if self.training else 0`` at
esa/mha.py:76,82; the kernels evaluate a hashed keep mask per (seed, head,
query, key), the seed drawn per call from torch's CPU generator.
"""
from __future__ import annotations

import torch
from torch import nn
from torch.nn.init import xavier_normal_

from .activations import mish
from .attention import HEAD_DIMS, draw_dropout_seed, varlen_attention
from .packing import PackedSets

BACKENDS = ("xformers", "torch", "flash_varlen", "hip")


def _uniform_cu(batch: int, n: int, device) -> torch.Tensor:
    return torch.arange(batch + 1, device=device, dtype=torch.int32) * n


def _heads(x: torch.Tensor, heads: int) -> torch.Tensor:
    """[..., H * hd] -> contiguous [tokens, H, hd]: float32 stays float32 (the fp32 kernels), any other
    dtype runs on the bf16 kernels."""
    dt = torch.float32 if x.dtype == torch.float32 else torch.bfloat16
    return x.reshape(-1, heads, x.shape[-1] // heads).to(dt).contiguous()


def attn_dropout(mab) -> float:
    """The attention dropout a MAB applies now: its dropout_p in training, 0 in eval (esa/mha.py:76,82)."""
    return float(mab.dropout_p) if mab.training else 0.0


def dense_attention(q, k, v, heads, dropout_p=0.0):
    """Per-batch-element attention over all positions: q [B, Nq, D], k/v [B, Nk, D] -> [B, Nq, D]."""
    b, nq, d = q.shape
    nk = k.shape[1]
    if d % heads or d // heads not in HEAD_DIMS:
        raise ValueError(f"head_dim {d / heads:g} is not supported by the kernels {HEAD_DIMS}")
    out = varlen_attention(_heads(q, heads), _heads(k, heads), _heads(v, heads), _uniform_cu(b, nq, q.device),
                           _uniform_cu(b, nk, q.device), nq, nk, dropout_p=dropout_p)
    return out.reshape(b, nq, d)


def masked_attention(q, k, v, heads, mask: PackedSets, packed: bool, dropout_p=0.0):
    """Masked self-attention (edge or node mode) over [B, N, D] inputs laid out as ``mask`` says."""
    b, n, d = q.shape
    if k.shape[1] != n or n != mask.max_items or b != mask.batch_size:
        raise ValueError("the mask needs queries and keys in the descriptor's [B, N] layout")
    if packed:
        cu = mask.cu_seqlens
        out = varlen_attention(_heads(mask.unpad(q), heads), _heads(mask.unpad(k), heads),
                               _heads(mask.unpad(v), heads), cu, cu, n, n, dropout_p=dropout_p,
                               **mask.kernel_mask(padded=False))
        return mask.pad(out.reshape(-1, d))
    cu = _uniform_cu(b, n, q.device)
    qh, kh, vh = _heads(q, heads), _heads(k, heads), _heads(v, heads)
    seed = draw_dropout_seed() if dropout_p > 0 else 0   # one keep mask for both calls
    out_m, lse = varlen_attention(qh, kh, vh, cu, cu, n, n, return_lse=True, dropout_p=dropout_p, dropout_seed=seed,
                                  **mask.kernel_mask(padded=True))
    out_d = varlen_attention(qh, kh, vh, cu, cu, n, n, dropout_p=dropout_p, dropout_seed=seed)
    dead = torch.isneginf(lse[0]).view(-1, 1, 1)   # the mask is the same for every head
    return torch.where(dead, out_d, out_m).reshape(b, n, d)


MASK_THRESHOLD = -1.0e4   # additive bias at or below this drops the pair (exp underflows to 0 in fp32)


def tensor_mask_csr(mask: torch.Tensor, b: int, nq: int, nk: int, heads: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The reference's dense mask tensor as a CSR adjacency over padded tokens: (indptr [B*Nq + 1], indices
    [nnz]) with key token b * Nk + j listed for query b * Nq + i when the pair may attend.

    ``mask``: float bias (0 keeps, <= -1e4 drops) or bool (True keeps), shape broadcastable to
    [B, H, Nq, Nk] with one pattern for all heads (the reference's [B, 1, N, N] expanded over heads,
    esa/mha.py:73).  Synchronises with the host (the nonzero count sizes the CSR).
    """
    if mask.dim() == 3:
        mask = mask.unsqueeze(1)
    if mask.dim() != 4 or mask.shape[0] != b or tuple(mask.shape[2:]) != (nq, nk) or mask.shape[1] not in (1, heads):
        raise ValueError(f"mask of shape {tuple(mask.shape)} does not match [B={b}, 1 or H={heads}, {nq}, {nk}]")
    if mask.dtype == torch.bool:
        keep = mask
    elif mask.is_floating_point():
        general = (mask != 0) & (mask > MASK_THRESHOLD)
        if bool(general.any()):
            raise NotImplementedError("only masking biases are supported: 0 (attend) or <= -1e4 (drop), as "
                                      "get_adj_mask_from_edge_index_* build them; a general additive bias is not")
        keep = mask == 0
    else:
        raise TypeError(f"a mask tensor must be bool or floating point (got {mask.dtype})")
    if keep.shape[1] > 1 and not bool((keep == keep[:, :1]).all()):
        raise NotImplementedError("masks that differ between heads are not supported")
    nz = keep[:, 0].nonzero()
    rows = nz[:, 0] * nq + nz[:, 1]
    indices = (nz[:, 0] * nk + nz[:, 2]).to(torch.int32).contiguous()
    bounds = torch.arange(b * nq + 1, device=mask.device, dtype=rows.dtype)
    indptr = torch.searchsorted(rows.contiguous(), bounds).to(torch.int32)
    return indptr, indices


def tensor_masked_attention(q, k, v, heads, mask: torch.Tensor, dropout_p=0.0):
    """Attention over [B, N, D] inputs with the reference's dense mask tensor (padded semantics: a row whose
    pairs are all dropped attends to all Nk keys, as a constant -99999 bias leaves softmax unchanged)."""
    b, nq, d = q.shape
    nk = k.shape[1]
    indptr, indices = tensor_mask_csr(mask.to(q.device), b, nq, nk, heads)
    cu_q, cu_k = _uniform_cu(b, nq, q.device), _uniform_cu(b, nk, q.device)
    qh, kh, vh = _heads(q, heads), _heads(k, heads), _heads(v, heads)
    seed = draw_dropout_seed() if dropout_p > 0 else 0   # one keep mask for both calls
    out_m, lse = varlen_attention(qh, kh, vh, cu_q, cu_k, nq, nk, return_lse=True, adj_indptr=indptr,
                                  adj_indices=indices, dropout_p=dropout_p, dropout_seed=seed)
    out_d = varlen_attention(qh, kh, vh, cu_q, cu_k, nq, nk, dropout_p=dropout_p, dropout_seed=seed)
    dead = torch.isneginf(lse[0]).view(-1, 1, 1)   # one pattern for every head
    return torch.where(dead, out_d, out_m).reshape(b, nq, d)


class MAB(nn.Module):
    """Multihead attention block (esa/mha.py:9-89): out = O + mish(fc_o(O)), V = fc_v(K)."""

    def __init__(self, dim_Q, dim_K, dim_V, num_heads, dropout_p=0.0, xformers_or_torch_attn="xformers"):
        super().__init__()
        if xformers_or_torch_attn not in BACKENDS:
            raise ValueError(f"unknown attention backend {xformers_or_torch_attn!r}; one of {BACKENDS}")
        self.xformers_or_torch_attn = xformers_or_torch_attn
        self.dim_Q, self.dim_K, self.dim_V = dim_Q, dim_K, dim_V
        self.num_heads = num_heads
        self.dropout_p = dropout_p
        self.fc_q = nn.Linear(dim_Q, dim_V, bias=True)
        self.fc_k = nn.Linear(dim_K, dim_V, bias=True)
        self.fc_v = nn.Linear(dim_K, dim_V, bias=True)
        self.fc_o = nn.Linear(dim_V, dim_V, bias=True)
        xavier_normal_(self.fc_q.weight)
        xavier_normal_(self.fc_k.weight)
        xavier_normal_(self.fc_v.weight)
        xavier_normal_(self.fc_o.weight)

    def forward(self, Q, K, adj_mask=None):
        if self.dim_V % self.num_heads:
            raise ValueError("Embedding dim is not divisible by nheads")
        p = attn_dropout(self)
        q = self.fc_q(Q)
        v = self.fc_v(K)
        k = self.fc_k(K)
        if adj_mask is None:
            out = dense_attention(q, k, v, self.num_heads, p)
        elif isinstance(adj_mask, PackedSets):
            out = masked_attention(q, k, v, self.num_heads, adj_mask, packed=self.xformers_or_torch_attn == "hip",
                                   dropout_p=p)
        elif isinstance(adj_mask, torch.Tensor):
            out = tensor_masked_attention(q, k, v, self.num_heads, adj_mask, p)
        else:
            raise TypeError("adj_mask must be None, an EdgeAdjacency / NodeAdjacency descriptor, or a mask tensor")
        out = out.to(q.dtype)
        return mish(self.fc_o(out), out)


class SAB(nn.Module):
    """Self-attention block (esa/mha.py:92-98)."""

    def __init__(self, dim_in, dim_out, num_heads, dropout, xformers_or_torch_attn):
        super().__init__()
        self.mab = MAB(dim_in, dim_in, dim_out, num_heads, dropout, xformers_or_torch_attn)

    def forward(self, X, adj_mask=None):
        return self.mab(X, X, adj_mask=adj_mask)


class PMA(nn.Module):
    """Pooling by multihead attention with learned seeds S [1, k, dim] (esa/mha.py:101-109).

    Without ``seq_lens`` the seeds attend over all N positions (the reference,
    which passes no mask at its call site, esa/masked_layers.py:593).  With
    ``seq_lens`` (an int tensor [B] or a packed-set descriptor) they attend over each
    set's valid tokens only.
    """

    def __init__(self, dim, num_heads, num_seeds, dropout, xformers_or_torch_attn):
        super().__init__()
        self.S = nn.Parameter(torch.Tensor(1, num_seeds, dim))
        nn.init.xavier_normal_(self.S)
        self.mab = MAB(dim, dim, dim, num_heads, dropout_p=dropout, xformers_or_torch_attn=xformers_or_torch_attn)

    def forward(self, X, adj_mask=None, seq_lens=None):
        S = self.S.repeat(X.size(0), 1, 1)
        if seq_lens is None:
            return self.mab(S, X, adj_mask=adj_mask)
        return pooled_attention(self.mab, S, X, seq_lens)


def pooled_attention(mab: MAB, S: torch.Tensor, X: torch.Tensor, seq_lens) -> torch.Tensor:
    """MAB(S, X) with each batch element's keys restricted to its first seq_lens[b] tokens."""
    b, n, d = X.shape
    k_seeds = S.shape[1]
    if isinstance(seq_lens, PackedSets):
        xk = seq_lens.unpad(X)
        cu_k = seq_lens.cu_seqlens
    else:
        lens = seq_lens.to(device=X.device, dtype=torch.int64)
        valid = torch.arange(n, device=X.device)[None, :] < lens[:, None]
        xk = X.reshape(b * n, d)[valid.reshape(-1)]
        cu_k = torch.zeros(b + 1, dtype=torch.int32, device=X.device)
        cu_k[1:] = torch.cumsum(lens, 0).to(torch.int32)
    q = mab.fc_q(S)
    v = mab.fc_v(xk)
    k = mab.fc_k(xk)
    h = mab.num_heads
    out = varlen_attention(_heads(q, h), _heads(k, h), _heads(v, h), _uniform_cu(b, k_seeds, X.device), cu_k,
                           k_seeds, n, dropout_p=attn_dropout(mab))
    out = out.reshape(b, k_seeds, d).to(q.dtype)
    return mish(mab.fc_o(out), out)

