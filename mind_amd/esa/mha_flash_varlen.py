"""MABFlashVarlen / SABFlashVarlen / PMAFlashVarlen (esa/mha_flash_varlen.py) on the gfx950 kernels.

Same constructors, parameter names and forward signatures as
esa/mha_flash_varlen.py:26-248, and the same arithmetic, including its
departures from esa/mha.py:
  * V = fc_v(fc_k(K)) in the padding-free path (esa/mha_flash_varlen.py:155-156);
  * the padding-free path ignores adj_mask (:55-78, :129-201);
  * PMAFlashVarlen always takes the padded path (:248), attending to padding.
The padding-free path casts to bf16 as the reference does (:147-151), unpads
the valid tokens, runs varlen attention over cu_seqlens and pads the result
with zeros (flash-attn's pad_input) before fc_o + mish.
"""
from __future__ import annotations

import torch
from torch import nn
from torch.nn import functional as F
from torch.nn.init import xavier_normal_

from .activations import mish
from .attention import varlen_attention
from .mha import _heads, attn_dropout, dense_attention, masked_attention, tensor_masked_attention
from .packing import PackedSets


def _linear(layer: nn.Linear, x: torch.Tensor) -> torch.Tensor:
    """Linear in the input's dtype (what autocast does under the reference's bf16-mixed training)."""
    b = layer.bias.to(x.dtype) if layer.bias is not None else None
    return F.linear(x, layer.weight.to(x.dtype), b)


class MABFlashVarlen(nn.Module):
    def __init__(self, dim_Q, dim_K, dim_V, num_heads, dropout_p=0.0):
        super().__init__()
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

    def forward(self, Q, K, seq_lens=None, adj_mask=None):
        # attention dropout: dropout_p in training, 0 in eval (esa/mha_flash_varlen.py:115,181)
        if seq_lens is None:
            return self._forward_padded(Q, K, adj_mask)
        return self._forward_varlen(Q, K, seq_lens, adj_mask)

    def _forward_padded(self, Q, K, adj_mask=None):
        """SDPA fallback (esa/mha_flash_varlen.py:81-126): V = fc_v(K), all N positions."""
        if self.dim_V % self.num_heads:
            raise ValueError("Embedding dim is not divisible by nheads")
        input_dtype = Q.dtype
        model_dtype = self.fc_q.weight.dtype
        if Q.dtype != model_dtype:
            Q = Q.to(model_dtype)
            K = K.to(model_dtype)
        q = self.fc_q(Q)
        v = self.fc_v(K)
        k = self.fc_k(K)
        p = attn_dropout(self)
        if adj_mask is None:
            out = dense_attention(q, k, v, self.num_heads, p)
        elif isinstance(adj_mask, PackedSets):
            out = masked_attention(q, k, v, self.num_heads, adj_mask, packed=False, dropout_p=p)
        elif isinstance(adj_mask, torch.Tensor):   # SDPA's attn_mask (esa/mha_flash_varlen.py:112-117)
            out = tensor_masked_attention(q, k, v, self.num_heads, adj_mask, p)
        else:
            raise TypeError("adj_mask must be None, an EdgeAdjacency / NodeAdjacency descriptor, or a mask tensor")
        out = out.to(q.dtype)
        out = mish(self.fc_o(out), out)
        return out.to(input_dtype) if out.dtype != input_dtype else out

    def _forward_varlen(self, Q, K, seq_lens, adj_mask=None):
        """Padding-free path (esa/mha_flash_varlen.py:129-201); adj_mask is ignored as there."""
        if self.dim_V % self.num_heads:
            raise ValueError("Embedding dim is not divisible by nheads")
        b, n = Q.size(0), Q.size(1)
        input_dtype = Q.dtype
        if input_dtype != torch.float16:
            Q = Q.to(torch.bfloat16)
            K = K.to(torch.bfloat16)
        q = _linear(self.fc_q, Q)
        k = _linear(self.fc_k, K)
        v = _linear(self.fc_v, k)        # V from the projected K (esa/mha_flash_varlen.py:156)
        lens = torch.as_tensor(seq_lens, device=Q.device).to(torch.int64)
        valid = (torch.arange(n, device=Q.device)[None, :] < lens[:, None]).reshape(-1)
        index = torch.nonzero(valid).squeeze(1)
        cu = torch.zeros(b + 1, dtype=torch.int32, device=Q.device)
        cu[1:] = torch.cumsum(valid.view(b, n).sum(1), 0).to(torch.int32)
        d = q.shape[-1]
        h = self.num_heads
        qp = _heads(q.reshape(b * n, d).index_select(0, index), h)
        kp = _heads(k.reshape(b * n, d).index_select(0, index), h)
        vp = _heads(v.reshape(b * n, d).index_select(0, index), h)
        out_p = varlen_attention(qp, kp, vp, cu, cu, n, n, dropout_p=attn_dropout(self)).reshape(-1, d).to(q.dtype)
        out = q.new_zeros(b * n, d).index_copy(0, index, out_p).view(b, n, d)
        out = mish(_linear(self.fc_o, out), out)
        return out.to(input_dtype) if out.dtype != input_dtype else out


class SABFlashVarlen(nn.Module):
    def __init__(self, dim_in, dim_out, num_heads, dropout):
        super().__init__()
        self.mab = MABFlashVarlen(dim_in, dim_in, dim_out, num_heads, dropout)

    def forward(self, X, seq_lens=None, adj_mask=None):
        return self.mab(X, X, seq_lens=seq_lens, adj_mask=adj_mask)


class PMAFlashVarlen(nn.Module):
    def __init__(self, dim, num_heads, num_seeds, dropout):
        super().__init__()
        self.S = nn.Parameter(torch.Tensor(1, num_seeds, dim))
        self.num_seeds = num_seeds
        nn.init.xavier_normal_(self.S)
        self.mab = MABFlashVarlen(dim, dim, dim, num_heads, dropout_p=dropout)

    def forward(self, X, seq_lens=None, adj_mask=None):
        S = self.S.repeat(X.size(0), 1, 1)
        return self.mab(S, X, seq_lens=None, adj_mask=adj_mask)   # padded path, as the reference (:248)


def get_seq_lens_from_mask(mask):
    """esa/mha_flash_varlen.py:252-264."""
    return mask.sum(dim=1).to(torch.int32)


def create_padding_mask(seq_lens, max_len=None, device=None):
    """esa/mha_flash_varlen.py:267-286."""
    if device is None:
        device = seq_lens.device
    if max_len is None:
        max_len = int(seq_lens.max().item())
    b = seq_lens.size(0)
    return torch.arange(max_len, device=device).unsqueeze(0).expand(b, -1) < seq_lens.unsqueeze(1)
