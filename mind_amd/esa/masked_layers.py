"""ESA backbone blocks with the interfaces of esa/masked_layers.py.

``SABComplete``, ``PMAComplete`` and ``ESA`` keep the constructor arguments,
submodule names and the tuple-in / tuple-out forwards of
esa/masked_layers.py:271-936, so a PretrainingESAModel or Estimator can hold
them unchanged and existing state_dicts load.  The difference is the mask:
``get_adj_mask_from_edge_index_edge`` returns an ``EdgeAdjacency`` descriptor
(O(E) device memory) instead of the [B, 1, N, N] bias built from a global
E x E comparison (esa/masked_layers.py:121-142, 217-268); the attention
kernels evaluate the share-an-endpoint predicate from it on the fly.
``get_adj_mask_from_edge_index_node`` returns a ``NodeAdjacency`` (a CSR of
the edges) instead of the node-mode bias (esa/masked_layers.py:79-118).

Backend ``xformers_or_torch_attn``:
  "xformers" / "torch"  the reference's padded semantics (see mha.py);
  "flash_varlen"        the reference's MABFlashVarlen path, quirks included
                        (seq_lens = node counts per graph, mask dropped,
                        V = fc_v(fc_k(K)), esa/masked_layers.py:422-438);
  "hip"                 native packed path: every attention layer works on the
                        valid tokens only (edge counts per graph), the masked
                        layers apply the edge mask, PMA pools over valid tokens.
                        ESA runs its encoder and the PMA's keys on the packed
                        [T, D] tokens end to end (layer norms, projections and
                        MLPs included), so no work is spent on padding; only the
                        returned token embeddings are padded again (zeros at
                        padding slots).
"""
from __future__ import annotations

import contextlib

import torch
from torch import nn
from torch.nn import functional as F

from .activations import mab_epilogue, mish
from .attention import pma_attention, varlen_attention
from .layer_norm import layer_norm
from .linear import apply, param_casts, qkv_projection
from .mha import PMA, SAB, _heads, attn_dropout, pooled_attention
from .mha_flash_varlen import PMAFlashVarlen, SABFlashVarlen
from .mlp_utils import GatedMLPMulti, SmallMLP
from .norm_layers import LN
from .packing import EdgeAdjacency, NodeAdjacency, PackedSets


def get_adj_mask_from_edge_index_edge(edge_index, batch_size, max_items, batch_mapping, xformers_or_torch_attn=None,
                                      use_bfloat16=True, device=None):
    """Edge-adjacency mask descriptor for the edge tokens of a batch.

    Replaces esa/masked_layers.py:217-268 (same arguments).  Token e is edge
    e of ``edge_index``; tokens e, f of one graph attend iff e != f and the
    edges share an endpoint.
    """
    return EdgeAdjacency.from_edge_index(edge_index, batch_mapping, batch_size, max_items)


def get_adj_mask_from_edge_index_node(edge_index, batch_size, max_items, batch_mapping, xformers_or_torch_attn=None,
                                      use_bfloat16=True, device=None):
    """Node-mode mask descriptor for the node tokens of a batch.

    Replaces esa/masked_layers.py:79-118 (same arguments): instead of the
    [B, 1, N, N] bias with 0 at (graph, local src, local dst) of every edge,
    a CSR adjacency by query node (``NodeAdjacency``); query node src attends
    to key node dst for every edge src -> dst.
    """
    return NodeAdjacency.from_edge_index(edge_index, batch_mapping, batch_size, max_items)


def _backend_check(name: str) -> None:
    if name not in ("xformers", "torch", "flash_varlen", "hip"):
        raise ValueError(f"unknown attention backend {name!r}")


class SABComplete(nn.Module):
    """Pre/post-norm SAB / MAB block (esa/masked_layers.py:271-494)."""

    def __init__(self, dim_in, dim_out, num_heads, dropout, idx, norm_type, use_mlp=False, mlp_hidden_size=64,
                 mlp_type="standard", node_or_edge="edge", xformers_or_torch_attn="xformers", residual_dropout=0,
                 set_max_items=0, use_bfloat16=True, num_mlp_layers=3, pre_or_post="pre",
                 num_layers_for_residual=0, use_mlp_ln=False, mlp_dropout=0, use_equivariant=False,
                 equivariant_lmax=2, equivariant_num_features=16, equivariant_fusion_method="add",
                 equivariant_cross_connection=True):
        super().__init__()
        _backend_check(xformers_or_torch_attn)
        if use_equivariant:
            raise NotImplementedError("EquivariantSAB (esa/equivariant_sab.py) is outside the ESA attention path")
        if pre_or_post != "pre":
            raise NotImplementedError("post-norm blocks are not on the benchmarked path (every config is pre-norm)")
        if norm_type != "LN":
            raise NotImplementedError("BatchRenorm blocks are not on the HIP path; use norm_type='LN'")
        self.dim_in, self.dim_out, self.num_heads = dim_in, dim_out, num_heads
        self.use_mlp, self.idx, self.mlp_hidden_size = use_mlp, idx, mlp_hidden_size
        self.node_or_edge = node_or_edge
        self.xformers_or_torch_attn = xformers_or_torch_attn
        self.residual_dropout = residual_dropout
        self.set_max_items = set_max_items
        self.use_bfloat16 = use_bfloat16
        self.num_mlp_layers = num_mlp_layers
        self.pre_or_post = pre_or_post
        self.use_equivariant = False
        if dim_in != dim_out:
            self.proj_1 = nn.Linear(dim_in, dim_out)
        if xformers_or_torch_attn == "flash_varlen":
            self.sab = SABFlashVarlen(dim_in, dim_out, num_heads, dropout)
        else:
            self.sab = SAB(dim_in, dim_out, num_heads, dropout, xformers_or_torch_attn)
        self.norm = LN(dim_in, num_elements=set_max_items if idx != 2 else None)
        self.mlp_type = mlp_type
        if use_mlp:
            cls = SmallMLP if mlp_type == "standard" else GatedMLPMulti
            self.mlp = cls(in_dim=dim_out, out_dim=dim_out, inter_dim=mlp_hidden_size, dropout_p=mlp_dropout,
                           num_layers=num_mlp_layers, use_ln=use_mlp_ln)
        self.norm_mlp = LN(dim_out, num_elements=set_max_items if idx != 2 else None)

    def forward(self, inp):
        X, edge_index, batch_mapping, max_items, adj_mask = inp[:5]
        X = self.norm(X)
        if isinstance(self.sab, SABFlashVarlen):
            # the reference's seq_lens: node counts per graph, mask dropped (esa/masked_layers.py:422-438)
            seq_lens = torch.bincount(batch_mapping, minlength=X.size(0)).to(torch.int32)
            out_attn = self.sab(X, seq_lens=seq_lens, adj_mask=None)
        elif self.idx == 1:
            out_attn = self.sab(X, adj_mask)
        elif self.idx == 0 and self.xformers_or_torch_attn == "hip" and isinstance(adj_mask, PackedSets):
            out_attn = _sab_valid_only(self.sab, X, adj_mask)
        else:
            out_attn = self.sab(X, None)
        if out_attn.shape[-1] != X.shape[-1]:
            X = self.proj_1(X)
        out = X + out_attn
        if self.use_mlp:
            out_mlp = self.mlp(self.norm_mlp(out))
            if out.shape[-1] == out_mlp.shape[-1]:
                out = out_mlp + out
        if self.residual_dropout > 0:
            out = F.dropout(out, p=self.residual_dropout)
        return out, edge_index, batch_mapping, max_items, adj_mask


def _sab_valid_only(sab: SAB, X: torch.Tensor, tokens: PackedSets) -> torch.Tensor:
    """Unmasked self-attention over each graph's valid tokens (the "hip" backend's S layers)."""
    mab = sab.mab
    q = apply(mab.fc_q, X)
    v = apply(mab.fc_v, X)
    k = apply(mab.fc_k, X)
    h, d, n = mab.num_heads, q.shape[-1], X.shape[1]
    cu = tokens.cu_seqlens
    out = varlen_attention(_heads(tokens.unpad(q), h), _heads(tokens.unpad(k), h), _heads(tokens.unpad(v), h),
                           cu, cu, n, n, dropout_p=attn_dropout(mab))
    out = tokens.pad(out.reshape(-1, d)).to(q.dtype)
    return mish(apply(mab.fc_o, out), out)


def _packed_mab(mab, xq: torch.Tensor, xk: torch.Tensor, cu_q: torch.Tensor, cu_k: torch.Tensor, max_q: int,
                max_k: int, mask_kwargs: dict, residual: torch.Tensor | None = None) -> torch.Tensor:
    """MAB (esa/mha.py:48-89, V = fc_v(K)) on packed rows: queries xq [Tq, D] and keys xk [Tk, D] grouped by
    cu_q / cu_k -> [Tq, D] (``xk is xq`` for self-attention), plus the block residual when given.  The
    projections and the fc_o + Mish epilogue run fused (qkv_projection, mab_epilogue)."""
    q, k, v = qkv_projection(mab.fc_q, mab.fc_k, mab.fc_v, xq, xk)
    h, d = mab.num_heads, q.shape[-1]
    out = varlen_attention(_heads(q, h), _heads(k, h), _heads(v, h), cu_q, cu_k, max_q, max_k,
                           dropout_p=attn_dropout(mab), **mask_kwargs)
    return mab_epilogue(out.reshape(-1, d).to(q.dtype), mab.fc_o, residual)


def _gemm_input_norm(ln: nn.LayerNorm, x: torch.Tensor) -> torch.Tensor:
    """ln(x) for a consumer that is a Linear: under autocast only the autocast-dtype rows are written (what
    the Linear would cast ln's fp32 output to)."""
    y, y_mm = layer_norm(x, ln, full=False, lowp=True)
    return y if y_mm is None else y_mm


def _sab_forward_packed(blk: "SABComplete", X: torch.Tensor, tokens: PackedSets) -> torch.Tensor:
    """SABComplete.forward (pre-norm, esa/masked_layers.py:418-483) on packed tokens X [T, D]: the masked
    layers (idx 1) apply the descriptor's mask, the unmasked ones (idx 0) attend over each graph's tokens."""
    X, x_mm = layer_norm(X, blk.norm.ln, full=True, lowp=True)
    x_mm = X if x_mm is None else x_mm
    mask_kwargs = tokens.kernel_mask(padded=False) if blk.idx == 1 else {}
    cu, n = tokens.cu_seqlens, tokens.max_items
    if blk.sab.mab.dim_V == X.shape[-1]:   # the residual add fused into the epilogue
        out = _packed_mab(blk.sab.mab, x_mm, x_mm, cu, cu, n, n, mask_kwargs, residual=X)
    else:
        out = blk.proj_1(X) + _packed_mab(blk.sab.mab, x_mm, x_mm, cu, cu, n, n, mask_kwargs)
    if blk.use_mlp:
        # out feeds the MLP's LayerNorm and the residual: the pass-through output hands the residual's
        # gradient to the LayerNorm backward, which adds it to its input gradient in the same pass
        y, y_mm, out_res = layer_norm(out, blk.norm_mlp.ln, full=False, lowp=True, passthrough=True)
        out_mlp = blk.mlp(y if y_mm is None else y_mm)
        if out.shape[-1] == out_mlp.shape[-1]:
            out = out_mlp + out_res
    if blk.residual_dropout > 0:
        out = F.dropout(out, p=blk.residual_dropout)
    return out


def _pma_forward_packed(blk: "PMAComplete", X: torch.Tensor, tokens: PackedSets) -> torch.Tensor:
    """PMAComplete.forward (esa/masked_layers.py:583-610) with packed keys X [T, D] -> [B, k, D]: the seeds
    of each graph attend over its tokens."""
    X, x_mm = layer_norm(X, blk.norm.ln, full=True, lowp=True)
    x_mm = X if x_mm is None else x_mm
    b, (k_seeds, d) = tokens.batch_size, blk.pma.S.shape[1:]
    mab = blk.pma.mab
    # MAB(S.repeat(B, 1, 1), X): the seeds are projected once and shared by every set (esa_pma_*)
    q, k, v = qkv_projection(mab.fc_q, mab.fc_k, mab.fc_v, blk.pma.S.reshape(k_seeds, d), x_mm)
    h = mab.num_heads
    o = pma_attention(_heads(q, h), _heads(k, h), _heads(v, h), tokens.cu_seqlens, tokens.max_items,
                      dropout_p=attn_dropout(mab))
    out = mab_epilogue(o.reshape(-1, d).to(q.dtype), mab.fc_o).reshape(b, k_seeds, d)
    if k_seeds == tokens.max_items:   # the reference's residual when the seed count equals N
        out = tokens.pad(X) + out
    if blk.use_mlp:
        out_mlp = blk.mlp(_gemm_input_norm(blk.norm_mlp.ln, out))
        if out.shape[-2] == out_mlp.shape[-2]:
            out = out_mlp + out
    if blk.residual_dropout > 0:
        out = F.dropout(out, p=blk.residual_dropout)
    return out


class PMAComplete(nn.Module):
    """Pre-norm PMA block (esa/masked_layers.py:497-621)."""

    def __init__(self, dim_hidden, num_heads, num_outputs, norm_type, dropout=0, use_mlp=False,
                 mlp_hidden_size=64, mlp_type="standard", xformers_or_torch_attn="xformers", set_max_items=0,
                 use_bfloat16=True, num_mlp_layers=3, pre_or_post="pre", num_layers_for_residual=0,
                 residual_dropout=0, use_mlp_ln=False, mlp_dropout=0):
        super().__init__()
        _backend_check(xformers_or_torch_attn)
        if pre_or_post != "pre":
            raise NotImplementedError("post-norm blocks are not on the benchmarked path (every config is pre-norm)")
        if norm_type != "LN":
            raise NotImplementedError("BatchRenorm blocks are not on the HIP path; use norm_type='LN'")
        self.use_mlp, self.mlp_hidden_size, self.num_heads = use_mlp, mlp_hidden_size, num_heads
        self.xformers_or_torch_attn = xformers_or_torch_attn
        self.set_max_items, self.use_bfloat16 = set_max_items, use_bfloat16
        self.residual_dropout, self.num_mlp_layers, self.pre_or_post = residual_dropout, num_mlp_layers, pre_or_post
        if xformers_or_torch_attn == "flash_varlen":
            self.pma = PMAFlashVarlen(dim_hidden, num_heads, num_outputs, dropout)
        else:
            self.pma = PMA(dim_hidden, num_heads, num_outputs, dropout, xformers_or_torch_attn)
        self.norm = LN(dim_hidden)
        self.mlp_type = mlp_type
        if use_mlp:
            cls = SmallMLP if mlp_type == "standard" else GatedMLPMulti
            self.mlp = cls(in_dim=dim_hidden, out_dim=dim_hidden, inter_dim=mlp_hidden_size, dropout_p=mlp_dropout,
                           num_layers=num_mlp_layers, use_ln=use_mlp_ln)
        self.norm_mlp = LN(dim_hidden)

    def forward(self, inp):
        X, edge_index, batch_mapping, max_items, adj_mask = inp[:5]
        X = self.norm(X)
        if isinstance(self.pma, PMAFlashVarlen):
            seq_lens = torch.bincount(batch_mapping, minlength=X.size(0)).to(torch.int32)
            out_attn = self.pma(X, seq_lens=seq_lens)
        elif self.xformers_or_torch_attn == "hip" and isinstance(adj_mask, PackedSets):
            out_attn = pooled_attention(self.pma.mab, self.pma.S.repeat(X.size(0), 1, 1), X, adj_mask)
        else:
            out_attn = self.pma(X)
        if out_attn.shape[-2] == X.shape[-2]:
            out = X + out_attn
        else:
            out = out_attn
        if self.use_mlp:
            out_mlp = self.mlp(self.norm_mlp(out))
            if out.shape[-2] == out_mlp.shape[-2]:
                out = out_mlp + out
        if self.residual_dropout > 0:
            out = F.dropout(out, p=self.residual_dropout)
        return out, edge_index, batch_mapping, max_items, adj_mask


class ESA(nn.Module):
    """Edge-set attention encoder + PMA decoder (esa/masked_layers.py:624-936)."""

    def __init__(self, num_outputs, dim_output, dim_hidden, num_heads, layer_types, node_or_edge="edge",
                 xformers_or_torch_attn="xformers", pre_or_post="pre", norm_type="LN", sab_dropout=0.0,
                 mab_dropout=0.0, pma_dropout=0.0, residual_dropout=0.0, pma_residual_dropout=0.0, use_mlps=False,
                 mlp_hidden_size=64, num_mlp_layers=2, mlp_type="gated_mlp", mlp_dropout=0.0, use_mlp_ln=False,
                 set_max_items=0, use_bfloat16=True, use_equivariant=False, equivariant_lmax=2,
                 equivariant_num_features=16, equivariant_fusion_method="add", equivariant_cross_connection=True):
        super().__init__()
        assert len(layer_types) == len(dim_hidden) and len(layer_types) == len(num_heads)
        _backend_check(xformers_or_torch_attn)
        if node_or_edge not in ("node", "edge"):
            raise ValueError(f"node_or_edge must be 'node' or 'edge' (got {node_or_edge!r})")
        self.dim_hidden, self.num_heads, self.layer_types = dim_hidden, num_heads, layer_types
        self.node_or_edge = node_or_edge
        self.xformers_or_torch_attn = xformers_or_torch_attn
        self.pre_or_post, self.norm_type = pre_or_post, norm_type
        self.use_bfloat16 = use_bfloat16
        self.use_distance_bias = False
        common = dict(pre_or_post=pre_or_post, use_mlp=use_mlps, mlp_hidden_size=mlp_hidden_size,
                      mlp_dropout=mlp_dropout, num_mlp_layers=num_mlp_layers, use_mlp_ln=use_mlp_ln,
                      norm_type=norm_type, mlp_type=mlp_type, set_max_items=set_max_items,
                      use_bfloat16=use_bfloat16, num_layers_for_residual=len(dim_hidden) * 2)
        has_pma = "P" in layer_types
        encoder, decoder = [], None
        pma_encountered, dim_pma, tracker = False, -1, 0
        for lt in layer_types:
            d_in, heads = dim_hidden[tracker], num_heads[tracker]
            d_out = (dim_hidden[tracker + 1] if has_pma else dim_hidden[tracker]) if lt != "P" else -1
            if lt == "S" and not pma_encountered:
                encoder.append(SABComplete(d_in, d_out, heads, idx=0, dropout=sab_dropout, node_or_edge=node_or_edge,
                                           xformers_or_torch_attn=xformers_or_torch_attn,
                                           residual_dropout=residual_dropout, **common))
            if lt == "M" and not pma_encountered:
                encoder.append(SABComplete(d_in, d_out, heads, idx=1, dropout=mab_dropout, node_or_edge=node_or_edge,
                                           xformers_or_torch_attn=xformers_or_torch_attn,
                                           residual_dropout=residual_dropout, **common))
            if lt == "P":
                pma_encountered = True
                dim_pma = d_in
                pcommon = {k: v for k, v in common.items() if k not in ("num_layers_for_residual",)}
                # a later "P" replaces the decoder (esa/masked_layers.py:778)
                decoder = [PMAComplete(d_in, heads, num_outputs, dropout=pma_dropout,
                                       residual_dropout=pma_residual_dropout,
                                       xformers_or_torch_attn=xformers_or_torch_attn,
                                       num_layers_for_residual=len(dim_hidden) * 2, **pcommon)]
            if lt == "S" and pma_encountered:
                decoder.append(SABComplete(d_in, d_out, heads, idx=2, dropout=sab_dropout, node_or_edge=node_or_edge,
                                           xformers_or_torch_attn=xformers_or_torch_attn,
                                           residual_dropout=residual_dropout, **common))
            if lt != "P":
                tracker += 1
        self.encoder = nn.Sequential(*encoder)
        if pma_encountered:
            self.decoder = nn.Sequential(*decoder)
        self.decoder_linear = nn.Linear(dim_hidden[-1], dim_output, bias=True)
        if has_pma and dim_hidden[0] != dim_pma:
            self.out_proj = nn.Linear(dim_hidden[0], dim_pma)
            self.dim_pma = dim_pma

    def forward(self, X, edge_index, batch_mapping, num_max_items, pos=None):
        build = get_adj_mask_from_edge_index_node if self.node_or_edge == "node" else get_adj_mask_from_edge_index_edge
        adj_mask = build(edge_index=edge_index, batch_mapping=batch_mapping, batch_size=X.shape[0],
                         max_items=num_max_items)
        if self.xformers_or_torch_attn == "hip" and isinstance(adj_mask, PackedSets):
            return self._forward_packed(X, edge_index, batch_mapping, num_max_items, adj_mask)
        enc, _, _, _, _ = self.encoder((X, edge_index, batch_mapping, num_max_items, adj_mask))
        if hasattr(self, "dim_pma") and self.dim_hidden[0] != self.dim_pma:
            X = self.out_proj(X)
        enc = enc + X
        node_embeddings_before_pma = enc
        if hasattr(self, "decoder"):
            out, _, _, _, _ = self.decoder((enc, edge_index, batch_mapping, num_max_items, adj_mask))
            out = out.mean(dim=1)
            return mish(self.decoder_linear(out)), node_embeddings_before_pma
        return mish(self.decoder_linear(enc)), enc

    def _forward_packed(self, X, edge_index, batch_mapping, num_max_items, tokens: PackedSets):
        """The "hip" forward of padded input: unpad, encode the packed tokens, pad the token embeddings.

        Without a PMA the head acts per token, and the result keeps the padded forward's [B, N, dim_output]
        shape (esa/masked_layers.py:929-936): the head runs on the padded embeddings, which are zero at the
        padding slots, so those slots hold mish(bias)."""
        with self._linear_casts():
            enc = self._encode_packed(tokens.unpad(X), tokens)
            enc_pad = tokens.pad(enc)
            if hasattr(self, "decoder"):
                return self._decode_packed(enc, tokens, edge_index, batch_mapping), enc_pad
            return mish(self.decoder_linear(enc_pad)), enc_pad

    def _linear_casts(self):
        """Under autocast, the blocks' Linear parameters cast once per forward in one concatenated cast
        (``linear.param_casts``) instead of one cast per parameter and call."""
        if not torch.is_autocast_enabled("cuda"):
            return contextlib.nullcontext()
        params = [t for m in self.modules() if isinstance(m, nn.Linear) for t in (m.weight, m.bias)]
        return param_casts(params, torch.get_autocast_dtype("cuda"))

    def _encode_packed(self, tokens_x: torch.Tensor, tokens: PackedSets) -> torch.Tensor:
        """Encoder blocks and the input residual on packed tokens [T, D] (esa/masked_layers.py:914-921)."""
        xp = tokens_x
        h = xp
        for blk in self.encoder:
            h = _sab_forward_packed(blk, h, tokens)
        if hasattr(self, "dim_pma") and self.dim_hidden[0] != self.dim_pma:
            xp = self.out_proj(xp)
        return h + xp

    def _decode_packed(self, enc: torch.Tensor, tokens: PackedSets, edge_index, batch_mapping) -> torch.Tensor:
        """PMA decoder, mean over seeds and the Mish head (esa/masked_layers.py:926-934) -> [B, dim_output]."""
        out = _pma_forward_packed(self.decoder[0], enc, tokens)
        for blk in list(self.decoder)[1:]:
            out, _, _, _, _ = blk((out, edge_index, batch_mapping, tokens.max_items, tokens))
        out = out.mean(dim=1)
        return mish(self.decoder_linear(out))

    def forward_packed(self, tokens_x: torch.Tensor, tokens: PackedSets, edge_index=None, batch_mapping=None):
        """ESA.forward (esa/masked_layers.py:849-936) on packed tokens, the "hip" backend's native entry.

        tokens_x [T, D] holds the set elements graph after graph (edge tokens straight from the edge MLP, in
        edge_index order; or node tokens), ``tokens`` their descriptor (``get_adj_mask_from_edge_index_edge``
        / ``_node`` or ``EdgeAdjacency`` / ``NodeAdjacency.from_edge_index``).  No padded [B, N, D] tensor is
        built: the reference's to_dense_batch (core/pretraining_model.py:211, esa/models.py:317) and the
        encoder's work on padding slots go away.  Returns (graph embeddings [B, dim_output], token
        embeddings before pooling [T, D]); ``enc`` equals the padded forward's at the valid slots.
        """
        if self.xformers_or_torch_attn != "hip":
            raise ValueError("forward_packed is the native 'hip' backend's entry; this ESA was built for "
                             f"{self.xformers_or_torch_attn!r}")
        if tokens_x.dim() != 2 or tokens_x.shape[0] != tokens.num_tokens:
            raise ValueError(f"tokens_x must be [T, D] with T = {tokens.num_tokens} (got {tuple(tokens_x.shape)})")
        with self._linear_casts():
            enc = self._encode_packed(tokens_x, tokens)
            if hasattr(self, "decoder"):
                return self._decode_packed(enc, tokens, edge_index, batch_mapping), enc
            # no PMA: the head acts on every token; packed, it returns [T, dim_output] (the padded entry pads)
            return mish(self.decoder_linear(enc)), enc
