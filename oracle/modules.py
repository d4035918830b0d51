"""Reference block arithmetic on CPU (test infrastructure; see oracle/__init__.py).

Functions take a module's state_dict (``prefix`` selects the submodule) and
restate the forward of the reference block in float64:
  mab_padded      esa/mha.py:48-89 with an optional additive [B, 1, N, N] bias
  mab_varlen      esa/mha_flash_varlen.py:129-201 (V = fc_v(fc_k(K)), valid tokens)
  mab_packed      the same block over packed valid tokens with an optional
                  boolean per-graph mask (the native "hip" path's arithmetic)
  mlp_standard    SmallMLP (esa/mlp_utils.py:6-48) without LayerNorm/dropout
  sab_complete    esa/masked_layers.py:408-494 (pre-norm branch)
  pma_complete    esa/masked_layers.py:574-621 (pre-norm branch), padded or packed keys
  esa             ESA.forward (esa/masked_layers.py:849-936): encoder, enc + X,
                  PMA decoder (+ later S layers on the seeds), mean over seeds,
                  mish(decoder_linear)
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from .attention import padded_attention, varlen_attention, varlen_attention_diff
from .packing import to_dense_batch

DT = torch.float64   # the checker's precision (the CPU baseline of bench.py times it in float32)


def _p(sd, prefix, name):
    return sd[prefix + name].cpu().to(DT)


def linear(sd, prefix, x):
    return x @ _p(sd, prefix, "weight").T + _p(sd, prefix, "bias")


def layer_norm(sd, prefix, x, eps=1e-8):
    """nn.LayerNorm(eps=1e-8) (esa/utils/norm_layers.py:36)."""
    mu = x.mean(-1, keepdim=True)
    var = ((x - mu) ** 2).mean(-1, keepdim=True)
    return (x - mu) / torch.sqrt(var + eps) * _p(sd, prefix, "weight") + _p(sd, prefix, "bias")


def mish(x):
    return x * torch.tanh(F.softplus(x))


def mish_grad(x):
    """d mish / dx = tanh(softplus x) + x sigmoid(x) (1 - tanh(softplus x)^2): the derivative of the F.mish /
    nn.Mish of esa/mha.py:87 and esa/mlp_utils.py:24-37."""
    t = torch.tanh(F.softplus(x))
    return t + x * torch.sigmoid(x) * (1 - t * t)


def _heads(x, h):
    return x.reshape(*x.shape[:-1], h, x.shape[-1] // h)


def mab_padded(sd, prefix, Q, K, heads, bias=None):
    """MAB over padded [B, N, D]: V = fc_v(K); softmax(QK^T/sqrt(hd) + bias) V; out + mish(fc_o(out))."""
    Q, K = Q.cpu().to(DT), K.cpu().to(DT)
    q = linear(sd, prefix + "fc_q.", Q)
    v = linear(sd, prefix + "fc_v.", K)
    k = linear(sd, prefix + "fc_k.", K)
    hd = q.shape[-1] // heads
    o = padded_attention(_heads(q, heads), _heads(k, heads), _heads(v, heads), 1.0 / np.sqrt(hd), bias, dtype=DT)
    o = o.reshape(Q.shape[0], Q.shape[1], -1)
    return o + mish(linear(sd, prefix + "fc_o.", o))


def mab_packed(sd, prefix, Qp, Kp, cu_q, cu_k, heads, edge_src=None, edge_dst=None, v_from_k=False, adj=None,
               dropout=None):
    """MAB over packed tokens [T, D] per segment; optional edge mask or node CSR ``adj``; V = fc_v(K) or
    fc_v(fc_k(K)); ``dropout`` as oracle.attention's (esa/mha.py:76,82 in training)."""
    Qp, Kp = torch.as_tensor(Qp).cpu().to(DT), torch.as_tensor(Kp).cpu().to(DT)
    q = linear(sd, prefix + "fc_q.", Qp)
    k = linear(sd, prefix + "fc_k.", Kp)
    v = linear(sd, prefix + "fc_v.", k if v_from_k else Kp)
    hd = q.shape[-1] // heads
    o = varlen_attention_diff(_heads(q, heads).contiguous(), _heads(k, heads).contiguous(),
                              _heads(v, heads).contiguous(), cu_q, cu_k, 1.0 / np.sqrt(hd), edge_src, edge_dst, adj,
                              dropout)
    o = o.reshape(Qp.shape[0], -1)
    return o + mish(linear(sd, prefix + "fc_o.", o))


def mab_varlen(sd, prefix, Q, K, seq_lens, heads):
    """MABFlashVarlen._forward_varlen on padded [B, N, D] with seq_lens: valid tokens, zeros at padding."""
    Q, K = Q.cpu().to(DT), K.cpu().to(DT)
    b, n, d = Q.shape
    lens = np.asarray(seq_lens, dtype=np.int64)
    valid = np.arange(n)[None, :] < lens[:, None]
    idx = torch.as_tensor(np.nonzero(valid.reshape(-1))[0])
    cu = np.concatenate([[0], np.cumsum(valid.sum(1))])
    q = linear(sd, prefix + "fc_q.", Q).reshape(b * n, d)[idx]
    k = linear(sd, prefix + "fc_k.", K).reshape(b * n, d)[idx]
    v = linear(sd, prefix + "fc_v.", k)
    o, _ = varlen_attention(_heads(q, heads), _heads(k, heads), _heads(v, heads), cu, cu, 1.0 / np.sqrt(d // heads),
                            dtype=DT)
    out = torch.zeros(b * n, d, dtype=DT)
    out[idx] = o.reshape(-1, d)
    out = out.reshape(b, n, d)
    return out + mish(linear(sd, prefix + "fc_o.", out))


def mlp_standard(sd, prefix, x, num_layers):
    """SmallMLP without LayerNorm/dropout (esa/mlp_utils.py:6-48): Linear+Mish ... Linear."""
    if num_layers == 1:
        return mish(linear(sd, prefix + "mlp.0.", x))
    i = 0
    for layer in range(num_layers):
        x = linear(sd, prefix + f"mlp.{i}.", x)
        i += 1
        if layer != num_layers - 1:
            x = mish(x)
            i += 1
    return x


def sab_complete(sd, prefix, X, heads, attn, num_mlp_layers=None):
    """Pre-norm block: X' = LN(X); out = X' + attn(X'); out += MLP(LN2(out)) (esa/masked_layers.py:418-483).

    ``attn(sd, prefix_of_mab, X')`` computes the attention sub-block.
    """
    X = X.cpu().to(DT)
    xn = layer_norm(sd, prefix + "norm.ln.", X)
    out = xn + attn(sd, prefix + "sab.mab.", xn)
    if num_mlp_layers:
        out = out + mlp_standard(sd, prefix + "mlp.", layer_norm(sd, prefix + "norm_mlp.ln.", out), num_mlp_layers)
    return out


def pma_complete(sd, prefix, X, heads, num_mlp_layers=None, cu=None, max_items=None, dropout=None):
    """Pre-norm PMA block (esa/masked_layers.py:574-621) -> [B, k, D].

    X' = LN(X) (:583); A = MAB(S.repeat(B, 1, 1), X') (esa/mha.py:108-109,
    V = fc_v(K)); the residual X' + A only when the seed count k equals the
    set size N (:595-603), else out = A; then out += MLP(LN2(out)) (:606-610).
    X is padded [B, N, D] (``cu`` None: the seeds attend over all N positions,
    padding included, as the reference does), or packed [T, D] with ``cu`` the
    set offsets (the seeds attend over each set's valid tokens) and
    ``max_items`` the padded N of the k == N test (padding slots then hold 0).
    """
    X = torch.as_tensor(X).cpu().to(DT)
    xn = layer_norm(sd, prefix + "norm.ln.", X)
    S = _p(sd, prefix + "pma.", "S")                       # [1, k, D]
    k, d = S.shape[1], S.shape[2]
    if cu is None:
        b, n = X.shape[0], X.shape[1]
        out = mab_padded(sd, prefix + "pma.mab.", S.repeat(b, 1, 1), xn, heads)
        res = xn
    else:
        cu = np.asarray(cu, dtype=np.int64)
        b, n = len(cu) - 1, int(max_items)
        seeds = S.reshape(k, d).repeat(b, 1)
        out = mab_packed(sd, prefix + "pma.mab.", seeds, xn, np.arange(b + 1) * k, cu, heads,
                         dropout=dropout).reshape(b, k, d)
        graph = np.repeat(np.arange(b), np.diff(cu))
        res = to_dense_batch(xn, graph, b, n)[0] if k == n else None
    if k == n:
        out = res + out
    if num_mlp_layers:
        out = out + mlp_standard(sd, prefix + "mlp.", layer_norm(sd, prefix + "norm_mlp.ln.", out), num_mlp_layers)
    return out


def esa(sd, X, layer_types, heads, num_mlp_layers, attn_m, attn_s, pool):
    """ESA.forward (esa/masked_layers.py:849-936) for equal hidden sizes -> (graph_emb [B, dim_output], enc).

    Encoder (the M/S layers before the first P, :700-760) as pre-norm
    SABComplete blocks, ``attn_m`` / ``attn_s`` computing the masked /
    unmasked MAB sub-block (callables ``(sd, mab_prefix, x)``); enc =
    encoder(X) + X (:917); the decoder's PMAComplete is ``pool(sd, prefix,
    enc)`` -> [B, k, D] (a later P replaces it, :778); S layers after the P act
    on the seeds with unmasked attention over the k seeds; out.mean(1) over the
    seeds (:928); graph_emb = mish(decoder_linear(out)) (:929).
    """
    X = torch.as_tensor(X).cpu().to(DT)
    types = list(layer_types)
    p_at = types.index("P") if "P" in types else len(types)
    h = X
    for i, lt in enumerate(types[:p_at]):
        h = sab_complete(sd, f"encoder.{i}.", h, heads, attn_m if lt == "M" else attn_s, num_mlp_layers)
    enc = h + X
    if p_at == len(types):
        return mish(linear(sd, "decoder_linear.", enc)), enc
    p_last = len(types) - 1 - types[::-1].index("P")
    out = pool(sd, "decoder.0.", enc)

    def seeds_attn(sd_, pre, x):
        return mab_padded(sd_, pre, x, x, heads)

    later_s = [lt for lt in types[p_last + 1:] if lt == "S"]   # an M after the P is not built (:743)
    for j in range(len(later_s)):
        out = sab_complete(sd, f"decoder.{j + 1}.", out, heads, seeds_attn, num_mlp_layers)
    return mish(linear(sd, "decoder_linear.", out.mean(1))), enc
