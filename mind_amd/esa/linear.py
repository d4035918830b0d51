"""nn.Linear for the packed ESA blocks, with a split-K weight gradient.

On packed edge tokens a Linear's weight gradient dW = g^T x reduces over all
T tokens of the batch (T = 131,072 in the encoder-stack benchmark) into a
small [out, in] matrix: one GEMM with K = T has only a few dozen output tiles
for 256 CUs.  ``linear`` computes it instead as S batched GEMMs over token
chunks (``torch.bmm`` with fp32 outputs) and sums the S fp32 partials, so the
reduction fills the chip and is rounded to the weight's dtype once, as the
single GEMM's fp32 accumulator is.  Forward (F.linear) and dx = g W are
unchanged; the bias gradient is a deterministic column sum (esa_column_sum).
Under autocast the inputs are cast as autocast casts F.linear's (x, weight
and bias to the autocast dtype); the autograd functions take the parameters
in their own dtype and cast them inside, so the fp32 weight and bias
gradients are returned as they are computed, in fp32, instead of being
rounded to the autocast dtype and cast back by a second kernel.

Reference: the nn.Linear layers of the MAB (esa/mha.py:12-15) and of the MLPs
(esa/mlp_utils.py:18-37).
"""
from __future__ import annotations

import contextlib
import contextvars
import ctypes

import torch
from torch import nn
from torch.nn import functional as F

from .. import _lib

_MIN_CHUNK = 4096               # tokens per chunk: below, a chunk's GEMM is too short to pay
_MAX_PARTIAL = 16 * 1024 * 1024  # fp32 values of all partials (64 MiB)
_MAX_SPLIT = 32


def split_count(tokens: int, out_features: int, in_features: int) -> int:
    """Chunks S of the split-K weight gradient (1 = a single GEMM): the largest power of two <= 32 with chunks
    of >= 4096 tokens and S * out * in fp32 partials within 64 MiB."""
    s = 1
    while (2 * s <= _MAX_SPLIT and tokens // (2 * s) >= _MIN_CHUNK
           and 2 * s * out_features * in_features <= _MAX_PARTIAL):
        s *= 2
    return s


def weight_grad(g: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """g^T x for g [T, out], x [T, in] (same dtype) in fp32, by split_count(T, out, in) token chunks."""
    t, o = g.shape
    i = x.shape[1]
    s = split_count(t, o, i)
    # bf16 device operands: products accumulated and returned in fp32 by the GEMM itself (out_dtype), no casts
    kw = {} if g.dtype == torch.float32 or not g.is_cuda else {"out_dtype": torch.float32}
    if t < _MIN_CHUNK:
        return torch.mm(g.t(), x, **kw) if kw else g.t().float().mm(x.float())
    c = t // s
    t0 = s * c
    parts = torch.bmm(g[:t0].view(s, c, o).transpose(1, 2), x[:t0].view(s, c, i), **kw)
    dw = parts.sum(0)
    if t0 < t:   # fewer than S leftover tokens: added by the GEMM's epilogue
        dw = torch.addmm(dw, g[t0:].t(), x[t0:], **kw)
    return dw


_CODES = {torch.float32: _lib.ESA_F32, torch.bfloat16: _lib.ESA_BF16}


def column_sum(g: torch.Tensor) -> torch.Tensor:
    """g.sum(0) of a device [rows, cols] tensor in fp32 through esa_column_sum (fixed order); shapes the kernel
    does not take (cols not a multiple of 4, other dtypes) use torch's sum."""
    rows, cols = g.shape
    if g.dtype not in _CODES or cols % 4 or cols < 4:
        return g.float().sum(0)
    g = g.contiguous()
    lib = _lib.load()
    n = ctypes.c_size_t(0)
    _lib.check(lib.esa_column_sum_workspace_size(rows, cols, ctypes.byref(n)), "esa_column_sum_workspace_size")
    ws = torch.empty(int(n.value), dtype=torch.uint8, device=g.device)
    out = torch.empty(cols, dtype=torch.float32, device=g.device)
    _lib.check(lib.esa_column_sum(g.data_ptr(), _CODES[g.dtype], rows, cols, out.data_ptr(), ws.data_ptr(),
                                  ws.numel(), _lib.stream_of(g)), "esa_column_sum")
    return out


_MAX_LINEAR_OUT = 3


def _aligned(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0


def _f32_linear_ok(x: torch.Tensor, pairs) -> bool:
    """Whether esa_linear_f32 takes F.linear(x, w, b) for every (w, b): fp32 device tensors, x [rows, K] and
    W [N, K] contiguous, K % 16 == 0, N % 64 == 0, 16-byte aligned rows."""
    if not (x.is_cuda and x.dtype == torch.float32 and x.dim() == 2 and x.is_contiguous() and _aligned(x)):
        return False
    k = x.shape[1]
    if k < 16 or k % 16 or x.shape[0] >= 2 ** 31:
        return False
    for w, b in pairs:
        if not (w.dtype == torch.float32 and w.dim() == 2 and w.shape[1] == k and w.shape[0] % 64 == 0
                and w.is_contiguous() and _aligned(w) and w.device == x.device):
            return False
        if b is not None and not (b.dtype == torch.float32 and b.shape == (w.shape[0],) and b.is_contiguous()
                                  and b.device == x.device):
            return False
    return True


def esa_linear(x: torch.Tensor, pairs) -> list[torch.Tensor]:
    """[F.linear(x, w, b) for (w, b) in pairs] through one launch of esa_linear_f32 (1-3 weights over one fp32
    input of the shapes ``_f32_linear_ok`` accepts; raises otherwise)."""
    pairs = list(pairs)
    if not 1 <= len(pairs) <= _MAX_LINEAR_OUT or not _f32_linear_ok(x, pairs):
        raise ValueError("esa_linear takes 1-3 fp32 weights [N % 64 == 0, K] over a contiguous fp32 x [rows, K], "
                         "K % 16 == 0")
    n = len(pairs)
    ys = [torch.empty(x.shape[0], w.shape[0], dtype=torch.float32, device=x.device) for w, _ in pairs]
    vp = ctypes.c_void_p
    w_arr = (vp * n)(*[w.data_ptr() for w, _ in pairs])
    b_arr = (vp * n)(*[None if b is None else b.data_ptr() for _, b in pairs])
    y_arr = (vp * n)(*[y.data_ptr() for y in ys])
    n_arr = (ctypes.c_int * n)(*[w.shape[0] for w, _ in pairs])
    _lib.check(_lib.load().esa_linear_f32(x.data_ptr(), x.shape[0], x.shape[1], n, w_arr, b_arr, y_arr, n_arr,
                                          _lib.stream_of(x)), "esa_linear_f32")
    return ys


def linear_fwd(x: torch.Tensor, pairs) -> list[torch.Tensor]:
    """[F.linear(x, w, b) for (w, b) in pairs] over 2-D x.  Two or three fp32 weights sharing the input (the
    MAB's Q / K / V projections) of the shapes esa_linear_f32 takes run as one launch of it; a single weight,
    and everything else, is F.linear (at one weight the library GEMM is as fast or faster)."""
    pairs = list(pairs)
    if 2 <= len(pairs) <= _MAX_LINEAR_OUT and _f32_linear_ok(x, pairs):
        return esa_linear(x, pairs)
    return [F.linear(x, w, b) for w, b in pairs]


def compute_dtype(x: torch.Tensor, *params: torch.Tensor | None):
    """The dtype a Linear over x computes in: the autocast dtype under autocast (x and the parameters are
    cast to it, as autocast casts F.linear's inputs), else x's dtype when every parameter has it; None for
    mixed dtypes outside autocast (the callers then leave the call to torch's own checks and errors)."""
    if x.is_cuda and torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return x.dtype if all(p is None or p.dtype == x.dtype for p in params) else None


_CAST_CACHE: contextvars.ContextVar = contextvars.ContextVar("esa_param_cast_cache", default=None)
_CAST_ALIGN = 128   # elements per cache slot boundary: every cached view starts 256-byte aligned in bf16


def cast_param(p: torch.Tensor | None, dt: torch.dtype):
    """p in dtype dt: the view cached by an enclosing ``param_casts`` when there is one, else p.to(dt)."""
    if p is None or p.dtype == dt:
        return p
    cache = _CAST_CACHE.get()
    if cache is not None:
        hit = cache.get(id(p))
        if hit is not None and hit[0] is p and hit[1].dtype == dt:
            return hit[1]
    return p.to(dt)


@contextlib.contextmanager
def param_casts(params, dt: torch.dtype):
    """Within the block, the Linear functions take the given fp32 device parameters cast to ``dt`` from one
    concatenated cast (a forward under autocast casts every Linear's weight and bias, about a hundred launches of
    a few microseconds for configuration 4's stack; here two or three).  The cached values equal p.to(dt) bit
    for bit; each parameter's slot starts 256-byte aligned."""
    ps, seen = [], set()
    for p in params:
        if p is not None and p.is_cuda and p.dtype == torch.float32 and p.dtype != dt and id(p) not in seen:
            seen.add(id(p))
            ps.append(p)
    if not ps:
        yield
        return
    pad = torch.zeros(_CAST_ALIGN, dtype=torch.float32, device=ps[0].device)
    pieces, offsets, off = [], [], 0
    for p in ps:
        pieces.append(p.detach().reshape(-1))
        offsets.append(off)
        off += p.numel()
        r = -off % _CAST_ALIGN
        if r:
            pieces.append(pad[:r])
            off += r
    flat = torch.cat(pieces).to(dt)
    cache = {id(p): (p, flat[o:o + p.numel()].view(p.shape)) for p, o in zip(ps, offsets)}
    token = _CAST_CACHE.set(cache)
    try:
        yield
    finally:
        _CAST_CACHE.reset(token)


class _Linear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias):
        w, b = cast_param(weight, x.dtype), cast_param(bias, x.dtype)
        ctx.save_for_backward(x, w)
        ctx.dtypes = (weight.dtype, None if bias is None else bias.dtype)
        return linear_fwd(x, [(w, b)])[0]

    @staticmethod
    def backward(ctx, g):
        x, w = ctx.saved_tensors
        wdt, bdt = ctx.dtypes
        g = g.contiguous()
        dx = g.mm(w) if ctx.needs_input_grad[0] else None
        dw = weight_grad(g, x).to(wdt) if ctx.needs_input_grad[1] else None
        db = column_sum(g).to(bdt) if bdt is not None and ctx.needs_input_grad[2] else None
        return dx, dw, db


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """F.linear(x, weight, bias) with the split-K weight gradient (device tensors; CPU tensors use F.linear)."""
    dt = compute_dtype(x, weight, bias) if x.is_cuda else None
    if dt is None:
        return F.linear(x, weight, bias)   # CPU, or mixed dtypes: torch's own type checks and errors
    x = x.to(dt)
    lead = x.shape[:-1]
    y = _Linear.apply(x.reshape(-1, x.shape[-1]).contiguous(), weight, bias)
    return y.view(*lead, weight.shape[0])


class _QKV(torch.autograd.Function):
    """q = fc_q(xq), k = fc_k(xk), v = fc_v(xk) (the MAB's V = fc_v(K), esa/mha.py:54-56).  The backward
    accumulates the input gradients of the projections that share an input in the GEMMs themselves
    (addmm with beta = 1) instead of separate add kernels, so self-attention's dx = gq Wq + gk Wk + gv Wv is
    three GEMMs and no add."""

    @staticmethod
    def forward(ctx, xq, xk, wq, bq, wk, bk, wv, bv):
        same = xk is None
        xk_ = xq if same else xk
        dt = xq.dtype
        # the parameters' own dtypes: the backward returns its fp32 gradients in them
        ctx.params = tuple(None if p is None else p.dtype for p in (wq, bq, wk, bk, wv, bv))
        wq, bq, wk, bk, wv, bv = (cast_param(p, dt) for p in (wq, bq, wk, bk, wv, bv))
        if same:
            q, k, v = linear_fwd(xq, [(wq, bq), (wk, bk), (wv, bv)])
        else:
            (q,) = linear_fwd(xq, [(wq, bq)])
            k, v = linear_fwd(xk_, [(wk, bk), (wv, bv)])
        ctx.save_for_backward(xq, None if same else xk, wq, wk, wv)
        ctx.same = same
        return q, k, v

    @staticmethod
    def backward(ctx, gq, gk, gv):
        xq, xk, wq, wk, wv = ctx.saved_tensors
        xk = xq if ctx.same else xk
        gq, gk, gv = gq.contiguous(), gk.contiguous(), gv.contiguous()
        dxq = dxk = None
        if ctx.same:
            if ctx.needs_input_grad[0]:
                dxq = gq.mm(wq)
                dxq.addmm_(gk, wk)
                dxq.addmm_(gv, wv)
        else:
            if ctx.needs_input_grad[0]:
                dxq = gq.mm(wq)
            if ctx.needs_input_grad[1]:
                dxk = gk.mm(wk)
                dxk.addmm_(gv, wv)
        grads = [dxq, dxk]
        for i, (g, x) in enumerate(((gq, xq), (gk, xk), (gv, xk))):
            wdt, bdt = ctx.params[2 * i], ctx.params[2 * i + 1]
            dw = weight_grad(g, x).to(wdt) if ctx.needs_input_grad[2 + 2 * i] else None
            db = column_sum(g).to(bdt) if bdt is not None and ctx.needs_input_grad[3 + 2 * i] else None
            grads += [dw, db]
        return tuple(grads)


def qkv_projection(fc_q: nn.Linear, fc_k: nn.Linear, fc_v: nn.Linear, xq: torch.Tensor, xk: torch.Tensor):
    """(fc_q(xq), fc_k(xk), fc_v(xk)) on 2-D token rows, with the fused-accumulation backward of _QKV on
    device tensors (``xk is xq`` for self-attention)."""
    params = (fc_q.weight, fc_q.bias, fc_k.weight, fc_k.bias, fc_v.weight, fc_v.bias)
    same = xk is xq
    dt = compute_dtype(xq, xk, *params) if xq.is_cuda else None
    if dt is None:
        return fc_q(xq), fc_k(xk), fc_v(xk)
    xq = xq.to(dt)
    xk_ = None if same else xk.to(dt).contiguous()
    return _QKV.apply(xq.contiguous(), xk_, *params)


def hookless(layer: nn.Module) -> bool:
    """True when calling ``layer`` would run no forward hooks or pre-hooks, so its forward may be replaced
    by an equivalent fused call."""
    return not (layer._forward_hooks or layer._forward_pre_hooks)


def apply(layer: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """layer(x), with hook-free nn.Linear layers through ``linear``."""
    if type(layer) is nn.Linear and hookless(layer):
        return linear(x, layer.weight, layer.bias)
    return layer(x)
