"""Pre-norm LayerNorm of the ESA blocks on the gfx950 kernels (esa_layer_norm_fwd / _bwd).

``layer_norm(x, ln, full=True, lowp=False, passthrough=False)`` returns ``(y, y_lp)``: y is
``ln(x)`` as torch evaluates it here (fp32 under autocast, x's dtype
otherwise; None when ``full`` is False) and y_lp is the same rows in the
autocast dtype, written by the same pass (None without autocast or when
``lowp`` is False).  The blocks use y as the residual and y_lp as the GEMM
input, which is what autocast would cast y to (esa/masked_layers.py:418-419,
471-483 with nn.LayerNorm(D, eps=1e-8), esa/utils/norm_layers.py:36).  The
backward sums the gradients of both outputs inside the kernel.

With ``passthrough=True`` a third value is returned: x itself (a view), to be
used in x's other places, such as the residual ``out = mlp(ln(x)) + x`` of a
pre-norm block (esa/masked_layers.py:478-483).  Its gradient then reaches the
same backward call, and the kernel adds it to dx instead of autograd summing
the two gradients of x in a separate pass.

Feature counts that are not a multiple of 4 or above 2048 use
torch.nn.functional.layer_norm; CPU tensors use the module itself.
"""
from __future__ import annotations

import ctypes

import torch
from torch import nn

from .. import _lib

_CODES = {torch.float32: _lib.ESA_F32, torch.bfloat16: _lib.ESA_BF16}
MAX_FEATURES = 2048


def supported(x: torch.Tensor, ln: nn.LayerNorm) -> bool:
    d = x.shape[-1]
    return (x.is_cuda and x.dtype in _CODES and len(ln.normalized_shape) == 1 and d % 4 == 0
            and 4 <= d <= MAX_FEATURES)


class _LayerNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x_in, weight, bias, eps, y_dtype, full, lowp, passthrough):
        x = x_in.contiguous()
        d = x.shape[-1]
        rows = x.numel() // d
        w32 = None if weight is None else weight.detach().float().contiguous()
        b32 = None if bias is None else bias.detach().float().contiguous()
        y = torch.empty(x.shape, dtype=y_dtype, device=x.device) if full else None
        ylp = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device) if lowp else None
        mean = torch.empty(rows, dtype=torch.float32, device=x.device)
        rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
        rc = _lib.load().esa_layer_norm_fwd(x.data_ptr(), _CODES[x.dtype], _lib.ptr(w32), _lib.ptr(b32), rows, d,
                                            float(eps), _lib.ptr(y), _CODES[y_dtype], _lib.ptr(ylp),
                                            mean.data_ptr(), rstd.data_ptr(), _lib.stream_of(x))
        _lib.check(rc, "esa_layer_norm_fwd")
        ctx.save_for_backward(x, w32, mean, rstd)
        ctx.set_materialize_grads(False)   # an unused output's gradient stays None (no zero tensor is read)
        ctx.param_dtypes = (None if weight is None else weight.dtype, None if bias is None else bias.dtype)
        ctx.outputs = (full, lowp, passthrough)
        outs = tuple(t for t in (y, ylp) if t is not None) + ((x_in.view_as(x_in),) if passthrough else ())
        return outs if len(outs) > 1 else outs[0]

    @staticmethod
    def backward(ctx, *grads):
        x, w32, mean, rstd = ctx.saved_tensors
        full, lowp, passthrough = ctx.outputs
        grads = list(grads)
        gy = grads.pop(0) if full else None
        gl = grads.pop(0) if lowp else None
        gr = grads.pop(0) if passthrough else None
        if gy is not None:
            gy = gy.contiguous()
            if gy.dtype not in _CODES:
                gy = gy.float()
        if gl is not None:
            gl = gl.to(torch.bfloat16).contiguous()
        if gr is not None:
            gr = gr.to(x.dtype).contiguous()
        d = x.shape[-1]
        rows = x.numel() // d
        dx = torch.empty_like(x)
        wdt, bdt = ctx.param_dtypes
        need_w = wdt is not None and ctx.needs_input_grad[1]
        need_b = bdt is not None and ctx.needs_input_grad[2]
        if gy is None and gl is None:
            return (torch.zeros_like(x) if gr is None else gr), None, None, None, None, None, None, None
        dw = torch.empty(d, dtype=torch.float32, device=x.device) if need_w else None
        db = torch.empty(d, dtype=torch.float32, device=x.device) if need_b else None
        lib = _lib.load()
        n = ctypes.c_size_t(0)
        _lib.check(lib.esa_layer_norm_bwd_workspace_size(rows, d, ctypes.byref(n)), "esa_layer_norm_bwd_workspace_size")
        ws = torch.empty(max(int(n.value), 1), dtype=torch.uint8, device=x.device) if (need_w or need_b) else None
        rc = lib.esa_layer_norm_bwd(x.data_ptr(), _CODES[x.dtype], _lib.ptr(w32), mean.data_ptr(), rstd.data_ptr(),
                                    _lib.ptr(gy), _CODES[gy.dtype] if gy is not None else _lib.ESA_F32, _lib.ptr(gl),
                                    _lib.ptr(gr), rows, d, dx.data_ptr(), _lib.ptr(dw), _lib.ptr(db), _lib.ptr(ws),
                                    0 if ws is None else ws.numel(), _lib.stream_of(x))
        _lib.check(rc, "esa_layer_norm_bwd")
        return (dx, None if dw is None else dw.to(wdt), None if db is None else db.to(bdt), None, None, None, None,
                None)


def layer_norm(x: torch.Tensor, ln: nn.LayerNorm, full: bool = True, lowp: bool = False, passthrough: bool = False):
    """(y, y_lp), or (y, y_lp, x) with ``passthrough``, of ``ln(x)``; see the module docstring."""
    amp = x.is_cuda and torch.is_autocast_enabled("cuda")
    lowp = lowp and amp
    if not (full or lowp):
        full = True
    if not supported(x, ln):
        y = ln(x)
        res = (y if full else None), (y.to(torch.get_autocast_dtype("cuda")) if lowp else None)
        return res + (x,) if passthrough else res
    if amp and torch.get_autocast_dtype("cuda") != torch.bfloat16:
        lowp = False
        full = True
    y_dtype = torch.float32 if amp else x.dtype
    out = _LayerNorm.apply(x, ln.weight, ln.bias, ln.eps, y_dtype, full, lowp, passthrough)
    if not isinstance(out, tuple):
        out = (out,)
    out = list(out)
    y = out.pop(0) if full else None
    ylp = out.pop(0) if lowp else None
    return (y, ylp, out[0]) if passthrough else (y, ylp)
