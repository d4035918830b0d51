"""Mish and the MAB's ``out + mish(fc_o(out))`` epilogue on the gfx950 kernels.

``mab_epilogue(o, fc_o, residual)`` fuses the whole epilogue of a MAB on
packed rows: fc_o's GEMM, Mish and the residual(s) in one pass
(``esa_mish_fwd``, or ``esa_mab_residual_fwd`` with the block's fp32
residual stream), and a backward whose input gradient needs no add kernel.

``mish(z, residual)`` computes ``residual + mish(z)`` (``mish(z)`` without a
residual) in one pass, evaluated in fp32 and rounded once, through
``esa_mish_fwd``; its backward is ``esa_mish_bwd``.  It serves the reference's
``out = out + F.mish(self.fc_o(out))`` (esa/mha.py:87,
esa/mha_flash_varlen.py:120,195), the MLP activations ``nn.Mish()``
(esa/mlp_utils.py:24-37) and the decoder head ``F.mish(decoder_linear(.))``
(esa/masked_layers.py:929,934).

Device tensors always go to the HIP kernels (an unbuilt library raises); CPU
tensors, which the kernels cannot take, use ``torch.nn.functional.mish``.
"""
from __future__ import annotations

import torch
from torch import nn
from torch.nn import functional as F

from .. import _lib

_DTYPES = {torch.float32: _lib.ESA_F32, torch.bfloat16: _lib.ESA_BF16}


class _Mish(torch.autograd.Function):
    @staticmethod
    def forward(ctx, z, residual):
        code = _DTYPES[z.dtype]
        z = z.contiguous()
        if residual is not None:
            residual = residual.contiguous()
        y = torch.empty_like(z)
        rc = _lib.load().esa_mish_fwd(z.data_ptr(), _lib.ptr(residual), z.numel(), code, y.data_ptr(),
                                      _lib.stream_of(z))
        _lib.check(rc, "esa_mish_fwd")
        ctx.save_for_backward(z)
        ctx.has_residual = residual is not None
        return y

    @staticmethod
    def backward(ctx, g):
        (z,) = ctx.saved_tensors
        g = g.to(z.dtype).contiguous()
        dz = torch.empty_like(z)
        rc = _lib.load().esa_mish_bwd(z.data_ptr(), g.data_ptr(), z.numel(), _DTYPES[z.dtype], dz.data_ptr(),
                                      _lib.stream_of(z))
        _lib.check(rc, "esa_mish_bwd")
        return dz, (g if ctx.has_residual else None)


def mish(z: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
    """``residual + mish(z)``, or ``mish(z)`` when residual is None."""
    if not z.is_cuda:
        return F.mish(z) if residual is None else residual + F.mish(z)
    if z.dtype not in _DTYPES:
        raise TypeError(f"mish: unsupported dtype {z.dtype}; use float32 or bfloat16")
    if residual is not None and (residual.dtype != z.dtype or residual.shape != z.shape):
        # Mixed precision or broadcasting: torch's promotion rules for the add.
        return residual + _Mish.apply(z, None)
    return _Mish.apply(z, residual)


class _MabEpilogue(torch.autograd.Function):
    """y = o + mish(fc_o(o)) (x is None) or y = x + r(o + mish(fc_o(o))) (x the block's fp32 residual, r() the
    rounding to o's dtype): fc_o's GEMM, then esa_mish_fwd / esa_mab_residual_fwd.  Backward: one kernel gives
    dz (and o's residual gradient r(g) when x is given), and o's gradient is r(g) + dz W in one GEMM (addmm,
    beta = 1)."""

    @staticmethod
    def forward(ctx, o, weight, bias, x):
        from .linear import cast_param, linear_fwd   # deferred: linear.py is a sibling with its own imports
        ctx.dtypes = (weight.dtype, None if bias is None else bias.dtype)   # the gradients are returned in these
        weight, bias = cast_param(weight, o.dtype), cast_param(bias, o.dtype)
        (z,) = linear_fwd(o, [(weight, bias)])
        lib, st, code = _lib.load(), _lib.stream_of(o), _DTYPES[o.dtype]
        if x is None:
            y = torch.empty_like(z)
            _lib.check(lib.esa_mish_fwd(z.data_ptr(), o.data_ptr(), z.numel(), code, y.data_ptr(), st),
                       "esa_mish_fwd")
        else:
            y = torch.empty(x.shape, dtype=torch.float32, device=x.device)
            _lib.check(lib.esa_mab_residual_fwd(z.data_ptr(), o.data_ptr(), x.data_ptr(), z.numel(), code,
                                                y.data_ptr(), st), "esa_mab_residual_fwd")
        ctx.save_for_backward(o, weight, z)
        ctx.has_x = x is not None
        return y

    @staticmethod
    def backward(ctx, g):
        from .linear import column_sum, weight_grad   # deferred: linear.py is a sibling with its own imports
        o, weight, z = ctx.saved_tensors
        lib, st, code = _lib.load(), _lib.stream_of(z), _DTYPES[z.dtype]
        dz = torch.empty_like(z)
        if ctx.has_x:
            g = g.float().contiguous()
            g_o = torch.empty_like(z)
            _lib.check(lib.esa_mab_residual_bwd(z.data_ptr(), g.data_ptr(), z.numel(), code, dz.data_ptr(),
                                                g_o.data_ptr(), st), "esa_mab_residual_bwd")
        else:
            g_o = g.to(z.dtype).contiguous()
            _lib.check(lib.esa_mish_bwd(z.data_ptr(), g_o.data_ptr(), z.numel(), code, dz.data_ptr(), st),
                       "esa_mish_bwd")
        wdt, bdt = ctx.dtypes
        do = torch.addmm(g_o, dz, weight) if ctx.needs_input_grad[0] else None
        dw = weight_grad(dz, o).to(wdt) if ctx.needs_input_grad[1] else None
        db = column_sum(dz).to(bdt) if bdt is not None and ctx.needs_input_grad[2] else None
        return do, dw, db, (g if ctx.has_x and ctx.needs_input_grad[3] else None)


def mab_epilogue(o: torch.Tensor, fc_o: nn.Linear, residual: torch.Tensor | None = None) -> torch.Tensor:
    """``o + mish(fc_o(o))`` (esa/mha.py:87) on 2-D token rows, plus the block residual when given
    (``residual + (o + mish(fc_o(o)))``, esa/masked_layers.py:471-472), fused on device tensors."""
    if not o.is_cuda:
        y = o + F.mish(fc_o(o))
        return y if residual is None else residual + y
    from .linear import compute_dtype
    w, b = fc_o.weight, fc_o.bias
    dt = compute_dtype(o, w, b)
    if dt not in _DTYPES or o.dim() != 2:
        o = o if dt is None else o.to(dt)
        y = mish(F.linear(o, w if dt is None else w.to(dt), b if dt is None or b is None else b.to(dt)), o)
        return y if residual is None else residual + y
    o = o.to(dt).contiguous()
    if residual is not None and (residual.dtype != torch.float32 or residual.shape != o.shape):
        return residual + _MabEpilogue.apply(o, w, b, None)
    return _MabEpilogue.apply(o, w, b, None if residual is None else residual.contiguous())


_FUSED_COLSUM_MIN_COLS = 1024


class _LinearMish(torch.autograd.Function):
    """y = mish(x W^T + b), an MLP's Linear -> Mish (esa/mlp_utils.py:18-37).  Forward: the GEMM, then
    esa_mish_fwd.  Backward: esa_mish_bwd_colsum writes dz and the bias gradient (dz's column sums) in one
    pass; dx = dz W and the split-K weight gradient follow.  Parameters enter in their own dtype and are cast
    inside, so their gradients are returned in it (fp32 under autocast)."""

    @staticmethod
    def forward(ctx, x, weight, bias):
        from .linear import cast_param, linear_fwd   # deferred: linear.py is a sibling with its own imports
        ctx.dtypes = (weight.dtype, None if bias is None else bias.dtype)
        w, b = cast_param(weight, x.dtype), cast_param(bias, x.dtype)
        (z,) = linear_fwd(x, [(w, b)])
        y = torch.empty_like(z)
        _lib.check(_lib.load().esa_mish_fwd(z.data_ptr(), None, z.numel(), _DTYPES[z.dtype], y.data_ptr(),
                                            _lib.stream_of(z)), "esa_mish_fwd")
        ctx.save_for_backward(x, w, z)
        return y

    @staticmethod
    def backward(ctx, g):
        import ctypes

        from .linear import column_sum, weight_grad
        x, w, z = ctx.saved_tensors
        wdt, bdt = ctx.dtypes
        lib, st, code = _lib.load(), _lib.stream_of(z), _DTYPES[z.dtype]
        g = g.to(z.dtype).contiguous()
        dz = torch.empty_like(z)
        rows, cols = z.shape
        db = None
        # fused from 1024 columns (129,850 x 2048 bf16: 334 vs 397 us for the two kernels); at 512 columns the
        # two cost the same (104 vs 105 us) and the two kernels run
        if bdt is not None and ctx.needs_input_grad[2] and cols % 4 == 0 and cols >= _FUSED_COLSUM_MIN_COLS:
            n = ctypes.c_size_t(0)
            _lib.check(lib.esa_column_sum_workspace_size(rows, cols, ctypes.byref(n)), "esa_column_sum_workspace_size")
            ws = torch.empty(int(n.value), dtype=torch.uint8, device=z.device)
            db = torch.empty(cols, dtype=torch.float32, device=z.device)
            _lib.check(lib.esa_mish_bwd_colsum(z.data_ptr(), g.data_ptr(), rows, cols, code, dz.data_ptr(),
                                               db.data_ptr(), ws.data_ptr(), ws.numel(), st), "esa_mish_bwd_colsum")
        else:
            _lib.check(lib.esa_mish_bwd(z.data_ptr(), g.data_ptr(), z.numel(), code, dz.data_ptr(), st),
                       "esa_mish_bwd")
            if bdt is not None and ctx.needs_input_grad[2]:
                db = column_sum(dz)
        dx = dz.mm(w) if ctx.needs_input_grad[0] else None
        dw = weight_grad(dz, x).to(wdt) if ctx.needs_input_grad[1] else None
        return dx, dw, None if db is None else db.to(bdt)


def linear_mish(x: torch.Tensor, layer: nn.Linear) -> torch.Tensor:
    """``mish(layer(x))`` with the fused backward of _LinearMish on device tensors."""
    if not x.is_cuda:
        return F.mish(layer(x))
    from .linear import compute_dtype, linear
    dt = compute_dtype(x, layer.weight, layer.bias)
    if dt not in _DTYPES:
        return mish(linear(x, layer.weight, layer.bias))
    x = x.to(dt)
    lead = x.shape[:-1]
    y = _LinearMish.apply(x.reshape(-1, x.shape[-1]).contiguous(), layer.weight, layer.bias)
    return y.view(*lead, layer.weight.shape[0])


class Mish(nn.Mish):
    """nn.Mish on the HIP kernel (no parameters; state dicts are unchanged)."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return mish(x)
