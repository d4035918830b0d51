"""Mish and the MAB's ``out + mish(fc_o(out))`` epilogue on the gfx950 kernels.

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


class Mish(nn.Mish):
    """nn.Mish on the HIP kernel (no parameters; state dicts are unchanged)."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return mish(x)
