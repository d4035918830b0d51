"""MLPs of the ESA blocks (esa/mlp_utils.py), same module and parameter names.

These are GEMM + activation stacks that stay on PyTorch (hipBLASLt); they are
restated so the ESA blocks run without flash-attn.  ``swiglu(gate, y)`` is
silu(gate) * y, the function flash_attn.ops.activations.swiglu computes
(esa/mlp_utils.py:3,83).
"""
from __future__ import annotations

from torch import nn
from torch.nn import functional as F

from .activations import Mish, linear_mish
from .linear import apply, hookless, linear


def swiglu(gate, y):
    return F.silu(gate) * y


class SmallMLP(nn.Module):
    """Linear/Mish stack (esa/mlp_utils.py:6-48)."""

    def __init__(self, in_dim, inter_dim, out_dim, dropout_p=0.0, num_layers=2, use_ln=False):
        super().__init__()
        if num_layers == 1:
            self.mlp = nn.Sequential(
                nn.Linear(in_dim, out_dim),
                nn.Dropout(p=dropout_p) if dropout_p > 0 else nn.Identity(),
                Mish(),
            )
            return
        layers = []
        for i in range(num_layers):
            d_in = in_dim if i == 0 else inter_dim
            d_out = out_dim if i == num_layers - 1 else inter_dim
            layers.append(nn.Linear(d_in, d_out))
            if i != num_layers - 1:
                if use_ln:
                    layers.append(nn.LayerNorm(inter_dim))
                layers.append(Mish())
            if dropout_p > 0:
                layers.append(nn.Dropout(p=dropout_p))
        self.mlp = nn.Sequential(*layers)

    def forward(self, x):
        layers = list(self.mlp)
        i = 0
        while i < len(layers):
            nxt = layers[i + 1] if i + 1 < len(layers) else None
            if (type(layers[i]) is nn.Linear and type(nxt) in (Mish, nn.Mish) and hookless(layers[i])
                    and hookless(nxt)):
                x = linear_mish(x, layers[i])   # Linear -> Mish: the bias gradient comes with Mish's backward
                i += 2
            else:
                x = apply(layers[i], x)
                i += 1
        return x


class GatedMLPSingle(nn.Module):
    """fc1 -> split (y, gate) -> swiglu -> fc2 (esa/mlp_utils.py:51-89)."""

    def __init__(self, in_dim, inter_dim, out_dim, dropout_p=0.0, use_ln=False):
        super().__init__()
        self.fc1 = nn.Linear(in_dim, 2 * inter_dim, bias=True)
        self.fc2 = nn.Linear(inter_dim, out_dim, bias=True)
        self.use_ln = use_ln
        if use_ln:
            self.ln = nn.LayerNorm(2 * inter_dim, eps=1e-8)

    def forward(self, x):
        y = linear(x, self.fc1.weight, self.fc1.bias)
        if self.use_ln:
            y = self.ln(y)
        y, gate = y.chunk(2, dim=-1)
        return linear(swiglu(gate, y), self.fc2.weight, self.fc2.bias)


class GatedMLPMulti(nn.Module):
    """Stack of GatedMLPSingle + Mish (esa/mlp_utils.py:92-129)."""

    def __init__(self, in_dim, inter_dim, out_dim, dropout_p=0.0, num_layers=2, use_ln=False):
        super().__init__()
        if num_layers == 1:
            self.mlp = nn.Sequential(
                GatedMLPSingle(in_dim, inter_dim, out_dim, dropout_p=dropout_p, use_ln=False),
                nn.Dropout(p=dropout_p) if dropout_p > 0 else nn.Identity(),
                Mish(),
            )
            return
        layers = []
        for i in range(num_layers):
            d_in = in_dim if i == 0 else inter_dim
            d_out = out_dim if i == num_layers - 1 else inter_dim
            layers.append(GatedMLPSingle(d_in, inter_dim, d_out, dropout_p=dropout_p, use_ln=use_ln))
            if dropout_p > 0:
                layers.append(nn.Dropout(p=dropout_p))
            layers.append(Mish())
        self.mlp = nn.Sequential(*layers)

    def forward(self, x):
        for layer in self.mlp:
            x = apply(layer, x)
        return x
