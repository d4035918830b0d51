"""Norm wrappers of the ESA blocks (esa/utils/norm_layers.py), same names."""
from torch import nn


class LN(nn.Module):
    """nn.LayerNorm(hidden_dim, eps=1e-8) behind a `.ln` attribute (esa/utils/norm_layers.py:27-37)."""

    def __init__(self, hidden_dim, num_elements=None):
        super().__init__()
        self.ln = nn.LayerNorm(hidden_dim, eps=1e-8)

    def forward(self, x):
        return self.ln(x)
