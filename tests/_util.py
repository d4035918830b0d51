"""Shared test helpers: seeded inputs and error metrics."""
from __future__ import annotations

import numpy as np
import torch

# Tolerances of the north-star parity bar for bf16 attention outputs.
BF16_MAX_ABS = 2e-2
BF16_MEAN_ABS = 2e-3


def seeded_normal(shape, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float32).to(dtype)


def err(a: torch.Tensor, b: torch.Tensor) -> tuple[float, float]:
    d = (a.detach().double().cpu() - b.detach().double().cpu()).abs()
    return float(d.max()) if d.numel() else 0.0, float(d.mean()) if d.numel() else 0.0


def assert_bf16_close(got, ref, scale: float = 1.0, what: str = ""):
    """max-abs <= 2e-2 * scale and mean-abs <= 2e-3 * scale."""
    mx, mn = err(got, ref)
    assert mx <= BF16_MAX_ABS * scale and mn <= BF16_MEAN_ABS * scale, (
        f"{what}: max-abs {mx:.3e} (bar {BF16_MAX_ABS * scale:.3e}), mean-abs {mn:.3e} "
        f"(bar {BF16_MEAN_ABS * scale:.3e})")


F32_REL = 1e-5


def assert_f32_close(got, ref, what: str = ""):
    """fp32 bar: max-abs <= 1e-5 * max(1, max |ref|) (relative, norm-wise)."""
    mx, _ = err(got, ref)
    bar = F32_REL * max(1.0, float(ref.abs().max()) if ref.numel() else 0.0)
    assert mx <= bar, f"{what}: max-abs {mx:.3e} > {bar:.3e} (fp32 bar)"


def grad_scale(ref: torch.Tensor) -> float:
    """Gradients are checked relative to their own magnitude (at least 1)."""
    return max(1.0, float(ref.abs().max()))


def cu_from_lengths(lengths) -> np.ndarray:
    return np.concatenate([[0], np.cumsum(np.asarray(lengths, dtype=np.int64))]).astype(np.int32)


def node_graph(seed, sizes, extra_dup=True, self_loops=True):
    """A PyG-style node batch (edge_index [2, E], batch [N]): random directed edges inside each graph, plus
    repeated edges (the first five again) and, optionally, self-loops."""
    rng = np.random.default_rng(seed)
    bm = np.concatenate([np.full(n, b) for b, n in enumerate(sizes)]).astype(np.int64)
    first = np.concatenate([[0], np.cumsum(sizes)[:-1]])
    src, dst = [], []
    for b, n in enumerate(sizes):
        e = 3 * n
        s = rng.integers(0, n, size=e) + first[b]
        d = rng.integers(0, n, size=e) + first[b]
        keep = s != d if not self_loops else np.ones(e, bool)
        src.append(s[keep])
        dst.append(d[keep])
    src, dst = np.concatenate(src), np.concatenate(dst)
    if extra_dup:
        src, dst = np.concatenate([src, src[:5]]), np.concatenate([dst, dst[:5]])
    return np.stack([src, dst]).astype(np.int64), bm
