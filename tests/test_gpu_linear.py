"""GPU parity of the fp32 Linear kernel (esa_linear_f32 through mind_amd.esa.linear.esa_linear) against fp64
products and torch's fp32 F.linear, and the routing of linear_fwd (two or three weights over one input take the
kernel, one weight F.linear).

Bar: fp32 accumulation over K products, taken norm-wise per output: max |got - ref64| <= 1e-5 * max(1, max
|ref64|) (the north-star fp32 bar); torch's fp32 GEMM meets the same bar on the same data.  Shapes: rows around
the 16-row wave and 64-row block edges, configuration 0's token count, K of 16-512, N of 64-512, one to three
weights over one input (the MAB's fc_q / fc_k / fc_v), with and without bias.
"""
import pytest
import torch
from torch.nn import functional as F

from mind_amd.esa import linear as L

pytestmark = pytest.mark.gpu


def _data(rows, k, ns, seed, bias=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, k, generator=g)
    pairs = [(torch.randn(n, k, generator=g) / k ** 0.5, torch.randn(n, generator=g) if bias else None) for n in ns]
    return x, pairs


def _check(device, rows, k, ns, seed, bias=True):
    x, pairs = _data(rows, k, ns, seed, bias)
    xd = x.to(device)
    pd = [(w.to(device), None if b is None else b.to(device)) for w, b in pairs]
    assert L._f32_linear_ok(xd, pd)
    got = L.esa_linear(xd, pd)
    torch.cuda.synchronize()
    for (w, b), y, (wd, bd) in zip(pairs, got, pd):
        ref = F.linear(x.double(), w.double(), None if b is None else b.double())
        bar = 1e-5 * max(1.0, float(ref.abs().max())) if ref.numel() else 0.0
        assert y.shape == ref.shape and y.dtype == torch.float32
        assert float((y.cpu().double() - ref).abs().max()) <= bar if ref.numel() else True
        tref = F.linear(xd, wd, bd).cpu().double()
        assert float((tref - ref).abs().max()) <= bar if ref.numel() else True


@pytest.mark.parametrize("rows", [1, 15, 16, 17, 63, 64, 65, 1000, 21752])
def test_rows(device, rows):
    _check(device, rows, 128, [128], seed=rows)


@pytest.mark.parametrize("k,ns", [(16, [64]), (128, [256]), (256, [128]), (512, [512]), (48, [64, 192])])
def test_k_and_n(device, k, ns):
    _check(device, 777, k, ns, seed=k + sum(ns))


@pytest.mark.parametrize("bias", [True, False])
def test_three_outputs_share_one_input(device, bias):
    _check(device, 3001, 128, [128, 128, 128], seed=5, bias=bias)
    _check(device, 129, 64, [64, 128, 256], seed=6, bias=bias)


def test_zero_rows_and_routing(device):
    x = torch.zeros(0, 128, device=device)
    w = torch.randn(128, 128, device=device)
    (y,) = L.esa_linear(x, [(w, None)])
    assert y.shape == (0, 128)
    # one weight: F.linear, bit for bit; two or three: the kernel
    xr = torch.randn(100, 128, device=device)
    (y1,) = L.linear_fwd(xr, [(w, None)])
    assert torch.equal(y1, F.linear(xr, w))
    y2 = L.linear_fwd(xr, [(w, None), (w, None)])
    assert all(torch.equal(a, b) for a, b in zip(y2, L.esa_linear(xr, [(w, None), (w, None)])))
    with pytest.raises(ValueError):
        L.esa_linear(xr, [(torch.randn(96, 128, device=device), None)])
    # shapes outside the kernel's (N % 64, bf16, a strided x) go to F.linear with the same results
    assert not L._f32_linear_ok(torch.zeros(8, 128, device=device), [(torch.zeros(96, 128, device=device), None)])
    assert not L._f32_linear_ok(torch.zeros(8, 128, device=device, dtype=torch.bfloat16),
                                [(torch.zeros(64, 128, device=device, dtype=torch.bfloat16), None)])
    xs = torch.randn(8, 256, device=device)[:, :128]
    assert not L._f32_linear_ok(xs, [(w, None)])
    (ys,) = L.linear_fwd(xs, [(w, None)])
    assert torch.equal(ys, F.linear(xs, w))


def test_deterministic(device):
    x, pairs = _data(5000, 256, [128, 256], 9)
    xd = x.to(device)
    pd = [(w.to(device), b.to(device)) for w, b in pairs]
    a = L.esa_linear(xd, pd)
    b = L.esa_linear(xd, pd)
    for u, v in zip(a, b):
        assert torch.equal(u, v)
