"""GPU parity of the Mish block epilogue kernels (esa_mish_fwd / esa_mish_bwd) against the oracle.

The kernels evaluate mish in fp32 and round once, so the bars are per element:
fp32 |got - ref| <= 1e-5 |ref| + 1e-6 * scale (the north-star fp32 bar, with an
absolute floor at the scale of the operands for values near zero); bf16
|got - ref| <= (2^-8 + 1e-5) |ref| + 1e-6 * scale, i.e. one rounding to bf16
(half an ulp is 2^-9 relative; 2^-8 allows the fp32 value to sit on the other
side of a rounding boundary) plus the fp32 error.
"""
import ctypes

import pytest
import torch

from mind_amd import _lib
from mind_amd.esa.activations import Mish, mish
from oracle import modules as OMod

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16]
CODE = {torch.float32: _lib.ESA_F32, torch.bfloat16: _lib.ESA_BF16}
REL = {torch.float32: 1e-5, torch.bfloat16: 2.0 ** -8 + 1e-5}


def _values(n, seed, dtype):
    """Normal values spread over [-25, 25] plus the special points of mish."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, generator=g, dtype=torch.float64) * 6.0
    special = torch.tensor([0.0, -0.0, 1e-30, -1e-30, -1.1924, 19.99, 20.0, 20.01, 100.0, -100.0, -20.0,
                            float("inf"), float("-inf"), float("nan"), -88.0, 88.0, 3.0e38, -3.0e38],
                           dtype=torch.float64)
    k = min(n, special.numel())
    x[:k] = special[:k]
    return x.to(dtype)


def _bits(t):
    """Bit patterns (NaN-safe bitwise equality)."""
    return t.view(torch.int32 if t.dtype == torch.float32 else torch.int16)


def _check(got, ref, dtype, scale, what):
    got = got.double().cpu()
    fin = torch.isfinite(ref)
    assert torch.equal(torch.isfinite(got), fin), f"{what}: non-finite pattern differs"
    nan = torch.isnan(ref)
    assert torch.equal(torch.isnan(got), nan), f"{what}: NaN pattern differs"
    assert torch.equal(got[~fin & ~nan], ref[~fin & ~nan]), f"{what}: infinities differ"
    bar = REL[dtype] * ref[fin].abs() + 1e-6 * scale
    over = (got[fin] - ref[fin]).abs() > bar
    assert not over.any(), (f"{what}: {int(over.sum())} values off; worst at "
                            f"{float((got[fin] - ref[fin]).abs().max()):.3e}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [1, 7, 8, 9, 4099, 1 << 20])
def test_mish_fwd_and_bwd(device, dtype, n):
    z = _values(n, seed=n, dtype=dtype)
    gr = _values(n, seed=n + 1, dtype=dtype).clamp(-8, 8)
    res = _values(n, seed=n + 2, dtype=dtype).clamp(-8, 8)
    zd, gd, rd = z.to(device), gr.to(device), res.to(device)
    y = torch.empty_like(zd)
    lib, st = _lib.load(), _lib.stream_of(zd)
    z64, g64, r64 = z.double(), gr.double(), res.double()
    ref = OMod.mish(z64)
    _lib.check(lib.esa_mish_fwd(zd.data_ptr(), None, n, CODE[dtype], y.data_ptr(), st), "fwd")
    _check(y, ref, dtype, 1.0, "mish")
    _lib.check(lib.esa_mish_fwd(zd.data_ptr(), rd.data_ptr(), n, CODE[dtype], y.data_ptr(), st), "fwd+res")
    _check(y, r64 + ref, dtype, 8.0, "res + mish")
    dz = torch.empty_like(zd)
    _lib.check(lib.esa_mish_bwd(zd.data_ptr(), gd.data_ptr(), n, CODE[dtype], dz.data_ptr(), st), "bwd")
    _check(dz, g64 * OMod.mish_grad(z64), dtype, 8.0, "g * mish'")


@pytest.mark.parametrize("dtype", DTYPES)
def test_mish_in_place_and_misaligned(device, dtype):
    """y may alias z; pointers off the 16-byte grid take the element-wise kernel with bitwise the same
    results."""
    n = 10_001
    z = _values(n, seed=3, dtype=dtype).to(device)
    lib, st = _lib.load(), _lib.stream_of(z)
    ref = torch.empty_like(z)
    _lib.check(lib.esa_mish_fwd(z.data_ptr(), None, n, CODE[dtype], ref.data_ptr(), st), "fwd")
    zz = z.clone()
    _lib.check(lib.esa_mish_fwd(zz.data_ptr(), None, n, CODE[dtype], zz.data_ptr(), st), "in place")
    assert torch.equal(_bits(zz), _bits(ref))
    buf = torch.empty(n + 1, dtype=dtype, device=device)
    buf[1:] = z
    out = torch.empty(n + 1, dtype=dtype, device=device)
    _lib.check(lib.esa_mish_fwd(buf[1:].data_ptr(), None, n, CODE[dtype], out[1:].data_ptr(), st), "misaligned")
    assert torch.equal(_bits(out[1:]), _bits(ref))
    g = _values(n, seed=4, dtype=dtype).clamp(-8, 8).to(device)
    dz = torch.empty_like(z)
    _lib.check(lib.esa_mish_bwd(z.data_ptr(), g.data_ptr(), n, CODE[dtype], dz.data_ptr(), st), "bwd")
    gbuf = torch.empty(n + 1, dtype=dtype, device=device)
    gbuf[1:] = g
    _lib.check(lib.esa_mish_bwd(buf[1:].data_ptr(), gbuf[1:].data_ptr(), n, CODE[dtype], out[1:].data_ptr(), st),
               "bwd misaligned")
    assert torch.equal(_bits(out[1:]), _bits(dz))


@pytest.mark.parametrize("dtype", DTYPES)
def test_mish_autograd_with_residual(device, dtype):
    """mish(z, r) = r + mish(z): gradients g * mish'(z) and g, as torch's `r + F.mish(z)`."""
    g = torch.Generator().manual_seed(5)
    z = (torch.randn(64, 96, generator=g) * 4).to(dtype)
    r = torch.randn(64, 96, generator=g).to(dtype)
    up = torch.randn(64, 96, generator=g).to(dtype)
    zd, rd = z.to(device).requires_grad_(True), r.to(device).requires_grad_(True)
    out = mish(zd, rd)
    out.backward(up.to(device))
    z64 = z.double()
    _check(out.detach(), r.double() + OMod.mish(z64), dtype, 4.0, "out")
    _check(zd.grad, up.double() * OMod.mish_grad(z64), dtype, 4.0, "dz")
    assert torch.equal(rd.grad.cpu(), up)
    # the module form (MLP activation), and a residual of another dtype (torch promotion)
    m = Mish()(zd.detach())
    _check(m, OMod.mish(z64), dtype, 1.0, "Mish()")
    if dtype == torch.bfloat16:
        mixed = mish(zd.detach(), rd.detach().float())
        assert mixed.dtype == torch.float32
        _check(mixed, r.double() + m.double().cpu(), torch.float32, 4.0, "mixed")


def test_mish_argument_errors(device):
    lib = _lib.load()
    z = torch.zeros(16, device=device)
    assert lib.esa_mish_fwd(z.data_ptr(), None, 16, 7, z.data_ptr(), None) == -5
    assert lib.esa_mish_fwd(z.data_ptr(), None, -1, _lib.ESA_F32, z.data_ptr(), None) == -2
    assert lib.esa_mish_bwd(None, z.data_ptr(), 16, _lib.ESA_F32, z.data_ptr(), None) == -1
    assert lib.esa_mish_bwd(None, None, 0, _lib.ESA_F32, None, None) == 0
    with pytest.raises(TypeError):
        mish(z.half())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("tokens,out_f,in_f", [(100, 48, 40), (3 * 4096 + 7, 64, 96), (65536 + 3, 512, 512),
                                               (40000, 2048, 512)])
def test_split_k_linear(device, dtype, tokens, out_f, in_f):
    """linear(x, W, b): forward and dx as F.linear's autograd; dW by token chunks against the fp64 oracle.

    dW bar: fp32 1e-5 relative to max |dW| (plus the fp32 accumulation over T terms, T 2^-24 max|g x|); bf16
    one rounding (2^-8 relative) plus the same accumulation term."""
    from mind_amd.esa.linear import linear, split_count
    gen = torch.Generator().manual_seed(tokens + out_f)
    x = torch.randn(tokens, in_f, generator=gen).to(dtype)
    w = (torch.randn(out_f, in_f, generator=gen) * 0.05).to(dtype)
    b = torch.randn(out_f, generator=gen).to(dtype)
    g = torch.randn(tokens, out_f, generator=gen).to(dtype)
    xd, wd, bd = (t.to(device).requires_grad_(True) for t in (x, w, b))
    y = linear(xd, wd, bd)
    y.backward(g.to(device))
    xr, wr, br = (t.to(device).requires_grad_(True) for t in (x, w, b))
    yr = torch.nn.functional.linear(xr, wr, br)
    yr.backward(g.to(device))
    assert torch.equal(y, yr)
    assert torch.equal(xd.grad, xr.grad)
    assert torch.equal(bd.grad, br.grad)
    ref = g.double().t() @ x.double()
    acc = tokens * 2.0 ** -24 * float((g.double().abs().max() * x.double().abs().max()))
    got = wd.grad.double().cpu()
    if dtype == torch.float32:
        assert float((got - ref).abs().max()) <= 1e-5 * float(ref.abs().max()) + acc
    else:
        assert bool(((got - ref).abs() <= 2.0 ** -8 * ref.abs() + acc).all())
    if tokens >= 65536:
        assert split_count(tokens, out_f, in_f) > 1


@pytest.mark.gpu
def test_split_k_linear_under_autocast(device):
    """fp32 parameters under autocast(bf16): the output is bf16 and gradients reach the fp32 parameters."""
    from mind_amd.esa.linear import linear
    gen = torch.Generator().manual_seed(9)
    lin = torch.nn.Linear(256, 128).to(device)
    x = torch.randn(20000, 256, generator=gen).to(device)
    g = torch.randn(20000, 128, generator=gen).to(device).to(torch.bfloat16)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = linear(x, lin.weight, lin.bias)
        yr = lin(x)
    assert y.dtype == torch.bfloat16 and torch.equal(y, yr)
    y.backward(g)
    assert lin.weight.grad.dtype == torch.float32
    ref = g.double().t().cpu() @ x.to(torch.bfloat16).double().cpu()
    assert_rel = (lin.weight.grad.double().cpu() - ref).abs() <= 2.0 ** -8 * ref.abs() + 20000 * 2.0 ** -24 * 40
    assert bool(assert_rel.all())
    assert torch.allclose(lin.bias.grad.double().cpu(), g.double().sum(0).cpu(), rtol=2.0 ** -7, atol=1e-2)
