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
    # bias gradient: fp32 column sum rounded once, against the fp64 sum
    rdb = g.double().sum(0)
    bacc = tokens * 2.0 ** -24 * float(g.double().abs().max())
    bbar = (2.0 ** -8 if dtype == torch.bfloat16 else 1e-5) * rdb.abs() + bacc
    assert bool(((bd.grad.double().cpu() - rdb).abs() <= bbar).all())
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


def _ln_oracle(x, w, b, g, eps=1e-8):
    """fp64 LayerNorm (the oracle's restatement, pinned against F.layer_norm) and its autograd gradients."""
    xd = x.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    bd = b.double().requires_grad_(True)
    sd = {"ln.weight": wd, "ln.bias": bd}
    y = OMod.layer_norm(sd, "ln.", xd, eps=eps)
    y.backward(g.double())
    return y.detach(), xd.grad, wd.grad, bd.grad


@pytest.mark.parametrize("passthrough", [False, True], ids=["plain", "passthrough"])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,feat", [(1, 4), (5, 128), (1000, 512), (4099, 512), (300, 260), (64, 2048)])
def test_layer_norm_fwd_bwd(device, dtype, rows, feat, passthrough):
    """y (x's dtype) plus its bf16 copy; backward with gradients on both outputs, against the fp64 oracle.
    With the pass-through output (x itself, as a residual uses it), its gradient is added to dx in the kernel:
    dx = the oracle's dx + that gradient.

    Bars: fp32 outputs 1e-5 * max(1, max|ref|) (the fp32 bar, norm-wise); bf16 outputs one rounding
    (2^-8 relative) + 1e-5 * scale (the fp32 evaluation's error); dweight / dbias 1e-5 * max(1, max|ref|) plus
    the fp32 accumulation over the rows (rows * 2^-24 * max|term|)."""
    from mind_amd.esa.layer_norm import _LayerNorm
    gen = torch.Generator().manual_seed(rows * 7 + feat)
    x = (torch.randn(rows, feat, generator=gen) * 3 + 1.5).to(dtype)
    w = torch.randn(feat, generator=gen)
    b = torch.randn(feat, generator=gen)
    gy = torch.randn(rows, feat, generator=gen).to(dtype)
    gl = torch.randn(rows, feat, generator=gen).to(torch.bfloat16)
    xd, wd, bd = x.to(device).requires_grad_(True), w.to(device).requires_grad_(True), b.to(device).requires_grad_(True)
    outs = _LayerNorm.apply(xd, wd, bd, 1e-8, dtype, True, True, passthrough)
    y, ylp = outs[:2]
    assert y.dtype == dtype and ylp.dtype == torch.bfloat16
    assert torch.equal(ylp, y.to(torch.bfloat16))
    gr = torch.randn(rows, feat, generator=gen).to(dtype)
    if passthrough:
        assert torch.equal(outs[2], xd.detach())
        torch.autograd.backward(list(outs), [gy.to(device), gl.to(device), gr.to(device)])
    else:
        torch.autograd.backward([y, ylp], [gy.to(device), gl.to(device)])
    ref, rdx, rdw, rdb = _ln_oracle(x, w, b, gy.double() + gl.double())
    if passthrough:
        rdx = rdx + gr.double()
    if dtype == torch.float32:
        assert_close = lambda got, r, what: _f32_norm_close(got, r, what)  # noqa: E731
    else:
        assert_close = lambda got, r, what: _check(got, r, torch.bfloat16, 10 * max(1.0, float(r.abs().max())),  # noqa: E731
                                                   what)
    assert_close(y.detach(), ref, "y")
    _check(ylp.detach(), ref, torch.bfloat16, max(1.0, float(ref.abs().max())), "y_lp")
    assert_close(xd.grad, rdx, "dx")
    xhat = (x.double() - x.double().mean(1, keepdim=True)) / x.double().std(1, unbiased=False, keepdim=True)
    gsum = (gy.double() + gl.double())
    for got, r, term in ((wd.grad, rdw, gsum * xhat), (bd.grad, rdb, gsum)):
        acc = rows * 2.0 ** -24 * float(term.abs().max())
        assert float((got.double().cpu() - r).abs().max()) <= 1e-5 * max(1.0, float(r.abs().max())) + acc


def _f32_norm_close(got, ref, what):
    got = got.detach().double().cpu()
    bar = 1e-5 * max(1.0, float(ref.abs().max()))
    assert float((got - ref).abs().max()) <= bar, f"{what}: {float((got - ref).abs().max()):.3e} > {bar:.3e}"


def test_layer_norm_module_under_autocast(device):
    """layer_norm(x, ln) under autocast: y equals F.layer_norm's fp32 output to the fp32 bar, y_lp is y rounded
    to bf16 bit for bit, gradients reach ln's fp32 parameters; the backward is deterministic."""
    from mind_amd.esa.layer_norm import layer_norm
    gen = torch.Generator().manual_seed(11)
    ln = torch.nn.LayerNorm(512, eps=1e-8).to(device)
    with torch.no_grad():
        ln.weight.normal_(generator=None)
        ln.bias.normal_()
    x = (torch.randn(3000, 512, generator=gen) * 2).to(device)
    g = torch.randn(3000, 512, generator=gen).to(device)
    grads = []
    for _ in range(2):
        ln.zero_grad()
        xd = x.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y, ylp = layer_norm(xd, ln, full=True, lowp=True)
            only_lp = layer_norm(xd, ln, full=False, lowp=True)[1]
        assert y.dtype == torch.float32 and ylp.dtype == torch.bfloat16
        assert torch.equal(ylp, y.to(torch.bfloat16)) and torch.equal(only_lp, ylp)
        ref = torch.nn.functional.layer_norm(x, (512,), ln.weight, ln.bias, 1e-8)
        _f32_norm_close(y, ref.double().cpu(), "y vs F.layer_norm")
        (y * g).sum().backward(retain_graph=True)
        ylp.float().mul(g).sum().backward()
        grads.append((xd.grad.clone(), ln.weight.grad.clone(), ln.bias.grad.clone()))
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_layer_norm_edge_cases(device):
    """Constant rows (var = 0: y = bias), no rows (zero parameter gradients), unsupported widths via torch."""
    from mind_amd.esa.layer_norm import _LayerNorm, layer_norm, supported
    w = torch.randn(64, device=device, requires_grad=True)
    b = torch.randn(64, device=device, requires_grad=True)
    x = torch.full((3, 64), 2.5, device=device)
    y = _LayerNorm.apply(x, w, b, 1e-8, torch.float32, True, False, False)
    assert torch.allclose(y, b.detach().expand(3, 64), atol=1e-6)
    e = torch.empty(0, 64, device=device, requires_grad=True)
    ye = _LayerNorm.apply(e, w, b, 1e-8, torch.float32, True, False, False)
    ye.sum().backward()
    assert torch.equal(w.grad, torch.zeros_like(w)) and torch.equal(b.grad, torch.zeros_like(b))
    ln = torch.nn.LayerNorm(6).to(device)
    x6 = torch.randn(4, 6, device=device)
    assert not supported(x6, ln)
    assert torch.equal(layer_norm(x6, ln)[0], ln(x6))
    # only the pass-through output carries a gradient: dx is that gradient
    xp = torch.randn(5, 64, device=device, requires_grad=True)
    _, _, xr = layer_norm(xp, torch.nn.LayerNorm(64).to(device), passthrough=True)
    (xr * 3).sum().backward()
    assert torch.equal(xp.grad, torch.full_like(xp, 3.0))
    lib = _lib.load()
    assert lib.esa_layer_norm_fwd(x.data_ptr(), 0, None, None, 3, 6, 1e-8, x.data_ptr(), 0, None, x.data_ptr(),
                                  x.data_ptr(), None) == -2


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,cols", [(0, 8), (1, 4), (31, 12), (1000, 512), (131072, 512), (5000, 2052),
                                       (70001, 1024)])
def test_column_sum(device, dtype, rows, cols):
    """esa_column_sum against the fp64 sum (bar: 1e-5 relative + rows 2^-24 max|x| of fp32 accumulation) and
    bitwise repeatable."""
    from mind_amd.esa.linear import column_sum
    gen = torch.Generator().manual_seed(rows + cols)
    x = torch.randn(rows, cols, generator=gen).to(dtype)
    xd = x.to(device)
    a = column_sum(xd)
    b = column_sum(xd)
    assert a.dtype == torch.float32 and torch.equal(a, b)
    ref = x.double().sum(0)
    bar = 1e-5 * ref.abs() + rows * 2.0 ** -24 * (float(x.double().abs().max()) if rows else 0.0) + 1e-30
    assert bool(((a.double().cpu() - ref).abs() <= bar).all())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,cols", [(0, 8), (1, 4), (37, 2048), (5000, 516), (131072, 512), (65539, 1024)])
def test_mish_bwd_colsum_matches_unfused(device, dtype, rows, cols):
    """esa_mish_bwd_colsum: dz bit-equal to esa_mish_bwd's and the bias gradient bit-equal to esa_column_sum over
    that dz (the same row ranges, order and rounding); no rows gives a zero bias gradient.  65,539 x 1024: 2048
    row ranges of 33 rows, one of them holding a single row and the 61 after it empty."""
    import ctypes
    from mind_amd.esa.linear import column_sum
    gen = torch.Generator().manual_seed(rows + 3 * cols)
    z = (torch.randn(rows, cols, generator=gen) * 4).to(dtype).to(device)
    g = torch.randn(rows, cols, generator=gen).to(dtype).to(device)
    lib, code = _lib.load(), _lib.ESA_F32 if dtype == torch.float32 else _lib.ESA_BF16
    st = _lib.stream_of(z)
    dz_ref = torch.empty_like(z)
    assert lib.esa_mish_bwd(z.data_ptr(), g.data_ptr(), z.numel(), code, dz_ref.data_ptr(), st) == 0
    n = ctypes.c_size_t(0)
    assert lib.esa_column_sum_workspace_size(rows, cols, ctypes.byref(n)) == 0
    ws = torch.empty(int(n.value), dtype=torch.uint8, device=device)
    dz = torch.full_like(z, float("nan"))
    db = torch.full((cols,), float("nan"), device=device)
    assert lib.esa_mish_bwd_colsum(z.data_ptr(), g.data_ptr(), rows, cols, code, dz.data_ptr(), db.data_ptr(),
                                   ws.data_ptr(), ws.numel(), st) == 0
    assert torch.equal(_bits(dz), _bits(dz_ref))
    if rows:
        assert torch.equal(db, column_sum(dz_ref))
    else:
        assert torch.equal(db, torch.zeros_like(db))
    assert lib.esa_mish_bwd_colsum(z.data_ptr(), g.data_ptr(), rows, 6, code, dz.data_ptr(), db.data_ptr(),
                                   ws.data_ptr(), ws.numel(), st) == -2   # ESA_ERR_SHAPE


@pytest.mark.parametrize("dout", [512, 2048], ids=["two_kernels", "fused_colsum"])
@pytest.mark.parametrize("autocast", [False, True], ids=["fp32", "autocast_bf16"])
def test_linear_mish_fused(device, autocast, dout):
    """linear_mish(x, fc) = mish(fc(x)) (an MLP's Linear -> Mish) against fp64 autograd on the operands the GEMM
    gets (bf16-rounded under autocast): output and the gradients of x, weight and bias, which reach the fp32
    parameters; both backward forms (the fused Mish + bias-gradient kernel from 1024 outputs, the two kernels
    below); SmallMLP takes this path."""
    from mind_amd.esa.activations import linear_mish
    from mind_amd.esa.mlp_utils import SmallMLP
    gen = torch.Generator().manual_seed(31 + autocast + dout)
    t, din = 3000, 256
    fc = torch.nn.Linear(din, dout).to(device)
    x = torch.randn(t, din, generator=gen)
    up = torch.randn(t, dout, generator=gen)
    xd = x.to(device).requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        y = linear_mish(xd, fc)
    assert y.dtype == (torch.bfloat16 if autocast else torch.float32)
    y.backward(up.to(device).to(y.dtype))
    assert fc.weight.grad.dtype == torch.float32 and fc.bias.grad.dtype == torch.float32
    rnd = (lambda v: v.to(torch.bfloat16).double()) if autocast else (lambda v: v.double())
    w64 = rnd(fc.weight.detach().cpu()).requires_grad_(True)
    b64 = rnd(fc.bias.detach().cpu()).requires_grad_(True)
    x64 = rnd(x).requires_grad_(True)
    ref = OMod.mish(x64 @ w64.t() + b64)
    ref.backward(up.to(y.dtype).double())
    if autocast:
        _bf16_bar(y, ref.detach(), "y")
        _bf16_bar(xd.grad, x64.grad, "d x")
        _bf16_bar(fc.weight.grad, w64.grad, "d weight")
        _bf16_bar(fc.bias.grad, b64.grad, "d bias")
    else:   # the fp32 bar, norm-wise
        for got, r, what in ((y, ref.detach(), "y"), (xd.grad, x64.grad, "d x"), (fc.weight.grad, w64.grad, "dw"),
                             (fc.bias.grad, b64.grad, "db")):
            _f32_norm_close(got, r, what)
    # SmallMLP (Linear -> Mish -> Linear) routes its first pair through linear_mish: same values as the module
    mlp = SmallMLP(din, dout, din, num_layers=2).to(device)
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        got = mlp(xd.detach())
        ref_mlp = mlp.mlp[2](linear_mish(xd.detach(), mlp.mlp[0]))
    assert torch.equal(got, ref_mlp)


def _bf16_bar(got, ref, what):
    """The north-star bf16 bar, scaled by the reference's magnitude (at least 1)."""
    from tests._util import assert_bf16_close, grad_scale
    assert_bf16_close(got.detach().float().cpu(), ref, grad_scale(ref), what)


@pytest.mark.parametrize("with_residual", [False, True])
def test_mab_epilogue_fused(device, with_residual):
    """mab_epilogue(o, fc_o, x) = x + (o + mish(fc_o(o))) under autocast(bf16) against the fp64 expression on the
    same bf16-rounded operands; gradients of o, x, fc_o.weight and fc_o.bias by fp64 autograd."""
    from mind_amd.esa.activations import mab_epilogue
    gen = torch.Generator().manual_seed(21 + with_residual)
    t, d = 3000, 256
    fc = torch.nn.Linear(d, d).to(device)
    o = torch.randn(t, d, generator=gen).to(torch.bfloat16)
    x = torch.randn(t, d, generator=gen) if with_residual else None
    up = torch.randn(t, d, generator=gen)
    od = o.to(device).requires_grad_(True)
    xd = x.to(device).requires_grad_(True) if with_residual else None
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = mab_epilogue(od, fc, xd)
    assert y.dtype == (torch.float32 if with_residual else torch.bfloat16)
    y.backward(up.to(device).to(y.dtype))
    # fp64 reference on the operands autocast hands the GEMM (bf16 weight and bias)
    w64 = fc.weight.detach().to(torch.bfloat16).double().cpu().requires_grad_(True)
    b64 = fc.bias.detach().to(torch.bfloat16).double().cpu().requires_grad_(True)
    o64 = o.double().requires_grad_(True)
    ref = o64 + OMod.mish(o64 @ w64.t() + b64)
    if with_residual:
        x64 = x.double().requires_grad_(True)
        ref = x64 + ref
    g64 = up.to(y.dtype).double()
    ref.backward(g64)
    _bf16_bar(y, ref.detach(), "y")
    _bf16_bar(od.grad, o64.grad, "d o")
    _bf16_bar(fc.weight.grad, w64.grad, "d weight")
    _bf16_bar(fc.bias.grad, b64.grad, "d bias")
    if with_residual:
        assert torch.equal(xd.grad.cpu(), up)


@pytest.mark.parametrize("self_attn", [True, False])
def test_qkv_projection(device, self_attn):
    """qkv_projection: outputs are F.linear's (bit for bit); input and parameter gradients, with the shared
    input's gradient accumulated inside the GEMMs, against fp64 autograd."""
    from mind_amd.esa.linear import qkv_projection
    gen = torch.Generator().manual_seed(31 + self_attn)
    tq, tk, d = 2048 if self_attn else 64, 2048, 128
    fcs = [torch.nn.Linear(d, d).to(device) for _ in range(3)]
    xq = torch.randn(tq, d, generator=gen)
    xk = xq if self_attn else torch.randn(tk, d, generator=gen)
    gs = [torch.randn(tq, d, generator=gen), torch.randn(tk, d, generator=gen), torch.randn(tk, d, generator=gen)]
    xqd = xq.to(device).requires_grad_(True)
    xkd = xqd if self_attn else xk.to(device).requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        outs = qkv_projection(fcs[0], fcs[1], fcs[2], xqd, xkd)
        refs = [fcs[0](xqd), fcs[1](xkd), fcs[2](xkd)]
    for a, b in zip(outs, refs):
        assert a.dtype == torch.bfloat16 and torch.equal(a, b)
    torch.autograd.backward(list(outs), [g.to(device).to(torch.bfloat16) for g in gs])
    ws = [f.weight.detach().to(torch.bfloat16).double().cpu().requires_grad_(True) for f in fcs]
    bs = [f.bias.detach().to(torch.bfloat16).double().cpu().requires_grad_(True) for f in fcs]
    xq64 = xq.to(torch.bfloat16).double().requires_grad_(True)
    xk64 = xq64 if self_attn else xk.to(torch.bfloat16).double().requires_grad_(True)
    r = [xq64 @ ws[0].t() + bs[0], xk64 @ ws[1].t() + bs[1], xk64 @ ws[2].t() + bs[2]]
    torch.autograd.backward(r, [g.to(torch.bfloat16).double() for g in gs])
    _bf16_bar(xqd.grad, xq64.grad, "d xq")
    if not self_attn:
        _bf16_bar(xkd.grad, xk64.grad, "d xk")
    for f, w, b in zip(fcs, ws, bs):
        _bf16_bar(f.weight.grad, w.grad, "d weight")
        _bf16_bar(f.bias.grad, b.grad, "d bias")
