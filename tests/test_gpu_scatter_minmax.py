"""GPU parity of scatter_min / scatter_max (torch_scatter's semantics on the deterministic CSR), bit-exact:
values (as raw bits) and args against the oracle, which is pinned to torch_scatter's sequential CPU update,
torch's scatter_reduce and the documented example (tests/test_oracle_scatter_minmax.py)."""
import numpy as np
import pytest
import torch

from mind_amd import edges
from oracle import edges as OE

pytestmark = pytest.mark.gpu

_NAME = {torch.float32: "float32", torch.bfloat16: "bfloat16"}


def _bits(x: torch.Tensor) -> np.ndarray:
    return x.float().cpu().numpy().view(np.uint32)


def _check(device, src, index, n, maximum):
    """Library vs oracle on the same src (src already in its dtype) and index; returns the library's outputs."""
    fn = edges.scatter_max if maximum else edges.scatter_min
    out, arg = fn(src.to(device), index.to(device), dim=0, dim_size=n)
    assert out.dtype == src.dtype and arg.dtype == torch.int64
    assert out.shape == (n,) + tuple(src.shape[1:]) and arg.shape == out.shape
    ref_out, ref_arg = OE.scatter_minmax(src.float().numpy(), index.numpy(), n, maximum, _NAME[src.dtype])
    assert np.array_equal(arg.cpu().numpy().reshape(ref_arg.shape), ref_arg)
    assert np.array_equal(_bits(out).reshape(ref_out.shape), ref_out.view(np.uint32))
    return out, arg


@pytest.mark.parametrize("maximum", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(), (3,), (2, 4)])
def test_special_values_ties_empty_and_dropped(device, dtype, maximum, shape):
    """Small-integer values (many ties) with NaN, +-inf, the dtype's largest finite value and -0 mixed in,
    nodes without edges and indices outside [0, N) (dropped)."""
    rng = np.random.default_rng(len(shape) * 7 + int(maximum))
    e, n = 5000, 900
    y = rng.integers(-6, 7, size=(e,) + shape).astype(np.float32)
    u = rng.random(y.shape)
    big = np.float32(np.uint32(0x7F7F0000).view(np.float32)) if dtype == torch.bfloat16 else np.finfo(np.float32).max
    y[u < 0.03] = np.nan
    y[(u >= 0.03) & (u < 0.05)] = np.inf
    y[(u >= 0.05) & (u < 0.07)] = -np.inf
    y[(u >= 0.07) & (u < 0.09)] = big
    y[(u >= 0.09) & (u < 0.11)] = -big
    y[(u >= 0.11) & (u < 0.14)] = -0.0
    index = torch.as_tensor(rng.integers(-2, n + 2, size=e))
    _check(device, torch.as_tensor(y).to(dtype), index, n, maximum)


@pytest.mark.parametrize("maximum", [False, True])
def test_encoder_shape_closest_neighbour(device, maximum):
    """The encoder's call (core/molecular_encoder.py:214): close-range distances in (0.5, 3) of ~2M edges
    to 65,536 nodes, fp32, edges in random order; plus repeatability and torch's scatter_reduce."""
    rng = np.random.default_rng(11)
    n, e = 65536, 2_000_000
    dist = torch.as_tensor(rng.uniform(0.5, 3.0, size=e).astype(np.float32))
    index = torch.as_tensor(rng.integers(0, n, size=e))
    out, arg = _check(device, dist, index, n, maximum)
    again, again_arg = (edges.scatter_max if maximum else edges.scatter_min)(dist.to(device), index.to(device),
                                                                            dim=0, dim_size=n)
    assert torch.equal(out, again) and torch.equal(arg, again_arg)
    red = torch.zeros(n, device=device).scatter_reduce(0, index.to(device), dist.to(device),
                                                         "amax" if maximum else "amin", include_self=False)
    assert torch.equal(out, red)


def test_gradient_goes_to_the_attaining_edge(device):
    """d out[n] / d src[e] = 1 for e = argmin[n], else 0 (torch_scatter's backward); nodes without edges
    pass nothing."""
    rng = np.random.default_rng(5)
    e, n = 3000, 400
    y = torch.as_tensor(rng.integers(-20, 20, size=(e, 2)).astype(np.float32))
    index = torch.as_tensor(rng.integers(0, n + 50, size=e))   # some nodes >= n: dropped
    src = y.to(device).requires_grad_(True)
    out, arg = edges.scatter_min(src, index.to(device), dim_size=n + 10)   # 10 more nodes: empty
    up = torch.randn(out.shape, generator=torch.Generator().manual_seed(1))
    out.backward(up.to(device))
    _, ref_arg = OE.scatter_minmax(y.numpy(), index.numpy(), n + 10)
    gref = np.zeros((e + 1, 2), np.float32)
    for node in range(n + 10):
        for c in range(2):
            gref[ref_arg[node, c], c] += up[node, c].item()
    assert np.array_equal(src.grad.cpu().numpy(), gref[:e])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_csr_reuse_and_no_edges(device, dtype):
    """A CSR built once serves several reductions; zero edges give zeros with arg = 0 (= src.size(0))."""
    rng = np.random.default_rng(9)
    e, n = 1000, 64
    index = torch.as_tensor(rng.integers(0, n, size=e)).to(device)
    csr = edges.CSR.build(index, n)
    a = torch.as_tensor(rng.standard_normal(e).astype(np.float32)).to(dtype).to(device)
    lo, lo_arg = edges.scatter_min(a, index, dim_size=n, csr=csr)
    hi, hi_arg = edges.scatter_max(a, index, dim_size=n, csr=csr)
    assert bool((lo <= hi).all())
    assert torch.equal(a[lo_arg], lo) and torch.equal(a[hi_arg], hi)
    empty = torch.zeros(0, dtype=dtype, device=device)
    out, arg = edges.scatter_min(empty, torch.zeros(0, dtype=torch.int64, device=device), dim_size=5)
    assert torch.equal(out.cpu(), torch.zeros(5, dtype=dtype)) and torch.equal(arg.cpu(), torch.zeros(5, dtype=torch.int64))
