"""GPU parity of the fp32 attention kernels against the fp64 oracle.

fp32 inputs (the reference's fp32 modules, configuration 0).  Bar: 1e-5
relative, taken norm-wise per tensor: max|got - ref| <= 1e-5 * max(1, max|ref|)
for outputs and each gradient, and the same for the log-sum-exp.
"""
import numpy as np
import pytest
import torch

from mind_amd import generators
from mind_amd.esa import attention as A
from oracle import attention as OA
from tests._util import cu_from_lengths, err, seeded_normal

pytestmark = pytest.mark.gpu

H, D = 8, 16
REL = 1e-5


def _close(got, ref, what):
    mx, _ = err(got, ref)
    bar = REL * max(1.0, float(ref.abs().max()) if ref.numel() else 0.0)
    assert mx <= bar, f"{what}: max-abs {mx:.3e} > {bar:.3e}"


def _inputs(tq, tk, seed, heads=H, hd=D):
    f = torch.float32
    return (seeded_normal((tq, heads, hd), seed, f), seeded_normal((tk, heads, hd), seed + 1, f),
            seeded_normal((tk, heads, hd), seed + 2, f), seeded_normal((tq, heads, hd), seed + 3, f))


def _check(device, lengths_q, lengths_k, seed, src=None, dst=None, heads=H, scale=0.25, hd=D, max_q=None):
    """max_q: the max_seqlen_q passed to the call (default: the true maximum); it only selects the route."""
    cu_q, cu_k = cu_from_lengths(lengths_q), cu_from_lengths(lengths_k)
    q, k, v, g = _inputs(int(cu_q[-1]), int(cu_k[-1]), seed, heads, hd)
    qd, kd, vd = (t.to(device).requires_grad_(True) for t in (q, k, v))
    cq, ck = torch.as_tensor(cu_q).to(device), torch.as_tensor(cu_k).to(device)
    s = None if src is None else torch.as_tensor(src, dtype=torch.int32).to(device)
    d = None if dst is None else torch.as_tensor(dst, dtype=torch.int32).to(device)
    mq = (int(np.diff(cu_q).max()) if len(cu_q) > 1 else 0) if max_q is None else max_q
    mk = int(np.diff(cu_k).max()) if len(cu_k) > 1 else 0
    out, lse = A.varlen_attention(qd, kd, vd, cq, ck, mq, mk, softmax_scale=scale, edge_src=s, edge_dst=d,
                                  return_lse=True)
    assert out.dtype == torch.float32
    out.backward(g.to(device))
    torch.cuda.synchronize()
    ref, lse_ref = OA.varlen_attention(q, k, v, cu_q, cu_k, scale, src, dst)
    _close(out.detach().cpu(), ref, "out")
    lse = lse.cpu().double()
    fin = torch.isfinite(lse_ref)
    assert torch.equal(torch.isfinite(lse), fin), "lse -inf pattern differs"
    if fin.any():
        _close(lse[fin], lse_ref[fin], "lse")
    rdq, rdk, rdv = OA.varlen_attention_bwd(g, q, k, v, cu_q, cu_k, scale, src, dst)
    _close(qd.grad.cpu(), rdq, "dq")
    _close(kd.grad.cpu(), rdk, "dk")
    _close(vd.grad.cpu(), rdv, "dv")


@pytest.mark.parametrize("lengths", [[1], [5, 0, 7], [31, 32, 33], [1, 2, 3, 64, 65, 100, 0, 17], [300]])
def test_f32_dense_ragged(device, lengths):
    _check(device, lengths, lengths, seed=sum(lengths) + 1000)


@pytest.mark.parametrize("seeds", [1, 4])
@pytest.mark.parametrize("lk", [[50, 1, 130, 77], [0, 9, 0, 260, 3], list(range(1, 41))])
def test_f32_cross_attention_pma_shape(device, seeds, lk):
    """PMA: k seeds per graph over the graph's tokens; graphs without tokens give zero rows; many short
    segments (each segment's queries form their own group)."""
    _check(device, [seeds] * len(lk), lk, seed=seeds + 1100 + len(lk))


@pytest.mark.parametrize("hd", [16, 24, 32, 64])
@pytest.mark.parametrize("seeds", [1, 3])
def test_f32_few_query_route_head_dims(device, hd, seeds):
    """Segments of at most four queries (max_seqlen_q <= 4: the PMA's expanded call) take the one-wave-per-query
    forward: long, empty and one-token key sets, every head dim; the backward is the tiled one."""
    _check(device, [seeds] * 5, [800, 0, 1, 63, 257], seed=1150 + hd + seeds, heads=128 // hd if hd != 24 else 8,
           hd=hd)


@pytest.mark.parametrize("hint", [1, 2])
def test_f32_few_query_hint_below_the_true_maximum(device, hint):
    """max_seqlen_q only chooses the route: with a hint below the true maximum (segments of up to 9 queries),
    the few-query forward walks the extra queries and the results still match the oracle."""
    _check(device, [9, 1, 0, 4, 7], [40, 3, 5, 130, 64], seed=1170 + hint, max_q=hint)


@pytest.mark.parametrize("hd", [16, 64])
def test_f32_few_query_dropout_matches_tiled(device, hd):
    """With dropout the few-query forward applies the keep mask of the tiled forward: both routes on one seed
    agree to the fp32 bar (outputs and log-sum-exp)."""
    heads = 128 // hd
    cu = torch.as_tensor(cu_from_lengths([2] * 6)).to(device)
    ck = torch.as_tensor(cu_from_lengths([300, 1, 0, 77, 128, 64])).to(device)
    q, k, v, _ = (t.to(device) for t in _inputs(12, int(ck[-1]), 1190 + hd, heads, hd))
    few = A.attn_fwd(q, k, v, cu, ck, 2, 300, 0.25, dropout_p=0.1, dropout_seed=77)
    tiled = A.attn_fwd(q, k, v, cu, ck, 0, 300, 0.25, dropout_p=0.1, dropout_seed=77)
    for a, b, what in zip(few, tiled, ("out", "lse")):
        a, b = a.cpu(), b.cpu()
        fin = torch.isfinite(b)
        assert torch.equal(torch.isfinite(a), fin), what
        _close(a[fin].double(), b[fin].double(), what)


def test_f32_masked_small_molecules(device):
    """Configuration 0's shape of batch: radius-5 small molecules, edge mask."""
    gb, _ = generators.small_molecules(seed=3, num_graphs=8)
    src, dst = gb.edge_index[0].astype(np.int32), gb.edge_index[1].astype(np.int32)
    _check(device, gb.edge_counts, gb.edge_counts, seed=1200, src=src, dst=dst)


def test_f32_masked_isolated_rows_give_zero(device):
    src = np.array([0, 2, 4], np.int32)
    dst = np.array([1, 3, 5], np.int32)
    _check(device, [3], [3], seed=1300, src=src, dst=dst)


def test_f32_dense_protein_like(device):
    gb = generators.protein_like(seed=5, num_graphs=3, n_min=40, n_max=100)
    _check(device, gb.edge_counts, gb.edge_counts, seed=1400)


def test_f32_backward_is_deterministic(device):
    cu = cu_from_lengths([70, 33, 128])
    q, k, v, g = _inputs(int(cu[-1]), int(cu[-1]), 1500)
    cq = torch.as_tensor(cu).to(device)
    runs = []
    for _ in range(2):
        qd, kd, vd = (t.to(device).requires_grad_(True) for t in (q, k, v))
        A.varlen_attention(qd, kd, vd, cq, cq, 128, 128).backward(g.to(device))
        runs.append((qd.grad.cpu(), kd.grad.cpu(), vd.grad.cpu()))
    for a, b in zip(*runs):
        assert torch.equal(a, b)


def test_mixed_dtypes_rejected(device):
    q = torch.zeros(4, 2, 16, device=device)
    k = torch.zeros(4, 2, 16, device=device, dtype=torch.bfloat16)
    cu = torch.tensor([0, 4], dtype=torch.int32, device=device)
    with pytest.raises(TypeError):
        A.attn_fwd(q, k, k, cu, cu, 4, 4, 0.25)
