"""GPU parity of the fp32 few-query attention kernels (attn_fwd_few_kernel, attn_dq_few_kernel,
attn_dkdv_few_kernel): unmasked fp32 calls whose max_seqlen_q is 1-4, the shape of the PMA's expanded call (k
seeds per set over the set's tokens), forward and backward, against the fp64 oracle; the same calls in bf16 (which
keep the MFMA kernels) against the same oracle.

Bars: bf16 max-abs 2e-2 and mean-abs 2e-3 (gradients scaled by max(1, max |reference|)); fp32 1e-5 relative.
max_seqlen_q only selects the route: a hint below the true maximum is still computed exactly (the kernels walk
every query of a segment).  Head dim 64 runs the few-query forward and the dense backward.
"""
import numpy as np
import pytest
import torch

from mind_amd.esa import attention as A
from oracle import attention as OA
from tests._util import assert_bf16_close, assert_f32_close, cu_from_lengths, grad_scale, seeded_normal

pytestmark = pytest.mark.gpu


def _check(device, dtype, lq, lk, hd, seed, hint=None, dropout=None):
    heads = 128 // hd if hd != 24 else 8
    cu_q, cu_k = cu_from_lengths(lq), cu_from_lengths(lk)
    tq, tk = int(cu_q[-1]), int(cu_k[-1])
    q = seeded_normal((tq, heads, hd), seed, dtype)
    k = seeded_normal((tk, heads, hd), seed + 1, dtype)
    v = seeded_normal((tk, heads, hd), seed + 2, dtype)
    g = seeded_normal((tq, heads, hd), seed + 3, dtype)
    scale = hd ** -0.5
    qd, kd, vd = (t.to(device).requires_grad_(True) for t in (q, k, v))
    cq, ck = torch.as_tensor(cu_q).to(device), torch.as_tensor(cu_k).to(device)
    mq = int(np.diff(cu_q).max()) if hint is None else hint
    kw = {} if dropout is None else {"dropout_p": dropout[0], "dropout_seed": dropout[1]}
    out, lse = A.varlen_attention(qd, kd, vd, cq, ck, mq, max(lk), softmax_scale=scale, return_lse=True, **kw)
    out.backward(g.to(device))
    torch.cuda.synchronize()
    ref, lse_ref = OA.varlen_attention(q, k, v, cu_q, cu_k, scale, dropout=dropout)
    rdq, rdk, rdv = OA.varlen_attention_bwd(g, q, k, v, cu_q, cu_k, scale, dropout=dropout)
    lse = lse.cpu().double()
    fin = torch.isfinite(lse_ref)
    assert torch.equal(torch.isfinite(lse), fin), "lse -inf pattern"
    pairs = [("out", out.detach(), ref), ("dq", qd.grad, rdq), ("dk", kd.grad, rdk), ("dv", vd.grad, rdv)]
    if dtype == torch.float32:
        for what, got, r in pairs:
            assert_f32_close(got.cpu(), r, what)
        assert_f32_close(lse[fin], lse_ref[fin], "lse")
    else:
        for what, got, r in pairs:
            assert_bf16_close(got.float().cpu(), r, 1.0 if what == "out" else grad_scale(r), what)
        assert float((lse[fin] - lse_ref[fin]).abs().max()) <= 1e-3 * max(1.0, float(lse_ref[fin].abs().max()))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hd", [16, 24, 32, 64])
@pytest.mark.parametrize("seeds", [1, 4])
def test_few_query_segments(device, dtype, hd, seeds):
    """k seeds per set over sets of 800, 0, 1, 63 and 257 keys (a set without keys gives zero rows and -inf
    LSE, and zero key gradients nowhere: every key belongs to a set with queries)."""
    _check(device, dtype, [seeds] * 5, [800, 0, 1, 63, 257], hd, seed=1300 + hd + seeds)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hint", [1, 3])
def test_hint_below_the_true_maximum(device, dtype, hint):
    """Segments of up to 9 queries called with max_seqlen_q = 1 or 3: forward, dQ and dK/dV still cover every
    query (a set with keys but no queries gets zero key gradients)."""
    _check(device, dtype, [9, 1, 0, 4, 7], [40, 3, 5, 130, 64], 16, seed=1350 + hint, hint=hint)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hd", [16, 24])
def test_few_query_dropout(device, dtype, hd):
    """Attention dropout on the few-query route against the oracle's keep mask (p = 0.3)."""
    _check(device, dtype, [4, 4, 4, 4], [37, 130, 1, 64], hd, seed=1370 + hd, dropout=(0.3, 77))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_pma_module_shape(device, dtype):
    """configuration 4's PMA shape at a smaller scale: 4 seeds, 32 heads of 16, 40 sets of 30-300 tokens."""
    rng = np.random.default_rng(3)
    lk = [int(x) for x in rng.integers(30, 300, size=40)]
    _check(device, dtype, [4] * len(lk), lk, 16, seed=1390)
