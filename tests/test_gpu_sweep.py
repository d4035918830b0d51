"""Seeded random sweep of the bf16 attention kernels against the fp64 oracle.

Each case draws a batch the hand-written cases do not cover together: ragged segments mixing empty, one-token,
tile-edge (31/32/33, 255/257) and random lengths; cross-attention with query and key segments of different
lengths (empty ones included); head counts of every block mapping of the dense kernels (1, 3, 4, 8, 16, 32);
and, for the edge mask, random per-token endpoint node ids (repeated edges and self-loop tokens included)
with one shared or two equal cu_seqlens arrays.  Forward output and all three gradients are checked at the
bf16 bar, gradients scaled by their own magnitude.
"""
import numpy as np
import pytest
import torch

from mind_amd.esa import attention as A
from oracle import attention as OA
from tests._util import assert_bf16_close, cu_from_lengths, grad_scale, seeded_normal

pytestmark = pytest.mark.gpu

D = 16
EDGE_LENGTHS = [0, 1, 2, 31, 32, 33, 64, 95, 128, 129, 255, 257]


def _lengths(rng: np.random.Generator, n: int) -> list[int]:
    out = [int(rng.choice(EDGE_LENGTHS)) if rng.random() < 0.5 else int(rng.integers(1, 300)) for _ in range(n)]
    if sum(out) == 0:
        out[0] = 7
    return out


def _run(device, q, k, v, g, cu_q, cu_k, src=None, dst=None, shared_cu=False):
    qd, kd, vd = (t.to(device).requires_grad_(True) for t in (q, k, v))
    cq = torch.as_tensor(cu_q, dtype=torch.int32).to(device)
    ck = cq if shared_cu else torch.as_tensor(cu_k, dtype=torch.int32).to(device)
    s = None if src is None else torch.as_tensor(src, dtype=torch.int32).to(device)
    d = None if dst is None else torch.as_tensor(dst, dtype=torch.int32).to(device)
    mq, mk = int(np.diff(cu_q).max()), int(np.diff(cu_k).max())
    out = A.varlen_attention(qd, kd, vd, cq, ck, mq, mk, softmax_scale=0.25, edge_src=s, edge_dst=d)
    out.backward(g.to(device))
    torch.cuda.synchronize()
    return out.detach().cpu(), qd.grad.cpu(), kd.grad.cpu(), vd.grad.cpu()


def _check(got, q, k, v, g, cu_q, cu_k, src=None, dst=None, what=""):
    out, dq, dk, dv = got
    ref, _ = OA.varlen_attention(q, k, v, cu_q, cu_k, 0.25, src, dst)
    assert_bf16_close(out, ref, what=f"{what} out")
    rdq, rdk, rdv = OA.varlen_attention_bwd(g, q, k, v, cu_q, cu_k, 0.25, src, dst)
    assert_bf16_close(dq, rdq, grad_scale(rdq), f"{what} dq")
    assert_bf16_close(dk, rdk, grad_scale(rdk), f"{what} dk")
    assert_bf16_close(dv, rdv, grad_scale(rdv), f"{what} dv")


@pytest.mark.parametrize("case", range(16))
def test_dense_sweep(device, case):
    rng = np.random.default_rng(7100 + case)
    nseg = int(rng.integers(1, 7))
    heads = [1, 3, 4, 8, 16, 32][case % 6]   # every block mapping of the dense kernels
    lq = _lengths(rng, nseg)
    cross = rng.random() < 0.4
    lk = _lengths(rng, nseg) if cross else lq
    cu_q, cu_k = cu_from_lengths(lq), cu_from_lengths(lk)
    tq, tk = int(cu_q[-1]), int(cu_k[-1])
    seed = 7200 + 10 * case
    q, k, v = (seeded_normal((t, heads, D), seed + i) for i, t in enumerate((tq, tk, tk)))
    g = seeded_normal((tq, heads, D), seed + 3)
    got = _run(device, q, k, v, g, cu_q, cu_k, shared_cu=not cross and rng.random() < 0.5)
    _check(got, q, k, v, g, cu_q, cu_k, what=f"case {case} (heads {heads}, q {lq}, k {lk})")


@pytest.mark.parametrize("case", range(10))
def test_edge_mask_sweep(device, case):
    rng = np.random.default_rng(7300 + case)
    nseg = int(rng.integers(1, 6))
    heads = [1, 2, 5, 8, 16][case % 5]
    lens = _lengths(rng, nseg)
    cu = cu_from_lengths(lens)
    t = int(cu[-1])
    # per-token endpoint node ids inside each segment's own node range: few nodes per segment give many
    # shared endpoints, repeated (src, dst) pairs and, with src == dst, self-loop tokens
    src = np.empty(t, np.int32)
    dst = np.empty(t, np.int32)
    base = 0
    for b, n_tok in enumerate(lens):
        n_nodes = max(1, int(rng.integers(1, max(2, n_tok // 2 + 2))))
        s, e = int(cu[b]), int(cu[b + 1])
        src[s:e] = base + rng.integers(0, n_nodes, size=n_tok)
        dst[s:e] = base + rng.integers(0, n_nodes, size=n_tok)
        base += n_nodes
    seed = 7400 + 10 * case
    q, k, v, g = (seeded_normal((t, heads, D), seed + i) for i in range(4))
    got = _run(device, q, k, v, g, cu, cu, src, dst, shared_cu=bool(case % 2))
    _check(got, q, k, v, g, cu, cu, src, dst, what=f"case {case} (heads {heads}, lengths {lens})")
