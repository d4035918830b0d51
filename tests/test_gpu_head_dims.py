"""GPU parity at head dims 24, 32 and 64 (ESA's dim / num_heads in MIND's YAMLs: 512 / 8 = 64 in qm9, unimol and
lba, 512 / 16 = 32 in coconut, 192 / 8 = 24 in rna; esa/mha.py:50-52 computes head_dim for any size).

Every path that takes a head dim: node-mode attention (the gather kernels over a CSR), the edge mask (the gather
kernels over the edge-mask plan's lists, including tiles past the list capacity), fp32 attention (the tiled fp32
kernels), dense bf16 attention (the MFMA kernels for wide heads), PMA seed pooling and the modules.  Inputs are
seeded; the oracle runs in fp64 on the same values.  Bars: bf16 max-abs 2e-2 / mean-abs 2e-3 (gradients scaled by
max(1, max|ref|)); fp32 1e-5 relative.  Softmax scale 1 / sqrt(head_dim), the modules' default.
"""
import math

import numpy as np
import pytest
import torch

from mind_amd import generators
from mind_amd.esa import attention as A
from mind_amd.esa.packing import NodeAdjacency
from oracle import attention as OA
from tests._util import assert_bf16_close, assert_f32_close, cu_from_lengths, grad_scale, node_graph, seeded_normal

pytestmark = pytest.mark.gpu


def _inputs(tq, tk, heads, hd, seed, dtype):
    return (seeded_normal((tq, heads, hd), seed, dtype), seeded_normal((tk, heads, hd), seed + 1, dtype),
            seeded_normal((tk, heads, hd), seed + 2, dtype), seeded_normal((tq, heads, hd), seed + 3, dtype))


def _close(got, ref, dtype, what, grad=False):
    if dtype == torch.float32:
        assert_f32_close(got, ref, what)
    else:
        assert_bf16_close(got, ref, grad_scale(ref) if grad else 1.0, what)


def _run_and_check(device, q, k, v, g, cu_q, cu_k, dtype, kernel_kw, oracle_kw, shared_cu=False, check_lse=True):
    hd = q.shape[-1]
    scale = 1.0 / math.sqrt(hd)
    qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
    cq = torch.as_tensor(cu_q, dtype=torch.int32).to(device)
    ck = cq if shared_cu else torch.as_tensor(cu_k, dtype=torch.int32).to(device)
    mq = int(np.diff(cu_q).max()) if len(cu_q) > 1 else 0
    mk = int(np.diff(cu_k).max()) if len(cu_k) > 1 else 0
    out, lse = A.varlen_attention(qd, kd, vd, cq, ck, mq, mk, softmax_scale=scale, return_lse=True, **kernel_kw)
    out.backward(g.to(device))
    torch.cuda.synchronize()
    ref, lse_ref = OA.varlen_attention(q, k, v, cu_q, cu_k, scale, **oracle_kw)
    rdq, rdk, rdv = OA.varlen_attention_bwd(g, q, k, v, cu_q, cu_k, scale, **oracle_kw)
    _close(out.detach().cpu(), ref, dtype, "out")
    if check_lse:
        fin = torch.isfinite(lse_ref)
        lse = lse.cpu().double()
        assert torch.equal(torch.isfinite(lse), fin), "lse -inf pattern differs"
        if fin.any():
            bar = 1e-5 * max(1.0, float(lse_ref[fin].abs().max())) if dtype == torch.float32 else math.log1p(2 ** -8)
            assert float((lse[fin] - lse_ref[fin]).abs().max()) <= bar, "lse"
    _close(qd.grad.cpu(), rdq, dtype, "dq", grad=True)
    _close(kd.grad.cpu(), rdk, dtype, "dk", grad=True)
    _close(vd.grad.cpu(), rdv, dtype, "dv", grad=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hd,heads", [(24, 8), (24, 3), (32, 8), (32, 3), (64, 8), (64, 5)])
def test_node_mode(device, hd, heads, dtype):
    """Node mode (CSR by query, repeated edges and self-loops, a one-node graph) at head dim 32 / 64, with head
    counts that fill and that do not fill a wave's heads per pass (8 at 32, 4 at 64)."""
    sizes = [60, 1, 45, 80, 17]
    ei, bm = node_graph(40 + hd + heads, sizes)
    na = NodeAdjacency.from_edge_index(torch.as_tensor(ei), torch.as_tensor(bm), len(sizes), max(sizes))
    cu = na.cu_seqlens.numpy()
    t = len(bm)
    print(f"[head-dims] node hd={hd} heads={heads} {dtype} tokens={t}", flush=True)
    q, k, v, g = _inputs(t, t, heads, hd, 7 * hd + heads, dtype)
    _run_and_check(device, q, k, v, g, cu, cu, dtype,
                   {"adj_indptr": na.indptr.to(device), "adj_indices": na.indices.to(device)},
                   {"adj": (na.indptr.numpy(), na.indices.numpy())})


@pytest.mark.parametrize("hd", [24, 32, 64])
def test_node_mode_planned_equals_per_call(device, hd):
    """A node plan built once gives bit-equal outputs and gradients to the per-call transpose at wide heads."""
    sizes = [70, 33, 90]
    ei, bm = node_graph(77 + hd, sizes)
    na = NodeAdjacency.from_edge_index(torch.as_tensor(ei).to(device), torch.as_tensor(bm).to(device), len(sizes),
                                       max(sizes))
    t = len(bm)
    q, k, v, g = (x.to(device) for x in _inputs(t, t, 4, hd, 91 + hd, torch.bfloat16))
    cu = na.cu_seqlens
    res = []
    for kw in ({"adj_indptr": na.indptr, "adj_indices": na.indices},
               {"adj_indptr": na.indptr, "adj_indices": na.indices, "adj_plan": na.plan()}):
        out, lse = A.attn_fwd(q, k, v, cu, cu, 0, 0, 1.0 / math.sqrt(hd), **kw)
        res.append((out, lse) + A.attn_bwd(g, q, k, v, out, lse, cu, cu, 0, 0, 1.0 / math.sqrt(hd), **kw))
    for a, b in zip(*res):
        assert torch.equal(a, b)


def _mixed_star_batch(seed):
    """Protein-like graphs around a 600-token star segment (its tiles are past the key-list capacity)."""
    gb = generators.protein_like(seed=seed, num_graphs=4, n_min=64, n_max=160)
    src_p, dst_p = gb.edge_index[0].astype(np.int32), gb.edge_index[1].astype(np.int32)
    hub = int(max(src_p.max(), dst_p.max())) + 1
    leaves = np.arange(hub + 1, hub + 301, dtype=np.int32)
    star_s = np.concatenate([np.full_like(leaves, hub), leaves])
    star_d = np.concatenate([leaves, np.full_like(leaves, hub)])
    c = gb.edge_counts
    src = np.concatenate([src_p[:c[0] + c[1]], star_s, src_p[c[0] + c[1]:]])
    dst = np.concatenate([dst_p[:c[0] + c[1]], star_d, dst_p[c[0] + c[1]:]])
    return src, dst, [int(c[0]), int(c[1]), star_s.size, int(c[2]), int(c[3])]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hd,heads", [(24, 8), (32, 8), (64, 8), (64, 3)])
@pytest.mark.parametrize("shared_cu", [True, False])
def test_edge_mask(device, hd, heads, dtype, shared_cu):
    """The edge mask at head dim 32 / 64: listed tiles and tiles past the list capacity in one batch, one
    cu_seqlens array (the symmetric plan) and two (the key tiles' own lists)."""
    src, dst, lengths = _mixed_star_batch(12)
    cu = cu_from_lengths(lengths)
    t = int(cu[-1])
    print(f"[head-dims] edge hd={hd} heads={heads} {dtype} shared={shared_cu} tokens={t}", flush=True)
    q, k, v, g = _inputs(t, t, heads, hd, 3 * hd + heads, dtype)
    _run_and_check(device, q, k, v, g, cu, cu, dtype,
                   {"edge_src": torch.as_tensor(src).to(device), "edge_dst": torch.as_tensor(dst).to(device)},
                   {"edge_src": src, "edge_dst": dst}, shared_cu=shared_cu)


@pytest.mark.parametrize("hd", [24, 32, 64])
def test_edge_plan_reuse_wide(device, hd):
    """A plan built once (esa_edge_plan_build) serves wide-head calls as it serves head dim 16: bit-equal to the
    per-call mask."""
    gb = generators.protein_like(seed=15, num_graphs=4, n_min=50, n_max=150)
    src = torch.as_tensor(gb.edge_index[0].astype(np.int32)).to(device)
    dst = torch.as_tensor(gb.edge_index[1].astype(np.int32)).to(device)
    cu = torch.as_tensor(gb.cu_seqlens).to(device)
    t = int(gb.cu_seqlens[-1])
    q, k, v, g = (x.to(device) for x in _inputs(t, t, 8, hd, 50 + hd, torch.bfloat16))
    plan = A.edge_plan(src, dst, cu)
    res = []
    for kw in ({"edge_src": src, "edge_dst": dst}, {"edge_plan": plan}):
        out, lse = A.attn_fwd(q, k, v, cu, cu, 0, 0, 1.0 / math.sqrt(hd), **kw)
        res.append((out, lse) + A.attn_bwd(g, q, k, v, out, lse, cu, cu, 0, 0, 1.0 / math.sqrt(hd), **kw))
    for a, b in zip(*res):
        assert torch.equal(a, b)


@pytest.mark.parametrize("hd", [32, 64])
def test_edge_mask_config2_wide(device, hd):
    """Configuration 2's full batch (65,536-token budget) at head dim `hd` with 256 / hd heads (dim 256): every
    output finite; the first, largest and last graphs against the oracle."""
    gb = generators.protein_budget(seed=0, token_budget=65536)
    cu = gb.cu_seqlens
    t = int(cu[-1])
    heads = 256 // hd
    src, dst = gb.edge_index[0].astype(np.int32), gb.edge_index[1].astype(np.int32)
    q, k, v, g = _inputs(t, t, heads, hd, 4321 + hd, torch.bfloat16)
    scale = 1.0 / math.sqrt(hd)
    qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
    cud = torch.as_tensor(cu).to(device)
    out = A.varlen_attention(qd, kd, vd, cud, cud, gb.max_seqlen, gb.max_seqlen, softmax_scale=scale,
                             edge_src=torch.as_tensor(src).to(device), edge_dst=torch.as_tensor(dst).to(device))
    out.backward(g.to(device))
    torch.cuda.synchronize()
    for x in (out, qd.grad, kd.grad, vd.grad):
        assert torch.isfinite(x.float()).all()
    for b in (0, int(np.argmax(gb.edge_counts)), gb.num_graphs - 1):
        s, e = int(cu[b]), int(cu[b + 1])
        sub = np.array([0, e - s], np.int32)
        ref, _ = OA.varlen_attention(q[s:e], k[s:e], v[s:e], sub, sub, scale, src[s:e], dst[s:e])
        assert_bf16_close(out.detach()[s:e].cpu(), ref, what=f"segment {b}")
        rdq, rdk, rdv = OA.varlen_attention_bwd(g[s:e], q[s:e], k[s:e], v[s:e], sub, sub, scale, src[s:e], dst[s:e])
        assert_bf16_close(qd.grad[s:e].cpu(), rdq, grad_scale(rdq), f"dq segment {b}")
        assert_bf16_close(kd.grad[s:e].cpu(), rdk, grad_scale(rdk), f"dk segment {b}")
        assert_bf16_close(vd.grad[s:e].cpu(), rdv, grad_scale(rdv), f"dv segment {b}")


@pytest.mark.parametrize("hd,heads", [(24, 8), (32, 4), (64, 8), (64, 3)])
@pytest.mark.parametrize("cross", [False, True])
def test_dense_f32(device, hd, heads, cross):
    """fp32 dense attention at wide heads, self-attention and cross-attention (distinct query and key
    segments, one without keys)."""
    lengths_q = [37, 130, 1, 64] if not cross else [5, 9, 3, 1]
    lengths_k = lengths_q if not cross else [100, 0, 47, 200]
    cu_q, cu_k = cu_from_lengths(lengths_q), cu_from_lengths(lengths_k)
    q, k, v, g = _inputs(int(cu_q[-1]), int(cu_k[-1]), heads, hd, 11 * hd + heads, torch.float32)
    _run_and_check(device, q, k, v, g, cu_q, cu_k, torch.float32, {}, {})


@pytest.mark.parametrize("hd,heads", [(24, 8), (24, 5), (32, 8), (32, 3), (64, 8), (64, 5)])
def test_dense_bf16(device, hd, heads):
    """Dense bf16 attention at wide heads (the MFMA kernels): segments of 1, tile-edge (32, 64, 65) and ragged
    lengths, a 300-token one, and an empty segment."""
    lengths = [1, 32, 64, 65, 0, 300, 17]
    cu = cu_from_lengths(lengths)
    t = int(cu[-1])
    print(f"[head-dims] dense bf16 hd={hd} heads={heads} tokens={t}", flush=True)
    q, k, v, g = _inputs(t, t, heads, hd, 5 * hd + heads, torch.bfloat16)
    _run_and_check(device, q, k, v, g, cu, cu, torch.bfloat16, {}, {})


@pytest.mark.parametrize("hd", [24, 32, 64])
def test_dense_bf16_cross(device, hd):
    """Cross-attention: distinct query and key segments, one set without keys (its rows 0, LSE -inf) and one
    without queries."""
    cu_q, cu_k = cu_from_lengths([5, 40, 3, 0, 70]), cu_from_lengths([100, 0, 47, 33, 129])
    q, k, v, g = _inputs(int(cu_q[-1]), int(cu_k[-1]), 4, hd, 17 + hd, torch.bfloat16)
    _run_and_check(device, q, k, v, g, cu_q, cu_k, torch.bfloat16, {}, {})


@pytest.mark.parametrize("hd,heads", [(24, 8), (32, 8), (64, 4)])
def test_dense_bf16_config1_wide(device, hd, heads):
    """Configuration 1's batch (32 protein-like graphs, 43,670 edge tokens) at head dim `hd` (dims 192, 256 and
    256): every output finite; the first, largest and last graphs against the oracle."""
    gb = generators.protein_like(seed=0)
    cu = gb.cu_seqlens
    t = int(cu[-1])
    q, k, v, g = _inputs(t, t, heads, hd, 1234 + hd, torch.bfloat16)
    scale = 1.0 / math.sqrt(hd)
    qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
    cud = torch.as_tensor(cu).to(device)
    out = A.varlen_attention(qd, kd, vd, cud, cud, gb.max_seqlen, gb.max_seqlen, softmax_scale=scale)
    out.backward(g.to(device))
    torch.cuda.synchronize()
    for x in (out, qd.grad, kd.grad, vd.grad):
        assert torch.isfinite(x.float()).all()
    for b in (0, int(np.argmax(gb.edge_counts)), gb.num_graphs - 1):
        s, e = int(cu[b]), int(cu[b + 1])
        sub = np.array([0, e - s], np.int32)
        ref, _ = OA.varlen_attention(q[s:e], k[s:e], v[s:e], sub, sub, scale)
        assert_bf16_close(out.detach()[s:e].cpu(), ref, what=f"segment {b}")
        rdq, rdk, rdv = OA.varlen_attention_bwd(g[s:e], q[s:e], k[s:e], v[s:e], sub, sub, scale)
        assert_bf16_close(qd.grad[s:e].cpu(), rdq, grad_scale(rdq), f"dq segment {b}")
        assert_bf16_close(kd.grad[s:e].cpu(), rdk, grad_scale(rdk), f"dk segment {b}")
        assert_bf16_close(vd.grad[s:e].cpu(), rdv, grad_scale(rdv), f"dv segment {b}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hd", [24, 32, 64])
def test_pma_wide(device, hd, dtype):
    """PMA seed pooling (esa_pma_fwd / _bwd) at wide heads: 4 seeds shared by every set, the seed gradient
    summed over sets, against the oracle on the seeds repeated per set."""
    lengths = [37, 130, 1, 64, 90]
    cu_k = cu_from_lengths(lengths)
    b, k_seeds, heads = len(lengths), 4, 4
    q = seeded_normal((k_seeds, heads, hd), 3 + hd, dtype)
    k = seeded_normal((int(cu_k[-1]), heads, hd), 4 + hd, dtype)
    v = seeded_normal((int(cu_k[-1]), heads, hd), 5 + hd, dtype)
    g = seeded_normal((b * k_seeds, heads, hd), 6 + hd, dtype)
    scale = 1.0 / math.sqrt(hd)
    qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
    out = A.pma_attention(qd, kd, vd, torch.as_tensor(cu_k).to(device), max(lengths), softmax_scale=scale)
    out.backward(g.to(device))
    torch.cuda.synchronize()
    q_rep = q.repeat(b, 1, 1)
    cu_q = cu_from_lengths([k_seeds] * b)
    ref, _ = OA.varlen_attention(q_rep, k, v, cu_q, cu_k, scale)
    rdq, rdk, rdv = OA.varlen_attention_bwd(g, q_rep, k, v, cu_q, cu_k, scale)
    rdq = rdq.view(b, k_seeds, heads, hd).sum(0)
    _close(out.detach().cpu(), ref, dtype, "out")
    _close(qd.grad.cpu(), rdq, dtype, "dseeds", grad=True)
    _close(kd.grad.cpu(), rdk, dtype, "dk", grad=True)
    _close(vd.grad.cpu(), rdv, dtype, "dv", grad=True)


@pytest.mark.parametrize("hd", [24, 32, 64])
def test_dense_bf16_deterministic(device, hd):
    gb = generators.protein_like(seed=4, num_graphs=3, n_min=60, n_max=120)
    cu = torch.as_tensor(gb.cu_seqlens).to(device)
    t = int(gb.cu_seqlens[-1])
    q, k, v, g = (x.to(device) for x in _inputs(t, t, 4, hd, 41, torch.bfloat16))
    res = []
    for _ in range(2):
        out, lse = A.attn_fwd(q, k, v, cu, cu, 0, 0, 1.0 / math.sqrt(hd))
        res.append((out, lse) + A.attn_bwd(g, q, k, v, out, lse, cu, cu, 0, 0, 1.0 / math.sqrt(hd)))
    for a, b in zip(*res):
        assert torch.equal(a, b)
