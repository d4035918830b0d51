"""Pins the CPU oracle against mathematics that fixes each function (no GPU).

The reference ships no golden vectors for this path and cannot be imported
(its xformers / flash_attn / torch_geometric / torch_scatter dependencies are
absent), so each oracle function is checked against an independent route:
a library routine, a brute-force loop, a closed form or an invariant, chosen
so that a dropped term, a wrong sign or index, or a transposed operand fails.
"""
import itertools

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from hypothesis import given, settings
from hypothesis import strategies as st

from mind_amd import generators
from oracle import attention as OA
from oracle import edges as OE
from oracle import mask as OM
from oracle import modules as OMod
from oracle import packing as OP
from tests._util import node_graph


# ---------------------------------------------------------------- mask

def _mask_loop(src, dst):
    """Independent restatement: set intersection of endpoint sets, i != j."""
    e = len(src)
    m = np.zeros((e, e), bool)
    for i in range(e):
        for j in range(e):
            m[i, j] = i != j and bool({src[i], dst[i]} & {src[j], dst[j]})
    return m


@given(st.lists(st.tuples(st.integers(0, 6), st.integers(0, 6)), min_size=1, max_size=14))
@settings(max_examples=60, deadline=None)
def test_edge_adjacency_matches_set_intersection(edges):
    src = np.array([a for a, _ in edges])
    dst = np.array([b for _, b in edges])
    assert np.array_equal(OM.edge_adjacency_global(src, dst), _mask_loop(src, dst))


def test_edge_adjacency_invariants_and_nnz_closed_form():
    for seed in range(3):
        gb, _ = generators.small_molecules(seed=seed, num_graphs=6)
        src, dst = gb.edge_index
        m = OM.edge_adjacency_global(src, dst)
        assert np.array_equal(m, m.T)
        assert not m.diagonal().any()
        gid = np.repeat(np.arange(gb.num_graphs), gb.edge_counts)
        assert not (m & (gid[:, None] != gid[None, :])).any()
        # (u -> v) and (v -> u) always share both endpoints
        pos = {(int(a), int(b)): i for i, (a, b) in enumerate(zip(src, dst))}
        for (a, b), i in pos.items():
            if (b, a) in pos:
                assert m[i, pos[(b, a)]]
        assert int(m.sum()) == OM.edge_mask_nnz(src, dst)


def test_edge_bias_padded_layout():
    gb, _ = generators.small_molecules(seed=4, num_graphs=4)
    gid = np.repeat(np.arange(gb.num_graphs), gb.edge_counts)
    n = int(gb.edge_counts.max()) + 5
    bias = OM.edge_bias_padded(gb.edge_index, gid, gb.num_graphs, n)
    assert bias.shape == (gb.num_graphs, 1, n, n)
    cu = gb.cu_seqlens
    for b in range(gb.num_graphs):
        s, e = int(cu[b]), int(cu[b + 1])
        blk = OM.edge_adjacency_segment(gb.edge_index[0], gb.edge_index[1], s, e)
        got = bias[b, 0].numpy() == 0
        assert np.array_equal(got[: e - s, : e - s], blk)
        assert not got[e - s:, :].any() and not got[:, e - s:].any()
    assert set(np.unique(bias.numpy())) <= {0.0, OM.MASK_FILL}


def test_node_bias_padded_local_ids():
    ei = np.array([[0, 1, 3, 4], [1, 0, 4, 3]])
    bm = np.array([0, 0, 0, 1, 1])
    bias = OM.node_bias_padded(ei, bm, 2, 3)
    assert bias[0, 0, 0, 1] == 0 and bias[0, 0, 1, 0] == 0 and bias[1, 0, 0, 1] == 0 and bias[1, 0, 1, 0] == 0
    assert (bias == 0).sum() == 4


def test_node_adjacency_csr_matches_reference_bias():
    """The CSR blocks equal the zero entries of the restated node-mode bias, and a plain loop over the edges."""
    from mind_amd.esa.packing import NodeAdjacency
    sizes = [7, 1, 12, 5]
    ei, bm = node_graph(3, sizes)
    n = 16
    na = NodeAdjacency.from_edge_index(torch.as_tensor(ei), torch.as_tensor(bm), len(sizes), n)
    indptr, indices = na.indptr.numpy(), na.indices.numpy()
    assert indptr[0] == 0 and indptr[-1] == indices.size == ei.shape[1]
    for i in range(len(bm)):   # rows ascending (a repeated edge appears twice, adjacent)
        row = indices[indptr[i]:indptr[i + 1]]
        assert np.all(np.diff(row) >= 0)
    bias = OM.node_bias_padded(ei, bm, len(sizes), n)
    cu = na.cu_seqlens.numpy()
    for b in range(len(sizes)):
        s, e = int(cu[b]), int(cu[b + 1])
        blk = OM.node_adjacency_segment(indptr, indices, s, e, s, e)
        assert np.array_equal(blk, bias[b, 0, : e - s, : e - s].numpy() == 0)
        loop = np.zeros((e - s, e - s), bool)
        for a_, c_ in ei.T:
            if s <= a_ < e:
                loop[a_ - s, c_ - s] = True
        assert np.array_equal(blk, loop)
    # the padded CSR reproduces the same pattern over [B * N] slots
    ip, ix = (t.numpy() for t in na.padded_csr())
    full = OM.node_adjacency_segment(ip, ix, 0, len(sizes) * n, 0, len(sizes) * n)
    for b in range(len(sizes)):
        blk = full[b * n:(b + 1) * n, b * n:(b + 1) * n]
        assert np.array_equal(blk, bias[b, 0].numpy() == 0)


def test_node_mask_attention_matches_reference_bias():
    """Oracle attention with the CSR mask equals the padded attention with the reference's -99999 node bias on
    every row with at least one out-edge."""
    from mind_amd.esa.packing import NodeAdjacency
    sizes = [6, 9, 4]
    ei, bm = node_graph(5, sizes)
    n, h, d = 12, 2, 16
    na = NodeAdjacency.from_edge_index(torch.as_tensor(ei), torch.as_tensor(bm), len(sizes), n)
    t = len(bm)
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(t, h, d, generator=g, dtype=torch.float64) for _ in range(3))
    cu = na.cu_seqlens.numpy()
    out, lse = OA.varlen_attention(q, k, v, cu, cu, 0.25, adj=(na.indptr.numpy(), na.indices.numpy()))
    pad = lambda x: na.pad(x)   # [B, N, H, D]
    ref = OA.padded_attention(pad(q), pad(k), pad(v), 0.25, OM.node_bias_padded(ei, bm, len(sizes), n,
                                                                                 dtype=torch.float64))
    ref = na.unpad(ref)
    has = torch.as_tensor(np.diff(na.indptr.numpy()) > 0)
    assert torch.allclose(out[has], ref[has], atol=1e-12)
    assert torch.isneginf(lse[:, ~has]).all() and (out[~has] == 0).all()


# ---------------------------------------------------------------- attention

def _sdpa_reference(q, k, v, cu_q, cu_k, scale, mask_fn=None):
    outs = []
    for b in range(len(cu_q) - 1):
        qs, qe, ks, ke = cu_q[b], cu_q[b + 1], cu_k[b], cu_k[b + 1]
        qb, kb, vb = (t.permute(1, 0, 2)[None] for t in (q[qs:qe], k[ks:ke], v[ks:ke]))
        am = None if mask_fn is None else torch.as_tensor(mask_fn(qs, qe))[None, None]
        with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.MATH):
            o = F.scaled_dot_product_attention(qb, kb, vb, attn_mask=am, scale=scale)
        outs.append(o[0].permute(1, 0, 2))
    return torch.cat(outs)


def test_varlen_attention_matches_sdpa():
    g = torch.Generator().manual_seed(0)
    lq, lk = [5, 9, 1, 30], [7, 9, 3, 12]
    cu_q, cu_k = np.cumsum([0] + lq), np.cumsum([0] + lk)
    q = torch.randn(cu_q[-1], 3, 16, generator=g, dtype=torch.float64)
    k = torch.randn(cu_k[-1], 3, 16, generator=g, dtype=torch.float64)
    v = torch.randn(cu_k[-1], 3, 16, generator=g, dtype=torch.float64)
    out, lse = OA.varlen_attention(q, k, v, cu_q, cu_k, 0.25)
    ref = _sdpa_reference(q, k, v, cu_q, cu_k, 0.25)
    assert torch.allclose(out, ref, atol=1e-12, rtol=1e-10)
    # lse closed form for the first segment
    qb, kb = q[0:5].permute(1, 0, 2), k[0:7].permute(1, 0, 2)
    assert torch.allclose(lse[:, 0:5], torch.logsumexp(qb @ kb.transpose(1, 2) * 0.25, -1), atol=1e-12)


def test_varlen_attention_edge_mask_matches_sdpa_bool_mask():
    gb, _ = generators.small_molecules(seed=7, num_graphs=3)
    cu = gb.cu_seqlens
    src, dst = gb.edge_index
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(int(cu[-1]), 2, 16, generator=g, dtype=torch.float64) for _ in range(3))
    out, _ = OA.varlen_attention(q, k, v, cu, cu, 0.25, src, dst)
    ref = _sdpa_reference(q, k, v, cu, cu, 0.25, lambda s, e: OM.edge_adjacency_segment(src, dst, s, e))
    assert torch.allclose(out, ref, atol=1e-12)


def test_attention_special_cases():
    g = torch.Generator().manual_seed(2)
    v = torch.randn(6, 2, 16, generator=g, dtype=torch.float64)
    k = torch.randn(6, 2, 16, generator=g, dtype=torch.float64)
    # L = 1: the output is the single value row
    out, _ = OA.varlen_attention(torch.randn(1, 2, 16, dtype=torch.float64), k[:1], v[:1], [0, 1], [0, 1], 0.25)
    assert torch.allclose(out, v[:1])
    # q = 0: uniform weights, output = mean of v
    out, lse = OA.varlen_attention(torch.zeros(3, 2, 16, dtype=torch.float64), k, v, [0, 3], [0, 6], 0.25)
    assert torch.allclose(out, v.mean(0, keepdim=True).expand(3, 2, 16))
    assert torch.allclose(lse, torch.full_like(lse, np.log(6.0)))
    # a single admissible key: output = that key's value (edges 0 and 1 share node 1, edge 2 is isolated)
    src, dst = np.array([0, 1, 5]), np.array([1, 2, 6])
    out, lse = OA.varlen_attention(torch.randn(3, 2, 16, dtype=torch.float64), k[:3], v[:3], [0, 3], [0, 3], 0.25,
                                   src, dst)
    assert torch.allclose(out[0], v[1]) and torch.allclose(out[1], v[0])
    assert torch.all(out[2] == 0) and torch.isneginf(lse[:, 2]).all()


def test_minus_inf_mask_equals_reference_bias():
    """-inf masking == the reference's -99999 additive bias when a row has an admissible key."""
    gb, _ = generators.small_molecules(seed=9, num_graphs=3)
    gid = np.repeat(np.arange(gb.num_graphs), gb.edge_counts)
    n = int(gb.edge_counts.max())
    bias = OM.edge_bias_padded(gb.edge_index, gid, gb.num_graphs, n, dtype=torch.float64)
    g = torch.Generator().manual_seed(3)
    qp, kp, vp = (torch.randn(gb.num_graphs, n, 2, 16, generator=g, dtype=torch.float64) for _ in range(3))
    padded = OA.padded_attention(qp, kp, vp, 0.25, bias)
    cu = gb.cu_seqlens
    valid = torch.zeros(gb.num_graphs, n, dtype=torch.bool)
    for b, L in enumerate(gb.edge_counts):
        valid[b, :L] = True
    out, _ = OA.varlen_attention(qp[valid], kp[valid], vp[valid], cu, cu, 0.25, *gb.edge_index)
    assert torch.allclose(padded[valid], out, atol=1e-10)


def test_attention_backward_matches_autograd_and_finite_differences():
    g = torch.Generator().manual_seed(4)
    cu = np.array([0, 4, 9])
    src, dst = np.array([0, 1, 2, 1, 4, 5, 6, 5, 4]), np.array([1, 2, 3, 0, 5, 6, 7, 4, 7])
    q, k, v, go = (torch.randn(9, 2, 16, generator=g, dtype=torch.float64) for _ in range(4))
    for es, ed in ((None, None), (src, dst)):
        dq, dk, dv = OA.varlen_attention_bwd(go, q, k, v, cu, cu, 0.25, es, ed)
        qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
        out, _ = OA.varlen_attention(qa, ka, va, cu, cu, 0.25, es, ed)
        (out * go).sum().backward()
        for a, b in ((dq, qa.grad), (dk, ka.grad), (dv, va.grad)):
            assert torch.allclose(a, b, atol=1e-10)
        # central differences on a few coordinates of k
        eps = 1e-6
        for idx in [(0, 0, 3), (5, 1, 7), (8, 0, 15)]:
            kp_, km_ = k.clone(), k.clone()
            kp_[idx] += eps
            km_[idx] -= eps
            fp = (OA.varlen_attention(q, kp_, v, cu, cu, 0.25, es, ed)[0] * go).sum()
            fm = (OA.varlen_attention(q, km_, v, cu, cu, 0.25, es, ed)[0] * go).sum()
            assert abs(float((fp - fm) / (2 * eps)) - float(dk[idx])) < 1e-6


# ---------------------------------------------------------------- gather / CSR / segment sums

def test_gather_concatenates_src_then_dst():
    x = np.arange(12, dtype=np.float32).reshape(6, 2)
    src, dst = np.array([5, 0, 2]), np.array([1, 1, 4])
    out = OE.edge_gather(x, src, dst)
    assert out.tolist() == [[10, 11, 2, 3], [0, 1, 2, 3], [4, 5, 8, 9]]


def test_edge_token_linear_matches_reference_expression():
    # the reference's own torch expression: Linear(torch.cat((x[src], x[dst]), 1))
    rng = np.random.default_rng(3)
    x = rng.standard_normal((9, 5))
    src, dst = rng.integers(0, 9, 40), rng.integers(0, 9, 40)
    lin = torch.nn.Linear(10, 7).double()
    xt = torch.as_tensor(x)
    ref = lin(torch.cat((xt[torch.as_tensor(src)], xt[torch.as_tensor(dst)]), 1)).detach().numpy()
    got = OE.edge_token_linear(x, src, dst, lin.weight.detach().numpy(), lin.bias.detach().numpy())
    assert np.abs(got - ref).max() < 1e-12
    # and the split-weight identity the fused kernel relies on
    w = lin.weight.detach().numpy()
    split = x[src] @ w[:, :5].T + x[dst] @ w[:, 5:].T + lin.bias.detach().numpy()
    assert np.abs(got - split).max() < 1e-12
    # with edge attributes appended (core/pretraining_model.py:157-159): torch.cat((x[src], x[dst], e), 1)
    e = rng.standard_normal((40, 3))
    lin3 = torch.nn.Linear(13, 7).double()
    ref3 = lin3(torch.cat((xt[torch.as_tensor(src)], xt[torch.as_tensor(dst)], torch.as_tensor(e)), 1))
    got3 = OE.edge_token_linear(x, src, dst, lin3.weight.detach().numpy(), lin3.bias.detach().numpy(), e)
    assert np.abs(got3 - ref3.detach().numpy()).max() < 1e-12


@given(st.lists(st.integers(0, 9), min_size=0, max_size=60))
@settings(max_examples=60, deadline=None)
def test_csr_build_loop(keys):
    keys = np.array(keys, dtype=np.int64)
    indptr, perm = OE.csr_build(keys, 10)
    for n in range(10):
        members = [i for i, kk in enumerate(keys) if kk == n]   # ascending edge ids
        assert perm[indptr[n]:indptr[n + 1]].tolist() == members
    assert indptr[-1] == len(keys)


def test_segment_sums():
    rng = np.random.default_rng(0)
    keys = rng.integers(0, 50, size=3000)
    indptr, perm = OE.csr_build(keys, 50)
    const = np.full((3000, 8), 0.25, np.float32)
    s = OE.segment_sum_sequential(const, perm, indptr)
    assert np.array_equal(s, np.repeat((np.bincount(keys, minlength=50) * 0.25)[:, None], 8, 1).astype(np.float32))
    y = rng.normal(size=(3000, 8)).astype(np.float32)
    s32 = OE.segment_sum_sequential(y, perm, indptr)
    s64 = OE.segment_sum_f64(y, keys, 50)
    assert np.allclose(s32, s64, rtol=1e-5, atol=1e-5)
    # explicit left-to-right fp32 loop for one node
    n = 7
    acc = np.float32(0)
    for i in range(indptr[n], indptr[n + 1]):
        acc = np.float32(acc + y[perm[i], 3])
    assert s32[n, 3] == acc


# ---------------------------------------------------------------- packing

@given(st.lists(st.integers(0, 6), min_size=1, max_size=12))
@settings(max_examples=60, deadline=None)
def test_positions_and_to_dense_batch(counts):
    gid = np.repeat(np.arange(len(counts)), counts)
    pos = OP.positions(gid)
    cu = OP.cu_seqlens(counts)
    assert np.array_equal(pos, np.arange(len(gid)) - cu[gid])
    x = torch.arange(len(gid), dtype=torch.float32)[:, None]
    n = max(counts) + 1
    dense, m = OP.to_dense_batch(x, gid, len(counts), n)
    assert torch.equal(dense[m], x)
    assert int(m.sum()) == len(gid)


def test_nearest_multiple_of_8():
    assert [OP.nearest_multiple_of_8(n) for n in (1, 8, 9, 16, 17)] == [8, 8, 16, 16, 24]


# ---------------------------------------------------------------- block arithmetic

def _mab_sd(d, zero_q=False, identity_o=False, seed=0):
    g = torch.Generator().manual_seed(seed)
    sd = {}
    for name in ("fc_q", "fc_k", "fc_v", "fc_o"):
        sd[f"{name}.weight"] = torch.randn(d, d, generator=g, dtype=torch.float64) / np.sqrt(d)
        sd[f"{name}.bias"] = torch.randn(d, generator=g, dtype=torch.float64) * 0.1
    if zero_q:
        sd["fc_q.weight"].zero_()
        sd["fc_q.bias"].zero_()
    if identity_o:
        sd["fc_o.weight"] = torch.eye(d, dtype=torch.float64)
        sd["fc_o.bias"] = torch.zeros(d, dtype=torch.float64)
    return sd


def test_mab_closed_forms_pin_v_convention():
    d, h = 32, 2
    sd = _mab_sd(d, zero_q=True, identity_o=True)
    g = torch.Generator().manual_seed(5)
    Q = torch.randn(2, 3, d, generator=g, dtype=torch.float64)
    K = torch.randn(2, 7, d, generator=g, dtype=torch.float64)
    lin = lambda name, x: x @ sd[f"{name}.weight"].T + sd[f"{name}.bias"]
    # uniform attention: O = mean over keys of V; esa/mha.py uses V = fc_v(K)
    o = lin("fc_v", K).mean(1, keepdim=True).expand(2, 3, d)
    out = OMod.mab_padded(sd, "", Q, K, h)
    assert torch.allclose(out, o + OMod.mish(o), atol=1e-12)
    # the varlen module uses V = fc_v(fc_k(K)) (esa/mha_flash_varlen.py:155-156)
    Kq = torch.randn(2, 7, d, generator=g, dtype=torch.float64)
    out_v = OMod.mab_varlen(sd, "", Kq, Kq, [7, 4], h)
    ov = torch.stack([lin("fc_v", lin("fc_k", Kq[0, :7])).mean(0), lin("fc_v", lin("fc_k", Kq[1, :4])).mean(0)])
    assert torch.allclose(out_v[0, 0], ov[0] + OMod.mish(ov[0]), atol=1e-12)
    assert torch.allclose(out_v[1, 0], ov[1] + OMod.mish(ov[1]), atol=1e-12)
    # padding rows of the varlen path: attention output 0 -> 0 + mish(fc_o(0)) = mish(0) = 0
    assert torch.allclose(out_v[1, 4:], torch.zeros(3, d, dtype=torch.float64))


def test_layer_norm_matches_torch():
    d = 24
    sd = {"ln.weight": torch.randn(d, dtype=torch.float64), "ln.bias": torch.randn(d, dtype=torch.float64)}
    x = torch.randn(5, d, dtype=torch.float64)
    ref = F.layer_norm(x, (d,), sd["ln.weight"], sd["ln.bias"], eps=1e-8)
    assert torch.allclose(OMod.layer_norm(sd, "ln.", x), ref, atol=1e-12)
    assert torch.allclose(OMod.mish(x), F.mish(x), atol=1e-12)


def test_mish_grad_matches_autograd_and_closed_forms():
    x = torch.linspace(-40, 40, 20001, dtype=torch.float64, requires_grad=True)
    F.mish(x).sum().backward()
    g = OMod.mish_grad(x.detach())
    assert torch.allclose(g, x.grad, rtol=1e-12, atol=1e-15)
    # mish'(0) = tanh(ln 2) = 3/5; mish' -> 1 for large x, -> 0 for very negative x
    assert abs(float(OMod.mish_grad(torch.zeros(1, dtype=torch.float64))) - 0.6) < 1e-15
    assert abs(float(OMod.mish_grad(torch.tensor([30.0], dtype=torch.float64))) - 1.0) < 1e-12
    assert abs(float(OMod.mish_grad(torch.tensor([-60.0], dtype=torch.float64)))) < 1e-20
    # the minimum of mish (x ~ -1.1924, mish ~ -0.30884): the derivative changes sign there
    lo, hi = torch.tensor([-1.1925], dtype=torch.float64), torch.tensor([-1.1923], dtype=torch.float64)
    assert float(OMod.mish_grad(lo)) < 0 < float(OMod.mish_grad(hi))
    assert abs(float(OMod.mish(torch.tensor([-1.1924], dtype=torch.float64))) + 0.30884) < 1e-5
