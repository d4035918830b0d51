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


# ---------------------------------------------------------------- block compositions

def _lin_sd(sd, prefix, d_in, d_out, g, zero=False, eye=False):
    w = torch.randn(d_out, d_in, generator=g, dtype=torch.float64) / np.sqrt(d_in)
    b = torch.randn(d_out, generator=g, dtype=torch.float64) * 0.1
    if zero:
        w, b = torch.zeros_like(w), torch.zeros_like(b)
    if eye:
        w, b = torch.eye(d_out, d_in, dtype=torch.float64), torch.zeros_like(b)
    sd[prefix + "weight"], sd[prefix + "bias"] = w, b


def _ln_sd(sd, prefix, d, g, zero=False):
    sd[prefix + "weight"] = torch.zeros(d, dtype=torch.float64) if zero else 1 + 0.3 * torch.randn(
        d, generator=g, dtype=torch.float64)
    sd[prefix + "bias"] = torch.zeros(d, dtype=torch.float64) if zero else 0.2 * torch.randn(
        d, generator=g, dtype=torch.float64)


def _block_sd(sd, prefix, d, hidden, g, mab_prefix="sab.mab.", zero_q=False, identity_o=False, mlp_last_zero=False,
              mlp_identity=False, zero_block=False):
    """Parameters of a pre-norm block with a 2-layer standard MLP under the reference's key names."""
    _ln_sd(sd, prefix + "norm.ln.", d, g, zero=zero_block)
    for name in ("fc_q", "fc_k", "fc_v", "fc_o"):
        _lin_sd(sd, prefix + mab_prefix + name + ".", d, d, g, zero=(name == "fc_q" and zero_q),
                eye=(name == "fc_o" and identity_o))
    if zero_block:   # v = 0 and fc_o(0) = 0: the attention sub-block outputs exactly 0
        sd[prefix + mab_prefix + "fc_v.bias"].zero_()
        sd[prefix + mab_prefix + "fc_o.bias"].zero_()
    _ln_sd(sd, prefix + "norm_mlp.ln.", d, g, zero=zero_block)
    h0 = d if mlp_identity else hidden
    _lin_sd(sd, prefix + "mlp.mlp.0.", d, h0, g, eye=mlp_identity)
    _lin_sd(sd, prefix + "mlp.mlp.2.", h0, d, g, zero=mlp_last_zero or zero_block, eye=mlp_identity)
    if zero_block:
        sd[prefix + "mlp.mlp.0.bias"].zero_()


def _lnf(sd, prefix, x):
    """torch's own LayerNorm with the block's parameters (eps 1e-8, esa/utils/norm_layers.py:36)."""
    return F.layer_norm(x, (x.shape[-1],), sd[prefix + "weight"], sd[prefix + "bias"], eps=1e-8)


def _linf(sd, prefix, x):
    return F.linear(x, sd[prefix + "weight"], sd[prefix + "bias"])


@pytest.mark.parametrize("num_layers", [1, 2, 3])
def test_mlp_standard_matches_reference_sequential(num_layers):
    """SmallMLP's layer walk (esa/mlp_utils.py:18-44) built from torch modules in the reference's order:
    [Linear, Identity, Mish] for one layer; Linear, Mish, ..., Linear otherwise."""
    d_in, inter, d_out = 12, 20, 12
    if num_layers == 1:
        seq = torch.nn.Sequential(torch.nn.Linear(d_in, d_out), torch.nn.Identity(), torch.nn.Mish())
    else:
        layers = []
        for i in range(num_layers):
            a = d_in if i == 0 else inter
            b = d_out if i == num_layers - 1 else inter
            layers.append(torch.nn.Linear(a, b))
            if i != num_layers - 1:
                layers.append(torch.nn.Mish())
        seq = torch.nn.Sequential(*layers)
    torch.manual_seed(num_layers)
    seq = seq.double()
    sd = {"mlp." + k: v for k, v in seq.state_dict().items()}
    x = torch.randn(7, d_in, dtype=torch.float64, generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        assert torch.allclose(OMod.mlp_standard(sd, "", x, num_layers), seq(x), atol=1e-12)


def _one_segment(n, d, seed):
    return torch.randn(n, d, dtype=torch.float64, generator=torch.Generator().manual_seed(seed)) * 2 + 0.5


def test_sab_complete_closed_forms():
    """fc_q = 0 makes attention uniform: the MAB gives m + mish(m) with m the key-mean of fc_v(LN(X)), so a
    zero last MLP layer leaves out = LN(X) + m + mish(m) (the residual is on the normed X,
    esa/masked_layers.py:471-472); identity MLP Linears then add mish(LN2(out)) (:478-483)."""
    d, h, n = 16, 2, 9
    g = torch.Generator().manual_seed(11)
    X = _one_segment(n, d, 12)
    cu = [0, n]

    def attn(sd_, pre, x):
        return OMod.mab_packed(sd_, pre, x, x, cu, cu, h)

    sd = {}
    _block_sd(sd, "", d, 24, g, zero_q=True, identity_o=True, mlp_last_zero=True)
    xn = _lnf(sd, "norm.ln.", X)
    m = _linf(sd, "sab.mab.fc_v.", xn).mean(0, keepdim=True)
    ref = xn + (m + F.mish(m))
    got = OMod.sab_complete(sd, "", X, h, attn, 2)
    assert torch.allclose(got, ref, atol=1e-12)
    assert not torch.allclose(got, X + m + F.mish(m), atol=1e-3)   # a residual on X would fail

    sd2 = {}
    _block_sd(sd2, "", d, 24, g, zero_q=True, identity_o=True, mlp_identity=True)
    xn = _lnf(sd2, "norm.ln.", X)
    m = _linf(sd2, "sab.mab.fc_v.", xn).mean(0, keepdim=True)
    o1 = xn + m + F.mish(m)
    ref2 = o1 + F.mish(_lnf(sd2, "norm_mlp.ln.", o1))
    assert torch.allclose(OMod.sab_complete(sd2, "", X, h, attn, 2), ref2, atol=1e-12)


def test_mab_packed_equals_padded_with_reference_bias():
    """The packed MAB with the edge mask equals the reference's padded MAB with the restated -99999 bias
    (esa/masked_layers.py:217-268, esa/mha.py:73-77) on every valid row; likewise in node mode."""
    d, h = 16, 2
    g = torch.Generator().manual_seed(21)
    sd = {}
    for name in ("fc_q", "fc_k", "fc_v", "fc_o"):
        _lin_sd(sd, name + ".", d, d, g)
    gb, _ = generators.small_molecules(seed=4, num_graphs=3)
    n = OP.nearest_multiple_of_8(int(gb.edge_counts.max()) + 1)
    t = int(gb.cu_seqlens[-1])
    Xp = torch.randn(t, d, dtype=torch.float64, generator=g)
    gid = np.repeat(np.arange(gb.num_graphs), gb.edge_counts)
    X, valid = OP.to_dense_batch(Xp, gid, gb.num_graphs, n)
    src, dst = gb.edge_index
    assert OM.edge_adjacency_global(src, dst).any(1).all()   # every edge has a key: no uniform rows
    bias = OM.edge_bias_padded(gb.edge_index, gid, gb.num_graphs, n, dtype=torch.float64)
    ref = OMod.mab_padded(sd, "", X, X, h, bias)[valid]
    got = OMod.mab_packed(sd, "", Xp, Xp, gb.cu_seqlens, gb.cu_seqlens, h, src, dst)
    assert torch.allclose(got, ref, atol=1e-10)

    ei, bm = node_graph(5, [7, 11, 4], extra_dup=False, self_loops=False)
    counts = np.bincount(bm)
    nn_ = OP.nearest_multiple_of_8(int(counts.max()) + 1)
    Xn = torch.randn(len(bm), d, dtype=torch.float64, generator=g)
    Xpad, vmask = OP.to_dense_batch(Xn, bm, len(counts), nn_)
    nbias = OM.node_bias_padded(ei, bm, len(counts), nn_, dtype=torch.float64)
    order = np.lexsort((ei[1], ei[0]))
    indptr = OP.cu_seqlens(np.bincount(ei[0], minlength=len(bm)))
    indices = ei[1][order]
    has_key = np.diff(indptr) > 0
    ref_n = OMod.mab_padded(sd, "", Xpad, Xpad, h, nbias)[vmask]
    cu = OP.cu_seqlens(counts)
    got_n = OMod.mab_packed(sd, "", Xn, Xn, cu, cu, h, adj=(indptr, indices))
    assert torch.allclose(got_n[has_key], ref_n[torch.as_tensor(has_key)], atol=1e-10)


@pytest.mark.parametrize("packed", [True, False])
def test_pma_complete_closed_forms(packed):
    """fc_q = 0 and fc_o = I: every seed's MAB output is m + mish(m), m the key-mean of fc_v(LN(X)) over the
    set's valid tokens (packed) or all N positions, padding included (the reference, esa/mha.py:108-109 with
    no mask at esa/masked_layers.py:593); no residual unless k == N (:595-603), where the padded form adds
    LN(X) of every slot and the packed form LN(X) at valid slots and 0 at padding."""
    d, h = 16, 2
    g = torch.Generator().manual_seed(31)
    lens = [5, 8, 3]
    b, n = len(lens), 8
    cu = OP.cu_seqlens(lens)
    gid = np.repeat(np.arange(b), lens)
    Xp = _one_segment(int(cu[-1]), d, 32)
    X, valid = OP.to_dense_batch(Xp, gid, b, n)
    for k in (3, n):
        sd = {"pma.S": torch.randn(1, k, d, dtype=torch.float64, generator=g)}
        _block_sd(sd, "", d, 24, g, mab_prefix="pma.mab.", zero_q=True, identity_o=True, mlp_last_zero=True)
        xn = _lnf(sd, "norm.ln.", X)             # padding rows: LN(0) = the LN bias
        v = _linf(sd, "pma.mab.fc_v.", xn)
        if packed:
            m = torch.stack([v[i, :lens[i]].mean(0) for i in range(b)])
            res = xn * valid[..., None]
            got = OMod.pma_complete(sd, "", Xp, h, 2, cu=cu, max_items=n)
        else:
            m = v.mean(1)
            res = xn
            got = OMod.pma_complete(sd, "", X, h, 2)
        att = (m + F.mish(m))[:, None, :].expand(b, k, d)
        ref = res + att if k == n else att
        assert torch.allclose(got, ref, atol=1e-12), (packed, k)
    # the MLP half: identity Linears give out + mish(LN2(out))
    sd = {"pma.S": torch.randn(1, 3, d, dtype=torch.float64, generator=g)}
    _block_sd(sd, "", d, 24, g, mab_prefix="pma.mab.", zero_q=True, identity_o=True, mlp_identity=True)
    xn = _lnf(sd, "norm.ln.", X)
    v = _linf(sd, "pma.mab.fc_v.", xn)
    m = torch.stack([v[i, :lens[i]].mean(0) for i in range(b)]) if packed else v.mean(1)
    o1 = (m + F.mish(m))[:, None, :].expand(b, 3, d)
    ref = o1 + F.mish(_lnf(sd, "norm_mlp.ln.", o1))
    got = OMod.pma_complete(sd, "", Xp, h, 2, cu=cu, max_items=n) if packed else OMod.pma_complete(sd, "", X, h, 2)
    assert torch.allclose(got, ref, atol=1e-12)


@pytest.mark.parametrize("layer_types", ["MSP", "MMSSMMSSP", "MSPS"])
def test_esa_composition_closed_form(layer_types):
    """Encoder blocks whose LayerNorms, fc_v / fc_o biases and MLP output are zero output exactly 0, so
    enc = X (enc = encoder(X) + X, esa/masked_layers.py:917) whatever their other weights; a later S on the
    seeds is zeroed the same way.  The decoder PMA with fc_q = 0, fc_o = I gives m + mish(m) for every seed,
    m the key-mean of fc_v(LN(enc)), and graph_emb = mish(W mean_seeds + b) (:928-929).  A zeroed S block
    after the P maps the seeds to exactly 0 (its residual is on the normed input, also zero), which leaves
    graph_emb = mish(b)."""
    d, h, k = 16, 2, 3
    g = torch.Generator().manual_seed(41)
    lens = [6, 9, 4]
    b, n = len(lens), 16
    cu = OP.cu_seqlens(lens)
    gid = np.repeat(np.arange(b), lens)
    Xp = _one_segment(int(cu[-1]), d, 42)
    X, valid = OP.to_dense_batch(Xp, gid, b, n)
    sd = {}
    types = list(layer_types)
    p_at = types.index("P")
    for i in range(p_at):
        _block_sd(sd, f"encoder.{i}.", d, 24, g, zero_block=True)
    sd["decoder.0.pma.S"] = torch.randn(1, k, d, dtype=torch.float64, generator=g)
    _block_sd(sd, "decoder.0.", d, 24, g, mab_prefix="pma.mab.", zero_q=True, identity_o=True, mlp_last_zero=True)
    for j in range(len(types) - p_at - 1):
        _block_sd(sd, f"decoder.{j + 1}.", d, 24, g, zero_block=True)
    _lin_sd(sd, "decoder_linear.", d, 5, g)

    def attn(sd_, pre, x):
        return OMod.mab_packed(sd_, pre, x, x, cu, cu, h)

    def pool(sd_, pre, x):
        return OMod.pma_complete(sd_, pre, x, h, 2, cu=cu, max_items=n)

    g_emb, enc = OMod.esa(sd, Xp, layer_types, h, 2, attn, attn, pool)
    assert torch.equal(enc, Xp)
    v = _linf(sd, "decoder.0.pma.mab.fc_v.", _lnf(sd, "decoder.0.norm.ln.", Xp))
    m = torch.stack([v[cu[i]:cu[i + 1]].mean(0) for i in range(b)])
    ref = F.mish(_linf(sd, "decoder_linear.", m + F.mish(m)))
    if layer_types.endswith("S"):
        ref = F.mish(sd["decoder_linear.bias"]).expand(b, 5)
    assert torch.allclose(g_emb, ref, atol=1e-12)

    def attn_p(sd_, pre, x):
        return OMod.mab_padded(sd_, pre, x, x, h)

    def pool_p(sd_, pre, x):
        return OMod.pma_complete(sd_, pre, x, h, 2)

    g_pad, enc_pad = OMod.esa(sd, X, layer_types, h, 2, attn_p, attn_p, pool_p)
    assert torch.equal(enc_pad, X)
    vp = _linf(sd, "decoder.0.pma.mab.fc_v.", _lnf(sd, "decoder.0.norm.ln.", X)).mean(1)   # padding included
    ref_p = F.mish(_linf(sd, "decoder_linear.", vp + F.mish(vp)))
    if layer_types.endswith("S"):
        ref_p = F.mish(sd["decoder_linear.bias"]).expand(b, 5)
    assert torch.allclose(g_pad, ref_p, atol=1e-12)


@pytest.mark.parametrize("mode", ["none", "edge", "node"])
def test_varlen_attention_diff_matches_dense_and_analytic_backward(mode):
    """The differentiable form the module oracle uses (analytic backward without a mask, the pair-list form
    with one) equals varlen_attention's output and varlen_attention_bwd's gradients."""
    gb, _ = generators.small_molecules(seed=8, num_graphs=3)
    cu = gb.cu_seqlens
    src, dst, adj = None, None, None
    if mode == "edge":
        src, dst = gb.edge_index
    t, h, d = int(cu[-1]), 3, 16
    if mode == "node":
        ei, bm = node_graph(9, [13, 8, 21])
        counts = np.bincount(bm)
        cu = OP.cu_seqlens(counts)
        t = len(bm)
        order = np.lexsort((ei[1], ei[0]))
        adj = (OP.cu_seqlens(np.bincount(ei[0], minlength=t)), ei[1][order])
    g = torch.Generator().manual_seed(4)
    q, k, v, go = (torch.randn(t, h, d, dtype=torch.float64, generator=g) for _ in range(4))
    qd, kd, vd = (x.clone().requires_grad_(True) for x in (q, k, v))
    out = OA.varlen_attention_diff(qd, kd, vd, cu, cu, 0.3, src, dst, adj)
    ref, _ = OA.varlen_attention(q, k, v, cu, cu, 0.3, src, dst, adj=adj)
    assert torch.allclose(out, ref, atol=1e-12)
    out.backward(go)
    rdq, rdk, rdv = OA.varlen_attention_bwd(go, q, k, v, cu, cu, 0.3, src, dst, adj=adj)
    for a, b in ((qd.grad, rdq), (kd.grad, rdk), (vd.grad, rdv)):
        assert torch.allclose(a, b, atol=1e-11)


def test_token_budget_batches_hand_case():
    # 3 + 4 fit, 5 would pass 8; 5 alone; 10 is oversize: a batch of its own; 1 + 1
    assert OP.token_budget_batches([3, 4, 5, 10, 1, 1], 8) == [[0, 1], [2], [3], [4, 5]]
    assert OP.token_budget_batches([], 8) == []
    assert OP.token_budget_batches([0, 0, 9, 0], 8) == [[0, 1], [2], [3]]


@given(st.lists(st.integers(0, 40), min_size=1, max_size=60), st.integers(0, 100))
@settings(max_examples=200, deadline=None)
def test_token_budget_batches_is_the_greedy_partition(counts, budget):
    """Contiguous in-order batches; each within the budget unless a single graph; and none could take the
    next graph: the properties that fix the greedy partition uniquely."""
    batches = OP.token_budget_batches(counts, budget)
    assert [i for b in batches for i in b] == list(range(len(counts)))
    for j, b in enumerate(batches):
        s = sum(counts[i] for i in b)
        assert s <= budget or len(b) == 1
        if j + 1 < len(batches):
            assert s + counts[batches[j + 1][0]] > budget


def test_padded_sdpa_equals_varlen_on_valid_rows():
    """The reference's padded fallback (torch SDPA over [B, H, N, D] with the key-padding mask) equals the
    per-set attention on every valid query row, forward and backward; with a pair bias it equals the masked
    attention (the edge mask's 0 / -99999 bias)."""
    lens = [5, 12, 1, 9]
    cu = OP.cu_seqlens(lens)
    t, h, d = int(cu[-1]), 2, 16
    g = torch.Generator().manual_seed(6)
    q, k, v, go = (torch.randn(t, h, d, dtype=torch.float64, generator=g) for _ in range(4))
    qd, kd, vd = (x.clone().requires_grad_(True) for x in (q, k, v))
    out = OA.padded_sdpa(qd, kd, vd, cu, cu, 16, 0.3, graphs_per_call=3)
    ref, _ = OA.varlen_attention(q, k, v, cu, cu, 0.3)
    assert torch.allclose(out, ref, atol=1e-12)
    out.backward(go)
    rdq, rdk, rdv = OA.varlen_attention_bwd(go, q, k, v, cu, cu, 0.3)
    for a, b in ((qd.grad, rdq), (kd.grad, rdk), (vd.grad, rdv)):
        assert torch.allclose(a, b, atol=1e-11)
    gb, _ = generators.small_molecules(seed=2, num_graphs=3)
    cu2 = gb.cu_seqlens
    src, dst = gb.edge_index
    t2 = int(cu2[-1])
    q2, k2, v2 = (torch.randn(t2, h, d, dtype=torch.float64, generator=g) for _ in range(3))

    def bias(b):
        s_, e_ = int(cu2[b]), int(cu2[b + 1])
        m = torch.as_tensor(OM.edge_adjacency_segment(src, dst, s_, e_))
        return torch.where(m, 0.0, OM.MASK_FILL)

    out2 = OA.padded_sdpa(q2, k2, v2, cu2, cu2, int(np.diff(cu2).max()), 0.25, pair_bias=bias)
    ref2, _ = OA.varlen_attention(q2, k2, v2, cu2, cu2, 0.25, src, dst)
    assert torch.allclose(out2, ref2, atol=1e-10)


def test_torch_gather_and_scatter_baselines_match_the_oracle():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((50, 6)).astype(np.float32)
    src, dst = rng.integers(0, 50, 300), rng.integers(0, 50, 300)
    h = OE.edge_gather_torch(torch.as_tensor(x), torch.as_tensor(src), torch.as_tensor(dst))
    assert np.array_equal(h.numpy(), OE.edge_gather(x, src, dst))
    y = rng.standard_normal((300, 6))
    assert np.allclose(OE.scatter_sum_torch(torch.as_tensor(y), torch.as_tensor(dst), 50).numpy(),
                       OE.segment_sum_f64(y, dst, 50), atol=1e-12)
