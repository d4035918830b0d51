"""GPU parity of node-mode (CSR adjacency) attention against the oracle.

The mask is the one get_adj_mask_from_edge_index_node (esa/masked_layers.py:79-118)
builds: query node src attends to key node dst for every edge src -> dst.
Kernels are called through the C ABI (mind_amd.esa.attention, mask kind
ESA_MASK_NODE).  Bars: bf16 max-abs 2e-2 / mean-abs 2e-3 (gradients scaled by
max(1, max|ref|)); fp32 1e-5 relative.  Graphs include repeated edges,
self-loops, nodes without out-edges, empty and one-node graphs.
"""
import numpy as np
import pytest
import torch

from mind_amd import generators
from mind_amd.esa import attention as A
from mind_amd.esa import masked_layers as ML
from mind_amd.esa.mha import SAB
from mind_amd.esa.packing import NodeAdjacency, nearest_multiple_of_8
from oracle import attention as OA
from oracle import mask as OM
from oracle import modules as OMod
from tests._util import assert_bf16_close, assert_f32_close, grad_scale, node_graph, seeded_normal

pytestmark = pytest.mark.gpu

D = 16


def _run(device, sizes, seed, heads, dtype, ei=None, bm=None):
    if ei is None:
        ei, bm = node_graph(seed, sizes)
    na = NodeAdjacency.from_edge_index(torch.as_tensor(ei), torch.as_tensor(bm), len(sizes), max(sizes + [1]))
    t = len(bm)
    q, k, v, g = (seeded_normal((t, heads, D), seed + i, dtype) for i in range(4))
    cu = na.cu_seqlens
    qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
    ip, ix = na.indptr.to(device), na.indices.to(device)
    out, lse = A.varlen_attention(qd, kd, vd, cu.to(device), cu.to(device), 0, 0, softmax_scale=0.25,
                                  adj_indptr=ip, adj_indices=ix, return_lse=True)
    out.backward(g.to(device))
    torch.cuda.synchronize()
    adj = (na.indptr.numpy(), na.indices.numpy())
    ref, lse_ref = OA.varlen_attention(q, k, v, cu.numpy(), cu.numpy(), 0.25, adj=adj)
    grads = OA.varlen_attention_bwd(g, q, k, v, cu.numpy(), cu.numpy(), 0.25, adj=adj)
    got = (out.detach().cpu(), lse.cpu(), qd.grad.cpu(), kd.grad.cpu(), vd.grad.cpu())
    return got, (ref, lse_ref) + tuple(grads), na


def _check(got, ref, dtype):
    out, lse, dq, dk, dv = got
    rout, rlse, rdq, rdk, rdv = ref
    fin = torch.isfinite(rlse)
    assert torch.equal(torch.isfinite(lse), fin), "lse -inf pattern (nodes without out-edges)"
    if dtype == torch.float32:
        assert_f32_close(out, rout, "out")
        assert float((lse.double()[fin] - rlse[fin]).abs().max()) <= 1e-5 * max(1.0, float(rlse[fin].abs().max()))
        for name, a, b in (("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
            assert_f32_close(a, b, name)
    else:
        assert_bf16_close(out, rout, what="out")
        # fp32 softmax over bf16 inputs: the LSE carries only fp32 rounding of bf16-exact scores
        assert float((lse.double()[fin] - rlse[fin]).abs().max()) < 1e-3
        for name, a, b in (("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
            assert_bf16_close(a, b, grad_scale(b), name)
    # rows without an admissible key: output 0
    dead = ~fin[0]
    assert (out[dead] == 0).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("heads", [16, 32, 5])
def test_node_mask_random_graphs(device, dtype, heads):
    sizes = [9, 1, 30, 17, 2, 25]
    got, ref, _ = _run(device, sizes, 11 + heads, heads, dtype)
    _check(got, ref, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_node_mask_isolated_nodes_and_empty_graph(device, dtype):
    """Graph 1 has no nodes, graph 2 no edges; node 0 has no out-edges."""
    sizes = [4, 0, 3, 5]
    ei = np.array([[1, 1, 2, 2, 2, 7, 8, 11, 11], [0, 2, 1, 3, 3, 8, 7, 10, 11]], dtype=np.int64)
    bm = np.concatenate([np.full(n, b) for b, n in enumerate(sizes)]).astype(np.int64)
    got, ref, na = _run(device, sizes, 3, 16, dtype, ei, bm)
    _check(got, ref, dtype)
    lse = got[1]
    for node in (0, 3, 4, 5, 6, 9, 10):      # no out-edges
        assert torch.isneginf(lse[:, node]).all()


@pytest.mark.parametrize("planned", [False, True])
def test_node_mask_many_segments(device, planned):
    """300 graphs of 0-6 nodes (a third of them empty): every token finds its segment among more than 64
    (empty segments share their start with the next one), with several tokens of different segments and row
    lengths in one wave."""
    rng = np.random.default_rng(77)
    sizes = [int(x) for x in rng.integers(0, 7, size=300)]
    sizes[-1] = max(sizes[-1], 1)
    if planned:
        ei, bm = node_graph(78, sizes)
        na = NodeAdjacency.from_edge_index(torch.as_tensor(ei).to(device), torch.as_tensor(bm).to(device),
                                           len(sizes), max(sizes))
        t = len(bm)
        q, k, v, g = (seeded_normal((t, 3, D), 600 + i, torch.float32) for i in range(4))
        qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
        cu = na.cu_seqlens
        out = A.varlen_attention(qd, kd, vd, cu, cu, 0, 0, softmax_scale=0.25, **na.kernel_mask(padded=False))
        out.backward(g.to(device))
        adj = (na.indptr.cpu().numpy(), na.indices.cpu().numpy())
        cun = cu.cpu().numpy()
        ref, _ = OA.varlen_attention(q, k, v, cun, cun, 0.25, adj=adj)
        rdq, rdk, rdv = OA.varlen_attention_bwd(g, q, k, v, cun, cun, 0.25, adj=adj)
        assert_f32_close(out.detach().cpu(), ref, "out")
        for name, a, b in (("dq", qd.grad, rdq), ("dk", kd.grad, rdk), ("dv", vd.grad, rdv)):
            assert_f32_close(a.cpu(), b, name)
    else:
        got, ref, _ = _run(device, sizes, 79, 3, torch.float32)
        _check(got, ref, torch.float32)


def test_node_mask_protein_like_full_size(device):
    """Config-1 protein graphs in node mode (radius edges, cap 16): every node attends to its neighbours."""
    gb = generators.protein_like(seed=0)
    sizes = [int(n) for n in gb.node_counts]
    got, ref, _ = _run(device, sizes, 5, 16, torch.bfloat16, gb.edge_index, gb.batch)
    _check(got, ref, torch.bfloat16)


def test_node_mask_backward_deterministic(device):
    sizes = [40, 33, 51]
    ei, bm = node_graph(2, sizes)
    na = NodeAdjacency.from_edge_index(torch.as_tensor(ei).to(device), torch.as_tensor(bm).to(device), 3, 51)
    t = len(bm)
    q, k, v, g = (seeded_normal((t, 16, D), 20 + i).to(device) for i in range(4))
    cu = na.cu_seqlens
    out, lse = A.attn_fwd(q, k, v, cu, cu, 0, 0, 0.25, adj_indptr=na.indptr, adj_indices=na.indices)
    r1 = A.attn_bwd(g, q, k, v, out, lse, cu, cu, 0, 0, 0.25, adj_indptr=na.indptr, adj_indices=na.indices)
    r2 = A.attn_bwd(g, q, k, v, out, lse, cu, cu, 0, 0, 0.25, adj_indptr=na.indptr, adj_indices=na.indices)
    for a, b in zip(r1, r2):
        assert torch.equal(a, b)


def _padded_nodes(sizes, n, d, seed):
    x = torch.randn(len(sizes), n, d, generator=torch.Generator().manual_seed(seed))
    valid = torch.zeros(len(sizes), n, dtype=torch.bool)
    for b, L in enumerate(sizes):
        valid[b, :L] = True
    return x, valid


@pytest.mark.parametrize("backend", ["hip", "xformers"])
def test_sab_node_mask(device, backend):
    """SAB with the node-mode mask: "hip" over valid nodes; "xformers" the reference's padded -99999 bias,
    rows without edges (and padding) softmaxing over all N positions."""
    sizes = [7, 12, 3, 10]
    dm, h = 64, 4
    n = nearest_multiple_of_8(max(sizes) + 1)
    ei, bm = node_graph(8, sizes)
    torch.manual_seed(4)
    m = SAB(dm, dm, h, 0.0, backend).to(device)
    X, valid = _padded_nodes(sizes, n, dm, 9)
    mask = ML.get_adj_mask_from_edge_index_node(torch.as_tensor(ei).to(device), len(sizes), n,
                                                torch.as_tensor(bm).to(device))
    got = m(X.to(device), adj_mask=mask).cpu()
    sd = {kk: vv.detach().cpu() for kk, vv in m.state_dict().items()}
    if backend == "hip":
        cu = mask.cu_seqlens.cpu().numpy()
        ref = OMod.mab_packed(sd, "mab.", X[valid], X[valid], cu, cu, h,
                              adj=(mask.indptr.cpu().numpy(), mask.indices.cpu().numpy()))
        assert_f32_close(got[valid], ref, "SAB hip node mask")
    else:
        bias = OM.node_bias_padded(ei, bm, len(sizes), n, dtype=torch.float64)
        ref = OMod.mab_padded(sd, "mab.", X, X, h, bias)
        assert_f32_close(got, ref, "SAB xformers node mask")


def test_esa_node_mode(device):
    """ESA in node mode (every MIND YAML's apply_attention_on: node): M, S, P over node tokens, "hip" backend."""
    sizes = [11, 6, 14]
    dm, h = 64, 4
    n = nearest_multiple_of_8(max(sizes) + 1)
    ei, bm = node_graph(12, sizes)
    torch.manual_seed(7)
    model = ML.ESA(num_outputs=1, dim_output=dm, dim_hidden=[dm, dm, dm], num_heads=[h, h, h], layer_types="MSP",
                   node_or_edge="node", xformers_or_torch_attn="hip", use_mlps=True, mlp_hidden_size=2 * dm,
                   num_mlp_layers=2, mlp_type="standard").to(device)
    X, valid = _padded_nodes(sizes, n, dm, 13)
    g_emb, enc = model(X.to(device), torch.as_tensor(ei).to(device), torch.as_tensor(bm).to(device), n)
    sd = {kk: vv.detach().cpu() for kk, vv in model.state_dict().items()}
    na = NodeAdjacency.from_edge_index(torch.as_tensor(ei), torch.as_tensor(bm), len(sizes), n)
    cu = na.cu_seqlens.numpy()
    adj = (na.indptr.numpy(), na.indices.numpy())
    xp = X.double()[valid]
    g_ref, enc_ref = OMod.esa(
        sd, xp, "MSP", h, 2,
        attn_m=lambda s_, p_, x: OMod.mab_packed(s_, p_, x, x, cu, cu, h, adj=adj),
        attn_s=lambda s_, p_, x: OMod.mab_packed(s_, p_, x, x, cu, cu, h),
        pool=lambda s_, p_, x: OMod.pma_complete(s_, p_, x, h, 2, cu=cu, max_items=n))
    assert_f32_close(enc.cpu()[valid], enc_ref, "ESA node-mode encoder (valid rows)")
    assert_f32_close(g_emb.cpu().reshape(g_ref.shape), g_ref, "ESA node-mode graph embedding")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_node_plan_equals_per_call_transpose(device, dtype):
    """A node plan built once (esa_node_plan_build, passed as adj_plan) gives the per-call path's forward and
    backward bit for bit on two calls in a row (repeated edges, self-loops, an empty and a one-node graph),
    and its first nnz ints are the CSR's indices (the forward reads the plan as the indices array)."""
    sizes = [37, 0, 64, 1, 90]
    ei, bm = node_graph(31, sizes)
    na = NodeAdjacency.from_edge_index(torch.as_tensor(ei).to(device), torch.as_tensor(bm).to(device), len(sizes),
                                       max(sizes))
    t, heads = len(bm), 16
    q, k, v, g = (seeded_normal((t, heads, D), 400 + i, dtype).to(device) for i in range(4))
    cu, ip, ix = na.cu_seqlens, na.indptr, na.indices
    plan = na.plan()
    assert torch.equal(plan[: 4 * ix.numel()].view(torch.int32), ix)
    out0, lse0 = A.attn_fwd(q, k, v, cu, cu, 0, 0, 0.25, adj_indptr=ip, adj_indices=ix)
    ref = A.attn_bwd(g, q, k, v, out0, lse0, cu, cu, 0, 0, 0.25, adj_indptr=ip, adj_indices=ix)
    for _ in range(2):
        out, lse = A.attn_fwd(q, k, v, cu, cu, 0, 0, 0.25, adj_indptr=ip, adj_indices=ix, adj_plan=plan)
        assert torch.equal(out, out0) and torch.equal(lse, lse0)
        got = A.attn_bwd(g, q, k, v, out, lse, cu, cu, 0, 0, 0.25, adj_indptr=ip, adj_indices=ix, adj_plan=plan)
        for name, a, b in zip(("dq", "dk", "dv"), got, ref):
            assert torch.equal(a, b), name


def test_node_plan_entries_outside_segment(device):
    """Entries naming a key of another segment are ignored by the planned backward as by the per-call one
    (the transposed rows list such a query under the foreign key; the key pass drops it by segment)."""
    cu = torch.tensor([0, 3, 7], dtype=torch.int32, device=device)
    # segments {0, 1, 2} and {3, .., 6}; row 0 lists key 5 (segment 1) beside its own keys, row 4 lists key 1
    rows = [[1, 2, 5], [0], [0, 1], [4, 6], [1, 3], [6], [3, 5]]
    ip = torch.tensor(np.cumsum([0] + [len(r) for r in rows]), dtype=torch.int32, device=device)
    ix = torch.tensor([j for r in rows for j in r], dtype=torch.int32, device=device)
    plan = A.node_plan(ip, ix, cu)
    q, k, v, g = (seeded_normal((7, 3, D), 500 + i, torch.float32).to(device) for i in range(4))
    out0, lse0 = A.attn_fwd(q, k, v, cu, cu, 0, 0, 0.25, adj_indptr=ip, adj_indices=ix)
    out, lse = A.attn_fwd(q, k, v, cu, cu, 0, 0, 0.25, adj_indptr=ip, adj_indices=ix, adj_plan=plan)
    assert torch.equal(out, out0) and torch.equal(lse, lse0)
    ref = A.attn_bwd(g, q, k, v, out0, lse0, cu, cu, 0, 0, 0.25, adj_indptr=ip, adj_indices=ix)
    got = A.attn_bwd(g, q, k, v, out, lse, cu, cu, 0, 0, 0.25, adj_indptr=ip, adj_indices=ix, adj_plan=plan)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    adj = (ip.cpu().numpy(), ix.cpu().numpy())
    cun = cu.cpu().numpy()
    rdq, rdk, rdv = OA.varlen_attention_bwd(g.cpu(), q.cpu(), k.cpu(), v.cpu(), cun, cun, 0.25, adj=adj)
    for a, b in zip(got, (rdq, rdk, rdv)):
        assert_f32_close(a.cpu(), b, "planned grads vs oracle")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_node_plan_cross_attention(device, dtype):
    """Queries and keys in different segment arrays (3 segments: 5/0/9 queries over 7/4/6 keys, an empty
    query segment and entries naming keys of other segments): the planned and per-call paths agree bit for
    bit and both meet the oracle bar; a plan over distinct key segments needs total_k."""
    rng = np.random.default_rng(90)
    lq, lk = [5, 0, 9], [7, 4, 6]
    cq, ck = np.cumsum([0] + lq), np.cumsum([0] + lk)
    rows = []
    for b in range(3):
        for _ in range(lq[b]):
            own = rng.choice(np.arange(ck[b], ck[b + 1]), size=int(rng.integers(0, lk[b] + 1)), replace=False)
            other = rng.integers(0, ck[-1], size=int(rng.integers(0, 3)))
            rows.append(sorted(int(x) for x in np.concatenate([own, other])))
    ip = torch.tensor(np.cumsum([0] + [len(r) for r in rows]), dtype=torch.int32, device=device)
    ix = torch.tensor([j for r in rows for j in r], dtype=torch.int32, device=device)
    cu_q = torch.tensor(cq, dtype=torch.int32, device=device)
    cu_k = torch.tensor(ck, dtype=torch.int32, device=device)
    tq, tk = int(cq[-1]), int(ck[-1])
    q, g = (seeded_normal((tq, 4, D), 700 + i, dtype).to(device) for i in range(2))
    k, v = (seeded_normal((tk, 4, D), 710 + i, dtype).to(device) for i in range(2))
    with pytest.raises(ValueError):
        A.node_plan(ip, ix, cu_q, cu_k)
    plan = A.node_plan(ip, ix, cu_q, cu_k, total_k=tk)
    out0, lse0 = A.attn_fwd(q, k, v, cu_q, cu_k, 0, 0, 0.25, adj_indptr=ip, adj_indices=ix)
    out, lse = A.attn_fwd(q, k, v, cu_q, cu_k, 0, 0, 0.25, adj_indptr=ip, adj_indices=ix, adj_plan=plan)
    assert torch.equal(out, out0) and torch.equal(lse, lse0)
    ref_g = A.attn_bwd(g, q, k, v, out0, lse0, cu_q, cu_k, 0, 0, 0.25, adj_indptr=ip, adj_indices=ix)
    got_g = A.attn_bwd(g, q, k, v, out, lse, cu_q, cu_k, 0, 0, 0.25, adj_indptr=ip, adj_indices=ix, adj_plan=plan)
    for a_, b_ in zip(got_g, ref_g):
        assert torch.equal(a_, b_)
    adj = (ip.cpu().numpy(), ix.cpu().numpy())
    rout, rlse = OA.varlen_attention(q.cpu(), k.cpu(), v.cpu(), cq, ck, 0.25, adj=adj)
    rdq, rdk, rdv = OA.varlen_attention_bwd(g.cpu(), q.cpu(), k.cpu(), v.cpu(), cq, ck, 0.25, adj=adj)
    _check((out.cpu(), lse.cpu()) + tuple(x.cpu() for x in got_g), (rout, rlse, rdq, rdk, rdv), dtype)


def test_node_mask_argument_errors(device):
    q = torch.zeros(4, 16, 16, dtype=torch.bfloat16, device=device)
    cu = torch.tensor([0, 4], dtype=torch.int32, device=device)
    ip = torch.tensor([0, 1, 1, 2], dtype=torch.int32, device=device)   # 3 rows for 4 queries
    ix = torch.tensor([1, 0], dtype=torch.int32, device=device)
    with pytest.raises(ValueError):
        A.attn_fwd(q, q, q, cu, cu, 4, 4, 0.25, adj_indptr=ip, adj_indices=ix)
    with pytest.raises(ValueError):
        A.attn_fwd(q, q, q, cu, cu, 4, 4, 0.25, edge_src=ix, edge_dst=ix, adj_indptr=ip, adj_indices=ix)


@pytest.mark.parametrize("dm,h,drop", [(256, 16, False), (512, 32, False), (512, 16, False), (512, 8, False),
                                       (192, 8, False), (192, 8, True)])
def test_esa_node_mode_bf16_train_step(device, dm, h, drop, monkeypatch):
    """ESA in node mode trained bf16-mixed (fp32 parameters under torch.autocast(bfloat16),
    core/train_pretrain.py:753) on the 32 protein-like graphs of configuration 1 as node graphs (9,603 nodes,
    radius edges), layers M-S-M-S-P, MLP 2 x (2 D), through the packed entry: the masked layers run on the
    batch's node plan (forward and backward).  D = 256 with 16 heads (head dim 16); D = 512 with 8 heads (head
    dim 64, the qm9 / unimol YAMLs' dim and heads, core/pretraining_config_qm9.yaml:27-28) and with 16 heads
    (head dim 32, pretraining_config_coconut.yaml:21-22), D = 192 with 8 heads (head dim 24, the rna YAML,
    pretraining_config_rna.yaml:51-54), and D = 512 with 32 heads of 16 as the control of the head-dim-16 kernels
    at that width.  The loss is restricted to the smallest and the largest graph, so the
    fp64 oracle over those two graphs alone gives the embeddings, dX and the parameter gradients.  Bar: bf16,
    scaled by max(1, max |reference|).  At D = 512 and 192 the parameter gradients are checked by their relative L2 error
    (<= 3e-2) and the max-abs bar: a weight gradient sums bf16 products over D-wide rows through five
    bf16-mixed layers, and there the head-dim-16 control reaches the same errors as head dims 32 and 64
    (relative norm 0.7-2.5e-2, mean-abs 0.5-4.3e-3 of max |ref|, by parameter) while each attention call's
    own error is the same at all three head dims (relative 2.2-2.5e-3 for out, dQ, dK, dV).
    With ``drop`` the model trains with the rna YAML's attention dropout (sab / mab 0.08, pma 0.05,
    pretraining_config_rna.yaml:76-78): the seeds the library draws per attention call are recorded in call
    order and the oracle's layers take the same seeds with the two graphs' global token ids."""
    from mind_amd.esa.masked_layers import ESA
    layers = "MSMSP"
    print(f"[node-esa] D={dm} heads={h} head_dim={dm // h}", flush=True)
    gb = generators.protein_like(seed=3)
    sizes = gb.node_counts.astype(np.int64)
    t = int(sizes.sum())
    n = nearest_multiple_of_8(int(sizes.max()) + 1)
    torch.manual_seed(0)
    rates = {"sab_dropout": 0.08, "mab_dropout": 0.08, "pma_dropout": 0.05} if drop else {}
    model = ESA(num_outputs=2, dim_output=dm, dim_hidden=[dm] * len(layers), num_heads=[h] * len(layers),
                layer_types=layers, node_or_edge="node", xformers_or_torch_attn="hip", use_mlps=True,
                mlp_hidden_size=2 * dm, num_mlp_layers=2, mlp_type="standard", **rates)
    model.train()
    seeds = []
    if drop:
        draw = A.draw_dropout_seed

        def record():
            seeds.append(draw())
            return seeds[-1]
        monkeypatch.setattr(A, "draw_dropout_seed", record)
    gen = torch.Generator().manual_seed(1)
    with torch.no_grad():
        for name, prm in model.named_parameters():
            base = (1.0 if name.endswith("weight") else 0.0) if ".ln." in name else 0.0
            prm.copy_(base + (0.1 if ".ln." in name else 0.05) * torch.randn(prm.shape, generator=gen))
    model = model.to(device)
    ei, bm = torch.as_tensor(gb.edge_index).to(device), torch.as_tensor(gb.batch).to(device)
    na = NodeAdjacency.from_edge_index(ei, bm, gb.num_graphs, n)
    x = torch.randn(t, dm, generator=torch.Generator().manual_seed(2))
    xd = x.to(device).requires_grad_(True)
    sel = [int(np.argmin(sizes)), int(np.argmax(sizes))]
    first = np.concatenate([[0], np.cumsum(sizes)])
    rows = np.concatenate([np.arange(first[b], first[b + 1]) for b in sel])
    gg = torch.randn(2, dm, generator=torch.Generator().manual_seed(3))
    ge = torch.randn(rows.size, dm, generator=torch.Generator().manual_seed(4))
    with torch.autocast("cuda", dtype=torch.bfloat16):
        g_emb, enc = model.forward_packed(xd, na)
    rows_d, sel_d = torch.as_tensor(rows).to(device), torch.as_tensor(sel).to(device)
    loss = (g_emb.float().index_select(0, sel_d) * gg.to(device)).sum() + \
        (enc.float().index_select(0, rows_d) * ge.to(device)).sum()
    loss.backward()
    torch.cuda.synchronize()
    # the two graphs' CSR over their own node numbering (graph sel[0]'s nodes first)
    src, dst = gb.edge_index
    local = np.full(t, -1, np.int64)
    local[rows] = np.arange(rows.size)
    keep = local[src] >= 0
    rs, cs = local[src[keep]], local[dst[keep]]
    o = np.lexsort((cs, rs))
    indptr = np.searchsorted(rs[o], np.arange(rows.size + 1))
    adj = (indptr, cs[o])
    cu = np.array([0, sizes[sel[0]], sizes[sel[0]] + sizes[sel[1]]])
    sd = {k: v.detach().cpu().double().requires_grad_(True) for k, v in model.state_dict().items()}
    xr = x.double()[torch.as_tensor(rows)].clone().requires_grad_(True)
    calls = iter(seeds)
    if drop:
        assert len(seeds) == len(layers)   # one attention call per layer
    k_seeds = 2
    seed_ids = np.concatenate([np.arange(b * k_seeds, (b + 1) * k_seeds) for b in sel])   # PMA queries b * k + s

    def drop_of(p, q_ids):
        return (p, next(calls), q_ids, rows) if drop else None
    g_ref, enc_ref = OMod.esa(
        sd, xr, layers, h, 2,
        attn_m=lambda s_, p_, z: OMod.mab_packed(s_, p_, z, z, cu, cu, h, adj=adj, dropout=drop_of(0.08, rows)),
        attn_s=lambda s_, p_, z: OMod.mab_packed(s_, p_, z, z, cu, cu, h, dropout=drop_of(0.08, rows)),
        pool=lambda s_, p_, z: OMod.pma_complete(s_, p_, z, h, 2, cu=cu, max_items=n,
                                                 dropout=drop_of(0.05, seed_ids)))
    ((g_ref * gg.double()).sum() + (enc_ref * ge.double()).sum()).backward()
    assert_bf16_close(g_emb.detach().float().cpu()[sel], g_ref.detach(), grad_scale(g_ref.detach()), "graph emb")
    assert_bf16_close(enc.detach().float().cpu()[torch.as_tensor(rows)], enc_ref.detach(),
                      grad_scale(enc_ref.detach()), "token emb")
    assert_bf16_close(xd.grad.cpu()[torch.as_tensor(rows)], xr.grad, grad_scale(xr.grad), "dX")
    params = dict(model.named_parameters())
    for name in ("encoder.0.sab.mab.fc_q.weight", "encoder.0.sab.mab.fc_k.weight", "encoder.0.norm.ln.weight",
                 "encoder.2.sab.mab.fc_v.bias", "encoder.2.mlp.mlp.0.weight", "decoder.0.pma.S"):
        ref = sd[name].grad
        got = params[name].grad.float().cpu().reshape(ref.shape)
        if dm == 256:
            assert_bf16_close(got, ref, grad_scale(ref), f"d {name}")
        else:
            rel = float((got.double() - ref).norm() / ref.norm())
            assert rel <= 3e-2, f"d {name}: relative L2 error {rel:.3e}"
            assert float((got.double() - ref).abs().max()) <= 2e-2 * grad_scale(ref), f"d {name}: max-abs"
