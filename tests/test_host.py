"""Host-side logic that needs no GPU: generators and the EdgeAdjacency descriptor."""
import numpy as np
import pytest
import torch

from mind_amd import generators
from mind_amd.esa.packing import EdgeAdjacency, cu_seqlens_from_counts, nearest_multiple_of_8
from oracle import packing as OP


def test_radius_edges_definition():
    rng = np.random.default_rng(0)
    pos = rng.normal(scale=2.0, size=(40, 3))
    e = generators.radius_edges(pos, 3.0)
    d = np.linalg.norm(pos[:, None] - pos[None], axis=-1)
    want = {(j, i) for i in range(40) for j in range(40) if i != j and d[j, i] <= 3.0}
    assert set(map(tuple, e.T.tolist())) == want
    # ordered by target then source
    keys = e[1] * 1000 + e[0]
    assert np.all(np.diff(keys) > 0)


def test_radius_edges_cap_keeps_nearest():
    rng = np.random.default_rng(1)
    pos = rng.normal(scale=1.0, size=(60, 3))
    e = generators.radius_edges(pos, 10.0, cap=5)
    counts = np.bincount(e[1], minlength=60)
    assert np.all(counts == 5)
    d = np.linalg.norm(pos[:, None] - pos[None], axis=-1)
    for i in range(60):
        kept = e[0][e[1] == i]
        order = np.lexsort((np.arange(60), d[i]))
        order = order[order != i][:5]
        assert set(kept) == set(order)


def test_generators_are_deterministic_and_consistent():
    a = generators.protein_like(seed=3, num_graphs=4)
    b = generators.protein_like(seed=3, num_graphs=4)
    assert np.array_equal(a.edge_index, b.edge_index)
    assert a.num_tokens == int(a.edge_counts.sum()) == a.cu_seqlens[-1]
    gid_of_edge = a.batch[a.edge_index[0]]
    assert np.array_equal(gid_of_edge, np.repeat(np.arange(4), a.edge_counts))
    assert np.all(a.batch[a.edge_index[0]] == a.batch[a.edge_index[1]])
    assert not np.any(a.edge_index[0] == a.edge_index[1])
    c = generators.protein_budget(seed=1, token_budget=20000)
    assert c.num_tokens <= 20000
    # node budget (the node-mode line): the node count stays within the budget and the next graph would exceed
    # it; the edge-budget batch with the same seed is the same sequence of graphs cut at another point
    d = generators.protein_budget(seed=1, token_budget=5000, count="nodes")
    assert int(d.node_counts.sum()) <= 5000 and len(d.node_counts) >= 2
    assert np.array_equal(d.node_counts, c.node_counts[: len(d.node_counts)]) or \
        np.array_equal(c.node_counts, d.node_counts[: len(c.node_counts)])
    with pytest.raises(ValueError):
        generators.protein_budget(seed=1, count="graphs")
    src, dst = generators.block_local_edges(0, num_nodes=4096, num_edges=10000)
    assert np.all(src // 512 == dst // 512) and src.max() < 4096


def test_edge_adjacency_descriptor_cpu():
    gb, _ = generators.small_molecules(seed=2, num_graphs=5)
    n = nearest_multiple_of_8(int(gb.edge_counts.max()) + 1)
    ei = torch.as_tensor(gb.edge_index)
    m = EdgeAdjacency.from_edge_index(ei, torch.as_tensor(gb.batch), gb.num_graphs, n)
    assert np.array_equal(m.cu_seqlens.numpy(), gb.cu_seqlens)
    gid = np.repeat(np.arange(gb.num_graphs), gb.edge_counts)
    assert np.array_equal(m.position.numpy(), OP.positions(gid))
    x = torch.randn(gb.num_graphs, n, 7)
    packed = m.unpad(x)
    dense, valid = OP.to_dense_batch(packed, gid, gb.num_graphs, n)
    assert torch.equal(dense[valid], packed)
    assert torch.equal(m.pad(packed)[valid], packed) and torch.all(m.pad(packed)[~valid] == 0)
    src, dst = m.padded_nodes()
    pad_ids = torch.cat([src[(~valid).reshape(-1)], dst[(~valid).reshape(-1)]])
    assert torch.all(pad_ids < 0) and pad_ids.unique().numel() == pad_ids.numel()
    assert torch.equal(cu_seqlens_from_counts(torch.tensor([2, 0, 3])), torch.tensor([0, 2, 2, 5], dtype=torch.int32))


def test_split_count_rule():
    """Split-K chunk count: largest power of two <= 32 with >= 4096-token chunks and <= 2^24 fp32 partials."""
    from mind_amd.esa.linear import split_count
    assert split_count(131072, 512, 512) == 32
    assert split_count(131072, 2048, 512) == 16
    assert split_count(131072, 1536, 512) == 16
    assert split_count(8191, 512, 512) == 1
    assert split_count(8192, 512, 512) == 2
    assert split_count(10 ** 6, 4096, 4096) == 1
    for t, o, i in ((131072, 512, 512), (50000, 256, 128), (4096, 64, 64)):
        s = split_count(t, o, i)
        assert s & (s - 1) == 0 and s <= 32 and (s == 1 or (t // s >= 4096 and s * o * i <= 2 ** 24))


def test_block_functions_on_cpu_tensors():
    """On CPU tensors the block helpers are the plain torch expressions (the HIP kernels take device memory)."""
    from mind_amd.esa.activations import Mish, mab_epilogue, mish
    from mind_amd.esa.layer_norm import layer_norm
    from mind_amd.esa.linear import linear, qkv_projection
    torch.manual_seed(0)
    fc = torch.nn.Linear(8, 8)
    o, x = torch.randn(5, 8), torch.randn(5, 8)
    assert torch.allclose(mab_epilogue(o, fc), o + torch.nn.functional.mish(fc(o)))
    assert torch.allclose(mab_epilogue(o, fc, x), x + o + torch.nn.functional.mish(fc(o)))
    assert torch.allclose(mish(o, x), x + torch.nn.functional.mish(o))
    assert torch.allclose(Mish()(o), torch.nn.functional.mish(o))
    assert torch.allclose(linear(o, fc.weight, fc.bias), fc(o))
    fcs = [torch.nn.Linear(8, 8) for _ in range(3)]
    q, k, v = qkv_projection(*fcs, o, x)
    assert torch.allclose(q, fcs[0](o)) and torch.allclose(k, fcs[1](x)) and torch.allclose(v, fcs[2](x))
    ln = torch.nn.LayerNorm(8, eps=1e-8)
    y, y_lp = layer_norm(o, ln, full=True, lowp=True)
    assert torch.allclose(y, ln(o)) and y_lp is None
    _, _, xr = layer_norm(o, ln, full=False, lowp=True, passthrough=True)
    assert xr is o


@pytest.mark.parametrize("num_layers,use_ln", [(1, False), (2, False), (3, False), (3, True)])
def test_small_mlp_walks_every_layer_once(num_layers, use_ln):
    """SmallMLP.forward pairs each Linear with a following Mish (linear_mish) and applies the rest one by one:
    on CPU tensors its output equals the Sequential's, whatever the layer pattern."""
    from mind_amd.esa.mlp_utils import SmallMLP
    torch.manual_seed(num_layers)
    mlp = SmallMLP(12, 20, 8, num_layers=num_layers, use_ln=use_ln)
    x = torch.randn(5, 12)
    assert torch.allclose(mlp(x), mlp.mlp(x), atol=1e-6)


def test_small_mlp_keeps_module_hooks():
    """A Linear or Mish carrying forward hooks is called as a module (its hooks fire), not fused away."""
    from mind_amd.esa.mlp_utils import SmallMLP
    torch.manual_seed(0)
    mlp = SmallMLP(12, 20, 8, num_layers=3)
    seen = []
    mlp.mlp[1].register_forward_hook(lambda m, i, o: seen.append("mish1"))
    mlp.mlp[2].register_forward_pre_hook(lambda m, i: seen.append("linear2"))
    x = torch.randn(5, 12)
    assert torch.allclose(mlp(x), mlp.mlp(x), atol=1e-6)
    assert seen.count("mish1") == 2 and seen.count("linear2") == 2


def test_scatter_add_backward_drops_out_of_range_exactly():
    """Edges whose index is outside [0, dim_size) get a zero gradient even when the clamped row holds Inf."""
    from mind_amd.edges import _ScatterAdd
    index = torch.tensor([0, 5, -1, 1], dtype=torch.int32)
    ctx = type("Ctx", (), {})()
    ctx.saved_tensors = (index,)
    ctx.dim_size = 2
    g = torch.tensor([[float("inf")], [2.0]])
    grad = _ScatterAdd.backward(ctx, g)[0]
    assert grad[1].item() == 0.0 and grad[2].item() == 0.0 and grad[3].item() == 2.0


def _radix_pass_model(keys, vals, shift, tile=4096, threads=256, waves=4, bits=8):
    """numpy model of one pass of esa_csr_build's radix sort, step by step as the kernels take it: digit
    counts per tile, their exclusive scan in (digit, tile) order, then each element's slot = the scan entry
    + elements of the same digit in earlier rounds + in earlier waves of its round + in earlier lanes of its
    wave (the ballot match)."""
    n = keys.size
    nb = -(-n // tile)
    dig = (keys >> shift) & ((1 << bits) - 1)
    hist = np.zeros((1 << bits, nb), np.int64)
    for b in range(nb):
        hist[:, b] = np.bincount(dig[b * tile:(b + 1) * tile], minlength=1 << bits)
    offs = np.concatenate([[0], np.cumsum(hist.reshape(-1))])[:-1].reshape(hist.shape)
    out_k, out_v = np.empty_like(keys), np.empty_like(vals)
    for b in range(nb):
        run = offs[:, b].copy()
        for j in range(tile // threads):
            lo = b * tile + j * threads
            d = dig[lo:lo + threads]
            wcnt = np.zeros((waves, 1 << bits), np.int64)
            slots = []
            for t in range(d.size):
                w, lane = divmod(t, 64)
                same = d[w * 64:w * 64 + lane] == d[t]          # lanes below with the same digit
                slots.append((w, int(same.sum())))
            for t in range(d.size):
                wcnt[t // 64, d[t]] += 1
            for t in range(d.size):
                w, below = slots[t]
                pos = run[d[t]] + wcnt[:w, d[t]].sum() + below
                out_k[pos], out_v[pos] = keys[lo + t], vals[lo + t]
            run += wcnt.sum(0)
    return out_k, out_v


def test_radix_csr_order_is_stable():
    """The kernels' slot rule leaves (key, edge id) sorted by key with ties in ascending edge id: the model
    of the passes equals numpy's stable argsort on keys with repeated values across several tiles."""
    rng = np.random.default_rng(0)
    n_keys = 600
    keys = rng.integers(0, n_keys, size=9000).astype(np.int64)
    keys[::7] = 5                                  # a heavy key spread over every tile
    k, v = keys.copy(), np.arange(keys.size)
    for shift in (0, 8):                          # 600 < 2^16: two 8-bit passes
        k, v = _radix_pass_model(k, v, shift)
    assert np.array_equal(v, np.argsort(keys, kind="stable"))


def test_torch_library_ops_have_fake_implementations():
    """torch.ops.esa_hip.* are registered with shape functions: they trace under FakeTensorMode (no GPU)."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    import mind_amd.edges  # noqa: F401
    import mind_amd.esa.attention  # noqa: F401
    with FakeTensorMode():
        q = torch.empty(40, 4, 16, dtype=torch.bfloat16)
        cu = torch.empty(3, dtype=torch.int32)
        out, lse = torch.ops.esa_hip.varlen_attn_fwd(q, q, q, cu, cu, 20, 20, 0.25, None, None, None, None)
        assert out.shape == q.shape and lse.shape == (4, 40) and lse.dtype == torch.float32
        dq, dk, dv = torch.ops.esa_hip.varlen_attn_bwd(q, q, q, q, q, lse, cu, cu, 20, 20, 0.25, None, None, None,
                                                       None)
        assert dq.shape == dk.shape == dv.shape == q.shape
        x = torch.empty(10, 8)
        idx = torch.empty(30, dtype=torch.int32)
        assert torch.ops.esa_hip.edge_gather(x, idx, idx).shape == (30, 16)
        ip, perm = torch.ops.esa_hip.csr_build(idx, 10)
        assert ip.shape == (11,) and perm.shape == (30,)
        assert torch.ops.esa_hip.csr_segment_sum(torch.empty(30, 8), ip, perm).shape == (10, 8)
