"""GPU parity of the device-side batch assembly: the token-budget packer and the packed-set descriptors
(cu_seqlens, slots, node CSR), bit-exact against the oracle."""
import numpy as np
import pytest
import torch

from mind_amd import generators
from mind_amd.esa.packing import EdgeAdjacency, NodeAdjacency, token_budget_batches
from oracle import packing as OP
from tests._util import node_graph

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("g,budget,hi", [(1, 8, 5), (7, 8, 12), (1000, 65536, 3000), (100_000, 65536, 5000),
                                         (5000, 0, 3), (3000, 10, 30)])
def test_token_budget_pack_matches_greedy_rule(device, g, budget, hi):
    rng = np.random.default_rng(g + budget)
    counts = rng.integers(0, hi, size=g).astype(np.int32)
    counts[::17] = 0                       # graphs without edges
    if g > 3:
        counts[2] = budget + 7             # an oversize graph: a batch of its own
    bog, start, num = token_budget_batches(torch.as_tensor(counts).to(device), budget)
    ref = OP.token_budget_batches(counts, budget)
    n = int(num)
    assert n == len(ref)
    ref_of = np.empty(g, np.int32)
    for b, gs in enumerate(ref):
        ref_of[gs] = b
    assert np.array_equal(bog.cpu().numpy(), ref_of)
    assert np.array_equal(start.cpu().numpy()[: n + 1], np.array([b[0] for b in ref] + [g], np.int32))


def test_token_budget_pack_reproduces_the_generator_batch(device):
    """The configuration-2 generator draws graphs until the next would pass 65,536 edge tokens: packing its
    graphs' edge counts plus that one more graph gives exactly one full batch of them."""
    gb = generators.protein_budget(seed=0, token_budget=65536)
    counts = np.concatenate([gb.edge_counts, [65536]]).astype(np.int32)
    bog, start, num = token_budget_batches(torch.as_tensor(counts).to(device), 65536)
    assert int(num) == 2 and int(start[1]) == gb.num_graphs


def test_edge_descriptors_bit_exact(device):
    """EdgeAdjacency built on the device (no host synchronisation): cu_seqlens and each token's slot equal
    the oracle's closed form, and padding / unpadding round-trips through to_dense_batch's layout."""
    gb = generators.protein_budget(seed=1, token_budget=65536)
    n = OP.nearest_multiple_of_8(int(gb.edge_counts.max()) + 1)
    ei = torch.as_tensor(gb.edge_index).to(device)
    adj = EdgeAdjacency.from_edge_index(ei, torch.as_tensor(gb.batch).to(device), gb.num_graphs, n)
    gid = np.repeat(np.arange(gb.num_graphs), gb.edge_counts)
    assert np.array_equal(adj.cu_seqlens.cpu().numpy(), OP.cu_seqlens(gb.edge_counts))
    assert np.array_equal(adj.position.cpu().numpy(), OP.positions(gid))
    x = torch.randn(gb.num_tokens, 8)
    ref_pad, _ = OP.to_dense_batch(x, gid, gb.num_graphs, n)
    assert torch.equal(adj.pad(x.to(device)).cpu(), ref_pad)
    assert torch.equal(adj.unpad(ref_pad.to(device)).cpu(), x)


def test_node_descriptors_bit_exact(device):
    sizes = [13, 1, 40, 7, 22]
    ei, bm = node_graph(31, sizes)
    na = NodeAdjacency.from_edge_index(torch.as_tensor(ei).to(device), torch.as_tensor(bm).to(device), len(sizes),
                                       48)
    t = len(bm)
    assert np.array_equal(na.cu_seqlens.cpu().numpy(), OP.cu_seqlens(sizes))
    assert np.array_equal(na.position.cpu().numpy(), OP.positions(bm))
    order = np.lexsort((ei[1], ei[0]))
    assert np.array_equal(na.indptr.cpu().numpy(), OP.cu_seqlens(np.bincount(ei[0], minlength=t)))
    assert np.array_equal(na.indices.cpu().numpy(), ei[1][order].astype(np.int32))
