"""ESA forwards captured into a HIP graph (mind_amd.esa.graphs.GraphedForward) against the same forwards run
eagerly, bit for bit.

Each test replays the graph for two sets of input values of the captured shapes (and the first set again),
with eager forwards and host synchronisations between the replays, and compares every replay with the eager
forward of the same inputs: every kernel on these paths is deterministic, so a replay must reproduce the eager
bits exactly.  Cases: configuration 0's pipeline (one-hot atom types -> Linear -> [x_src || x_dst] -> Linear ->
ESA M-S-P in fp32, the edge-mask plan built inside the graph), and ESA in node mode under bf16 autocast (the
node plan built inside the graph).
"""
import numpy as np
import pytest
import torch

from mind_amd import _lib, generators
from mind_amd.edges import edge_gather
from mind_amd.esa.graphs import GraphedForward
from mind_amd.esa.masked_layers import ESA
from mind_amd.esa.packing import EdgeAdjacency, nearest_multiple_of_8

pytestmark = pytest.mark.gpu


def _replays_match(gf, eager, inputs_list):
    for inputs in inputs_list + inputs_list[:1]:
        ref = eager(*inputs)
        torch.cuda.synchronize()
        ref = tuple(r.clone() for r in ref)
        got = gf(*inputs)
        torch.cuda.synchronize()
        for g, r in zip(got, ref):
            assert g.shape == r.shape and g.dtype == r.dtype
            assert torch.equal(g, r), f"replay differs from eager by {float((g.float() - r.float()).abs().max())}"
        eager(*inputs)   # eager work between replays


def test_edge_token_block_fp32(device):
    gb, types = generators.small_molecules(seed=3, num_graphs=16)
    d, h = 128, 8
    torch.manual_seed(0)
    emb, proj = torch.nn.Linear(16, d).to(device), torch.nn.Linear(2 * d, d).to(device)
    model = ESA(num_outputs=1, dim_output=d, dim_hidden=[d, d, d], num_heads=[h, h, h], layer_types="MSP",
                xformers_or_torch_attn="hip", use_mlps=True, mlp_hidden_size=2 * d, num_mlp_layers=2,
                mlp_type="standard").to(device).eval()
    n = nearest_multiple_of_8(gb.max_seqlen + 1)

    def forward(types_d, ei, bm):
        with torch.no_grad():
            onehot = torch.nn.functional.one_hot(types_d, 16).float()
            tok = proj(edge_gather(emb(onehot), ei[0].int(), ei[1].int()))
            adj = EdgeAdjacency.from_edge_index(ei, bm, gb.num_graphs, n)
            return model(adj.pad(tok), ei, bm, n)

    ei = torch.as_tensor(gb.edge_index).to(device)
    bm = torch.as_tensor(gb.batch).to(device)
    a = torch.as_tensor(types).to(device)
    b = torch.as_tensor(np.random.default_rng(9).integers(0, 16, size=types.size)).to(device)
    gf = GraphedForward(forward, a, ei, bm)
    _replays_match(gf, forward, [(a, ei, bm), (b, ei, bm)])
    with pytest.raises(ValueError):
        gf(a[:-1], ei, bm)


def test_node_mode_bf16_autocast(device):
    gb = generators.protein_like(seed=5, num_graphs=6, n_min=40, n_max=160)
    counts = np.asarray(gb.node_counts)
    nb, dm, h = gb.num_graphs, 64, 4
    n = nearest_multiple_of_8(int(counts.max()) + 1)
    torch.manual_seed(2)
    model = ESA(num_outputs=2, dim_output=dm, dim_hidden=[dm] * 4, num_heads=[h] * 4, layer_types="MSMP",
                node_or_edge="node", xformers_or_torch_attn="hip", use_mlps=True, mlp_hidden_size=2 * dm,
                num_mlp_layers=2, mlp_type="standard").to(device).eval()
    ei = torch.as_tensor(gb.edge_index).to(device)
    bm = torch.as_tensor(gb.batch).to(device)

    def forward(x, ei_, bm_):
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, cache_enabled=False):
            return model(x, ei_, bm_, n)

    g = torch.Generator().manual_seed(4)
    xa = torch.randn(nb, n, dm, generator=g).to(device)
    xb = torch.randn(nb, n, dm, generator=g).to(device)
    gf = GraphedForward(forward, xa, ei, bm)
    _replays_match(gf, forward, [(xa, ei, bm), (xb, ei, bm)])


def test_capture_refused_while_profiling(device):
    _lib.profile_enable(True)
    try:
        with pytest.raises(RuntimeError, match="profiling"):
            GraphedForward(lambda x: x + 1, torch.zeros(4, device=device))
    finally:
        _lib.profile_enable(False)
