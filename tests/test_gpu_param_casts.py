"""The one-cast parameter cache of the packed ESA under autocast (mind_amd.esa.linear.param_casts): cached
casts equal p.to(bf16) bit for bit and start 256-byte aligned, and a bf16-mixed forward and backward of the
packed ESA gives the same outputs and gradients, bit for bit, with the cache as with one cast per call."""
import contextlib

import pytest
import torch

from mind_amd import generators
from mind_amd.esa import linear as L
from mind_amd.esa.masked_layers import ESA
from mind_amd.esa.packing import EdgeAdjacency, nearest_multiple_of_8

pytestmark = pytest.mark.gpu


def test_cached_casts_equal_and_aligned(device):
    g = torch.Generator().manual_seed(3)
    ps = [torch.randn(*shape, generator=g).to(device) for shape in [(7,), (130, 3), (512, 512), (1,), (64, 33)]]
    with L.param_casts(ps + [ps[0], None], torch.bfloat16):
        for p in ps:
            c = L.cast_param(p, torch.bfloat16)
            assert c.dtype == torch.bfloat16 and c.shape == p.shape
            assert torch.equal(c.view(torch.int16), p.to(torch.bfloat16).view(torch.int16))
            assert c.data_ptr() % 256 == 0
        other = torch.randn(5, device=device)
        assert torch.equal(L.cast_param(other, torch.bfloat16), other.to(torch.bfloat16))   # not cached: cast
        assert L.cast_param(ps[1], torch.float32) is ps[1]
    c = L.cast_param(ps[2], torch.bfloat16)   # outside: a fresh cast
    assert torch.equal(c, ps[2].to(torch.bfloat16))


def test_esa_train_step_unchanged(device, monkeypatch):
    gb = generators.protein_like(seed=2, num_graphs=4, n_min=40, n_max=120)
    d, h = 128, 8
    n = nearest_multiple_of_8(gb.max_seqlen + 1)
    ei = torch.as_tensor(gb.edge_index).to(device)
    bm = torch.as_tensor(gb.batch).to(device)
    adj = EdgeAdjacency.from_edge_index(ei, bm, gb.num_graphs, n)
    x = adj.pad(torch.randn(gb.num_tokens, d, generator=torch.Generator().manual_seed(5)).to(device))

    def run():
        torch.manual_seed(1)
        model = ESA(num_outputs=2, dim_output=d, dim_hidden=[d] * 3, num_heads=[h] * 3, layer_types="MSP",
                    xformers_or_torch_attn="hip", use_mlps=True, mlp_hidden_size=256, num_mlp_layers=2,
                    mlp_type="standard").to(device)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            emb, enc = model(x, ei, bm, n)
        (emb.float().pow(2).mean() + enc.float().pow(2).mean()).backward()
        return [emb, enc] + [p.grad for p in model.parameters()]

    cached = run()
    monkeypatch.setattr(ESA, "_linear_casts", lambda self: contextlib.nullcontext())
    plain = run()
    assert len(cached) == len(plain)
    for a, b in zip(cached, plain):
        assert (a is None) == (b is None)
        if a is not None:
            assert torch.equal(a, b)
