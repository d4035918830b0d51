"""Configuration 4 at its stated size: the ESA encoder stack M-M-S-S-M-M-S-S-P(4 seeds), D = 512, 32 heads,
MLP hidden 2048 (two layers), pre-norm, trained bf16-mixed (fp32 parameters under torch.autocast(bfloat16),
core/train_pretrain.py:753) on the 131,072-token budget batch of the protein-like generator.

The whole batch runs forward and backward through the packed native entry (ESA.forward_packed).  The loss is
restricted to the smallest and the largest graph, so the fp64 oracle (oracle.modules.esa over those two
graphs' tokens only: graphs never exchange information in ESA) gives the graph embeddings, the token
embeddings, the input gradient and every parameter gradient of the same loss.  Bar: bf16 (max-abs 2e-2,
mean-abs 2e-3), scaled by max(1, max |reference|).  The path checked includes the fused LayerNorm
(bf16 GEMM copy and residual pass-through), the fp32-residual MAB epilogue, the parameter casts inside the
Linear functions, the fused Mish-backward bias gradient of the 2048-wide MLP layer and the dense and
edge-masked bf16 attention kernels at 32 heads.
"""
import numpy as np
import pytest
import torch

from mind_amd import generators
from mind_amd.esa.masked_layers import ESA
from mind_amd.esa.packing import EdgeAdjacency, nearest_multiple_of_8
from oracle import modules as OMod
from tests._util import assert_bf16_close, grad_scale

pytestmark = pytest.mark.gpu

D, H, LAYERS, HIDDEN, SEEDS = 512, 32, "MMSSMMSSP", 2048, 4


def _model(device):
    torch.manual_seed(0)
    model = ESA(num_outputs=SEEDS, dim_output=D, dim_hidden=[D] * len(LAYERS), num_heads=[H] * len(LAYERS),
                layer_types=LAYERS, xformers_or_torch_attn="hip", use_mlps=True, mlp_hidden_size=HIDDEN,
                num_mlp_layers=2, mlp_type="standard")
    g = torch.Generator().manual_seed(1)
    with torch.no_grad():
        for name, prm in model.named_parameters():
            if ".ln." in name:   # LayerNorm affine parameters away from (1, 0), so they matter
                prm.copy_((1.0 if name.endswith("weight") else 0.0) + 0.1 * torch.randn(prm.shape, generator=g))
            elif prm.dim() >= 2 or name.endswith(".S"):
                prm.copy_(0.02 * torch.randn(prm.shape, generator=g))
            else:
                prm.copy_(0.02 * torch.randn(prm.shape, generator=g))
    return model.to(device)


def test_config4_stack_train_step(device):
    gb = generators.protein_budget(seed=0, token_budget=131072)
    t = gb.num_tokens
    n = nearest_multiple_of_8(gb.max_seqlen + 1)
    model = _model(device)
    ei = torch.as_tensor(gb.edge_index).to(device)
    bm = torch.as_tensor(gb.batch).to(device)
    adj = EdgeAdjacency.from_edge_index(ei, bm, gb.num_graphs, n)
    x = torch.randn(t, D, generator=torch.Generator().manual_seed(2))
    xd = x.to(device).requires_grad_(True)
    sel = [int(np.argmin(gb.edge_counts)), int(np.argmax(gb.edge_counts))]
    cu_all = gb.cu_seqlens
    rows = np.concatenate([np.arange(cu_all[b], cu_all[b + 1]) for b in sel])
    gg = torch.randn(2, D, generator=torch.Generator().manual_seed(3))
    ge = torch.randn(rows.size, D, generator=torch.Generator().manual_seed(4))
    print(f"[config4] {gb.num_graphs} graphs, {t} tokens; checking graphs {sel} "
          f"({[int(gb.edge_counts[b]) for b in sel]} tokens)", flush=True)

    with torch.autocast("cuda", dtype=torch.bfloat16):
        g_emb, enc = model.forward_packed(xd, adj)
    rows_d = torch.as_tensor(rows).to(device)
    sel_d = torch.as_tensor(sel).to(device)
    loss = (g_emb.float().index_select(0, sel_d) * gg.to(device)).sum() + \
        (enc.float().index_select(0, rows_d) * ge.to(device)).sum()
    loss.backward()
    torch.cuda.synchronize()
    assert torch.isfinite(g_emb.float()).all() and torch.isfinite(enc.float()).all()
    print("[config4] GPU step done", flush=True)

    sd = {k: v.detach().cpu().double().requires_grad_(True) for k, v in model.state_dict().items()}
    lens = [int(gb.edge_counts[b]) for b in sel]
    cu = np.array([0, lens[0], lens[0] + lens[1]])
    src, dst = gb.edge_index[0][rows], gb.edge_index[1][rows]
    xr = x.double()[torch.as_tensor(rows)].clone().requires_grad_(True)
    g_ref, enc_ref = OMod.esa(
        sd, xr, LAYERS, H, 2,
        attn_m=lambda s_, p_, z: OMod.mab_packed(s_, p_, z, z, cu, cu, H, src, dst),
        attn_s=lambda s_, p_, z: OMod.mab_packed(s_, p_, z, z, cu, cu, H),
        pool=lambda s_, p_, z: OMod.pma_complete(s_, p_, z, H, 2, cu=cu, max_items=n))
    ((g_ref * gg.double()).sum() + (enc_ref * ge.double()).sum()).backward()
    print("[config4] oracle done", flush=True)

    got_g = g_emb.detach().float().cpu()[sel]
    got_e = enc.detach().float().cpu()[torch.as_tensor(rows)]
    assert_bf16_close(got_g, g_ref.detach(), grad_scale(g_ref.detach()), "graph embeddings")
    assert_bf16_close(got_e, enc_ref.detach(), grad_scale(enc_ref.detach()), "token embeddings")
    assert_bf16_close(xd.grad.cpu()[torch.as_tensor(rows)], xr.grad, grad_scale(xr.grad), "dX")
    others = np.setdiff1d(np.arange(t), rows)
    assert float(xd.grad.cpu()[torch.as_tensor(others)].abs().max()) == 0.0   # graphs outside the loss
    params = dict(model.named_parameters())
    for name in ("encoder.0.sab.mab.fc_q.weight", "encoder.0.sab.mab.fc_v.bias", "encoder.1.norm.ln.weight",
                 "encoder.2.mlp.mlp.0.bias", "encoder.2.mlp.mlp.0.weight", "encoder.3.norm_mlp.ln.bias",
                 "encoder.4.sab.mab.fc_o.weight", "encoder.7.mlp.mlp.2.weight", "decoder.0.pma.S",
                 "decoder.0.pma.mab.fc_k.weight", "decoder.0.mlp.mlp.0.bias", "decoder_linear.weight"):
        ref = sd[name].grad
        assert_bf16_close(params[name].grad.float().cpu().reshape(ref.shape), ref, grad_scale(ref), f"d {name}")
