"""GPU parity of the reference-signature modules (MAB/SAB/PMA, MABFlashVarlen, blocks, ESA) against the oracle.

Weights are the modules' own random initialisation; the oracle reads the same
state_dict and restates the reference block in float64 on the CPU.  Inputs are
fp32, so the modules run the fp32 kernels: the bar is 1e-5 relative
(max-abs <= 1e-5 * max(1, max |reference|)).  Paths that run bf16 by design
(MABFlashVarlen's bf16 cast, esa/mha_flash_varlen.py:147-151) and the bf16
variants use the bf16 bar (max-abs 2e-2, mean-abs 2e-3, same scaling).
"""
import numpy as np
import pytest
import torch

from mind_amd import generators
from mind_amd.esa import masked_layers as ML
from mind_amd.esa.mha import MAB, PMA, SAB
from mind_amd.esa.mha_flash_varlen import MABFlashVarlen, PMAFlashVarlen
from mind_amd.esa.packing import EdgeAdjacency, nearest_multiple_of_8
from oracle import mask as OM
from oracle import modules as OMod
from tests._util import assert_bf16_close, assert_f32_close

pytestmark = pytest.mark.gpu

D, H = 128, 8


def _scale(ref):
    return max(1.0, float(ref.abs().max()))


def _batch(seed=0, num_graphs=5):
    gb, _ = generators.small_molecules(seed=seed, num_graphs=num_graphs)
    n = nearest_multiple_of_8(int(gb.edge_counts.max()) + 1)
    return gb, n


def _padded_tokens(gb, n, seed):
    x = torch.randn(gb.num_graphs, n, D, generator=torch.Generator().manual_seed(seed))
    valid = torch.zeros(gb.num_graphs, n, dtype=torch.bool)
    for b, L in enumerate(gb.edge_counts):
        valid[b, :L] = True
    return x, valid


def _sd(m):
    return {k: v.detach().cpu() for k, v in m.state_dict().items()}


def test_mab_dense_all_positions(device):
    torch.manual_seed(0)
    m = MAB(D, D, D, H).to(device)
    Q = torch.randn(3, 40, D, generator=torch.Generator().manual_seed(1))
    K = torch.randn(3, 56, D, generator=torch.Generator().manual_seed(2))
    got = m(Q.to(device), K.to(device)).cpu()
    ref = OMod.mab_padded(_sd(m), "", Q, K, H)
    assert_f32_close(got, ref, "MAB dense")


@pytest.mark.parametrize("backend", ["xformers", "torch"])
def test_sab_edge_mask_reference_semantics(device, backend):
    """Padded layout with the -99999 edge bias, every row including padding (esa/mha.py:73-77)."""
    gb, n = _batch(1)
    torch.manual_seed(1)
    m = SAB(D, D, H, 0.0, backend).to(device)
    X, _ = _padded_tokens(gb, n, 3)
    ei = torch.as_tensor(gb.edge_index)
    gid = np.repeat(np.arange(gb.num_graphs), gb.edge_counts)
    mask = EdgeAdjacency.from_edge_index(ei.to(device), torch.as_tensor(gb.batch).to(device), gb.num_graphs, n)
    got = m(X.to(device), adj_mask=mask).cpu()
    bias = OM.edge_bias_padded(gb.edge_index, gid, gb.num_graphs, n, dtype=torch.float64)
    ref = OMod.mab_padded(_sd(m), "mab.", X, X, H, bias)
    assert_f32_close(got, ref, f"SAB {backend} edge mask")


def test_sab_edge_mask_packed_hip(device):
    gb, n = _batch(2)
    torch.manual_seed(2)
    m = SAB(D, D, H, 0.0, "hip").to(device)
    X, valid = _padded_tokens(gb, n, 4)
    mask = EdgeAdjacency.from_edge_index(torch.as_tensor(gb.edge_index).to(device),
                                         torch.as_tensor(gb.batch).to(device), gb.num_graphs, n)
    got = m(X.to(device), adj_mask=mask).cpu()
    cu = gb.cu_seqlens
    Xp = X[valid]
    src, dst = gb.edge_index[0], gb.edge_index[1]
    ref_p = OMod.mab_packed(_sd(m), "mab.", Xp, Xp, cu, cu, H, src, dst)
    assert_f32_close(got[valid], ref_p, "SAB hip valid rows")
    # padding rows: attention output 0, then 0 + mish(fc_o(0))
    pad_ref = OMod.mish(OMod._p(_sd(m), "mab.", "fc_o.bias"))
    assert_f32_close(got[~valid], pad_ref.expand(int((~valid).sum()), D), "SAB hip padding rows")


def test_sab_hip_backward(device):
    gb, n = _batch(3, num_graphs=3)
    torch.manual_seed(3)
    m = SAB(D, D, H, 0.0, "hip").to(device)
    X, valid = _padded_tokens(gb, n, 5)
    mask = EdgeAdjacency.from_edge_index(torch.as_tensor(gb.edge_index).to(device),
                                         torch.as_tensor(gb.batch).to(device), gb.num_graphs, n)
    xd = X.to(device).requires_grad_(True)
    g = torch.randn(gb.num_graphs, n, D, generator=torch.Generator().manual_seed(6))
    g[~valid] = 0   # padding rows carry no loss (the oracle has no padding rows)
    m(xd, adj_mask=mask).backward(g.to(device))
    sd = {k: v.detach().cpu().double().requires_grad_(True) for k, v in m.state_dict().items()}
    xr = X.double()[valid].clone().requires_grad_(True)
    cu = gb.cu_seqlens
    ref = OMod.mab_packed(sd, "mab.", xr, xr, cu, cu, H, gb.edge_index[0], gb.edge_index[1])
    ref.backward(g.double()[valid])
    assert_f32_close(xd.grad.cpu()[valid], xr.grad, "dX")
    for name, p in m.named_parameters():
        if name == "mab.fc_k.bias":
            # Exactly zero: a bias shared by every key shifts each score row by a
            # constant, which softmax ignores; the fp32 kernels leave only rounding.
            assert float(sd[name].grad.abs().max()) < 1e-9
        assert_f32_close(p.grad.cpu(), sd[name].grad, f"d{name}")


def test_sab_hip_backward_bf16(device):
    """The bf16-mixed training dtype: bf16 module, bf16 kernels, bf16 bar."""
    gb, n = _batch(3, num_graphs=3)
    torch.manual_seed(3)
    m = SAB(D, D, H, 0.0, "hip").to(device).to(torch.bfloat16)
    X, valid = _padded_tokens(gb, n, 5)
    X = X.to(torch.bfloat16)
    mask = EdgeAdjacency.from_edge_index(torch.as_tensor(gb.edge_index).to(device),
                                         torch.as_tensor(gb.batch).to(device), gb.num_graphs, n)
    xd = X.to(device).requires_grad_(True)
    g = torch.randn(gb.num_graphs, n, D, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    g[~valid] = 0
    m(xd, adj_mask=mask).backward(g.to(device))
    sd = {k: v.detach().cpu().double().requires_grad_(True) for k, v in m.state_dict().items()}
    xr = X.double()[valid].clone().requires_grad_(True)
    cu = gb.cu_seqlens
    ref = OMod.mab_packed(sd, "mab.", xr, xr, cu, cu, H, gb.edge_index[0], gb.edge_index[1])
    ref.backward(g.double()[valid])
    assert_bf16_close(xd.grad.cpu()[valid], xr.grad, _scale(xr.grad), "dX")
    t = int(valid.sum())
    for name, p in m.named_parameters():
        if name == "mab.fc_k.bias":
            # Exactly zero: a bias shared by every key shifts each score row by a
            # constant, which softmax ignores.  The kernel's value is the sum of T
            # bf16-rounded dK rows (unit roundoff 2^-8, |dK| < 1): bound it by four
            # standard deviations of that rounding walk.
            assert float(sd[name].grad.abs().max()) < 1e-9
            assert float(p.grad.abs().max()) <= 4 * 2.0 ** -8 * t ** 0.5, f"d{name} = {p.grad.abs().max()}"
            continue
        assert_bf16_close(p.grad.cpu(), sd[name].grad, _scale(sd[name].grad), f"d{name}")


def test_mab_flash_varlen_path(device):
    gb, n = _batch(4)
    torch.manual_seed(4)
    m = MABFlashVarlen(D, D, D, H).to(device)
    X, _ = _padded_tokens(gb, n, 7)
    Xb = X.to(torch.bfloat16)
    lens = torch.as_tensor(gb.edge_counts, dtype=torch.int32)
    got = m(Xb.to(device), Xb.to(device), seq_lens=lens.to(device)).float().cpu()
    ref = OMod.mab_varlen(_sd(m), "", Xb, Xb, gb.edge_counts, H)
    assert_bf16_close(got, ref, _scale(ref), "MABFlashVarlen varlen")


def test_pma_dense_and_pooled(device):
    gb, n = _batch(5)
    torch.manual_seed(5)
    m = PMA(D, H, 4, 0.0, "hip").to(device)
    X, valid = _padded_tokens(gb, n, 8)
    S = m.S.detach().cpu().repeat(gb.num_graphs, 1, 1)
    got = m(X.to(device)).cpu()                        # reference semantics: all N positions
    ref = OMod.mab_padded(_sd(m), "mab.", S, X, H)
    assert_f32_close(got, ref, "PMA over all positions")
    lens = torch.as_tensor(gb.edge_counts)
    got_v = m(X.to(device), seq_lens=lens.to(device)).cpu()
    cu_q = np.arange(gb.num_graphs + 1) * 4
    ref_v = OMod.mab_packed(_sd(m), "mab.", S.reshape(-1, D), X[valid], cu_q, gb.cu_seqlens, H)
    assert_f32_close(got_v.reshape(-1, D), ref_v, "PMA over valid tokens")
    pf = PMAFlashVarlen(D, H, 4, 0.0).to(device)
    pf.load_state_dict(m.state_dict())
    got_f = pf(X.to(device), seq_lens=lens.to(device)).cpu()   # reference: padded fallback
    assert_f32_close(got_f, ref, "PMAFlashVarlen padded fallback")


def test_esa_hip_packed_backward(device):
    """The "hip" ESA runs packed end to end: gradients of the input (valid rows) and of parameters of every
    stage against autograd through the oracle; the returned embeddings are zero at padding slots."""
    gb, n = _batch(7, num_graphs=6)
    torch.manual_seed(7)
    model = ML.ESA(num_outputs=2, dim_output=D, dim_hidden=[D, D, D], num_heads=[H, H, H], layer_types="MSP",
                   xformers_or_torch_attn="hip", use_mlps=True, mlp_hidden_size=2 * D, num_mlp_layers=2,
                   mlp_type="standard").to(device)
    X, valid = _padded_tokens(gb, n, 17)
    xd = X.to(device).requires_grad_(True)
    ei = torch.as_tensor(gb.edge_index).to(device)
    bm = torch.as_tensor(gb.batch).to(device)
    g_emb, enc = model(xd, ei, bm, n)
    gg = torch.randn(g_emb.shape, generator=torch.Generator().manual_seed(1))
    ge = torch.randn(enc.shape, generator=torch.Generator().manual_seed(2)) * valid[..., None]
    ((g_emb * gg.to(device)).sum() + (enc * ge.to(device)).sum()).backward()
    assert float(enc.detach()[~valid.to(device)].abs().max()) == 0.0

    sd = {k: v.detach().cpu().double().requires_grad_(True) for k, v in model.state_dict().items()}
    cu = gb.cu_seqlens
    src, dst = gb.edge_index[0], gb.edge_index[1]
    xp = X.double()[valid].clone().requires_grad_(True)
    g_ref, enc_ref = OMod.esa(
        sd, xp, "MSP", H, 2,
        attn_m=lambda s_, p_, x: OMod.mab_packed(s_, p_, x, x, cu, cu, H, src, dst),
        attn_s=lambda s_, p_, x: OMod.mab_packed(s_, p_, x, x, cu, cu, H),
        pool=lambda s_, p_, x: OMod.pma_complete(s_, p_, x, H, 2, cu=cu, max_items=n))
    ((g_ref * gg.double()).sum() + (enc_ref * ge.double()[valid]).sum()).backward()
    assert_f32_close(g_emb.detach().cpu(), g_ref.detach(), "ESA graph embedding")
    assert_f32_close(xd.grad.cpu()[valid], xp.grad, "dX (valid rows)")
    params = dict(model.named_parameters())
    for name in ("encoder.0.sab.mab.fc_q.weight", "encoder.1.mlp.mlp.0.weight", "decoder.0.pma.S",
                 "decoder.0.pma.mab.fc_k.weight", "decoder_linear.weight"):
        if name not in params:
            continue
        assert_f32_close(params[name].grad.cpu().reshape(sd[name].grad.shape), sd[name].grad, f"d {name}")


@pytest.mark.parametrize("backend", ["hip", "xformers"])
def test_esa_block_config0_shape(device, backend):
    """M (masked), S, P(1 seed) with pre-norm and standard MLPs on a small-molecule batch."""
    gb, n = _batch(6, num_graphs=8)
    torch.manual_seed(6)
    model = ML.ESA(num_outputs=1, dim_output=D, dim_hidden=[D, D, D], num_heads=[H, H, H], layer_types="MSP",
                   xformers_or_torch_attn=backend, use_mlps=True, mlp_hidden_size=2 * D, num_mlp_layers=2,
                   mlp_type="standard").to(device)
    X, valid = _padded_tokens(gb, n, 9)
    ei = torch.as_tensor(gb.edge_index).to(device)
    bm = torch.as_tensor(gb.batch).to(device)
    g_emb, enc = model(X.to(device), ei, bm, n)
    g_emb, enc = g_emb.cpu(), enc.cpu()
    sd = _sd(model)
    cu = gb.cu_seqlens
    src, dst = gb.edge_index[0], gb.edge_index[1]
    gid = np.repeat(np.arange(gb.num_graphs), gb.edge_counts)
    if backend == "hip":
        g_ref, enc_ref = OMod.esa(
            sd, X.double()[valid], "MSP", H, 2,
            attn_m=lambda s_, p_, x: OMod.mab_packed(s_, p_, x, x, cu, cu, H, src, dst),
            attn_s=lambda s_, p_, x: OMod.mab_packed(s_, p_, x, x, cu, cu, H),
            pool=lambda s_, p_, x: OMod.pma_complete(s_, p_, x, H, 2, cu=cu, max_items=n))
        assert_f32_close(enc[valid], enc_ref, "ESA enc (valid rows)")
    else:
        bias = OM.edge_bias_padded(gb.edge_index, gid, gb.num_graphs, n, dtype=torch.float64)
        g_ref, enc_ref = OMod.esa(
            sd, X.double(), "MSP", H, 2,
            attn_m=lambda s_, p_, x: OMod.mab_padded(s_, p_, x, x, H, bias),
            attn_s=lambda s_, p_, x: OMod.mab_padded(s_, p_, x, x, H),
            pool=lambda s_, p_, x: OMod.pma_complete(s_, p_, x, H, 2))
        assert_f32_close(enc, enc_ref, "ESA enc (all rows)")
    assert_f32_close(g_emb.reshape(g_ref.shape), g_ref, "ESA graph embedding")


def test_esa_hip_without_pma_keeps_padded_shape(device):
    """layer_types without a P (core/pretraining_config_rna.yaml's pattern): ESA.forward returns the head
    applied per token as [B, N, dim_output] (esa/masked_layers.py:929-936), mish(bias) at padding slots, and
    forward_packed the same values packed [T, dim_output]; both against the fp64 oracle."""
    gb, n = _batch(11, num_graphs=5)
    torch.manual_seed(11)
    d_out = 24
    model = ML.ESA(num_outputs=1, dim_output=d_out, dim_hidden=[D, D], num_heads=[H, H], layer_types="MS",
                   xformers_or_torch_attn="hip", use_mlps=True, mlp_hidden_size=2 * D, num_mlp_layers=2,
                   mlp_type="standard").to(device)
    X, valid = _padded_tokens(gb, n, 12)
    ei = torch.as_tensor(gb.edge_index).to(device)
    bm = torch.as_tensor(gb.batch).to(device)
    with torch.no_grad():
        g_emb, enc = model(X.to(device), ei, bm, n)
        adj = EdgeAdjacency.from_edge_index(ei, bm, gb.num_graphs, n)
        g_pk, enc_pk = model.forward_packed(adj.unpad(X.to(device)), adj)
    assert g_emb.shape == (gb.num_graphs, n, d_out) and enc.shape == (gb.num_graphs, n, D)
    assert g_pk.shape == (int(gb.cu_seqlens[-1]), d_out)
    assert torch.equal(adj.unpad(g_emb), g_pk) and torch.equal(adj.unpad(enc), enc_pk)
    g_emb, enc = g_emb.cpu(), enc.cpu()
    sd = _sd(model)
    pad_ref = torch.nn.functional.mish(sd["decoder_linear.bias"].double())
    assert_f32_close(g_emb[~valid], pad_ref.expand(int((~valid).sum()), d_out), "head at padding slots")
    cu = gb.cu_seqlens
    src, dst = gb.edge_index[0], gb.edge_index[1]
    g_ref, enc_ref = OMod.esa(
        sd, X.double()[valid], "MS", H, 2,
        attn_m=lambda s_, p_, x: OMod.mab_packed(s_, p_, x, x, cu, cu, H, src, dst),
        attn_s=lambda s_, p_, x: OMod.mab_packed(s_, p_, x, x, cu, cu, H),
        pool=None)
    assert_f32_close(enc[valid], enc_ref, "ESA enc (valid rows)")
    assert_f32_close(g_emb[valid], g_ref, "ESA per-token head (valid rows)")


def test_state_dict_names_match_reference_layout():
    m = ML.ESA(num_outputs=4, dim_output=32, dim_hidden=[32, 32, 32], num_heads=[2, 2, 2], layer_types="MSP",
               xformers_or_torch_attn="hip", use_mlps=True, mlp_hidden_size=64, mlp_type="gated_mlp")
    names = set(m.state_dict())
    for key in ("encoder.0.sab.mab.fc_q.weight", "encoder.0.norm.ln.weight", "encoder.1.mlp.mlp.0.fc1.weight",
                "decoder.0.pma.S", "decoder.0.pma.mab.fc_o.bias", "decoder_linear.weight"):
        assert key in names, key


def test_config0_full_batch(device):
    """Configuration 0 at its stated size (64 small molecules, seed 0), fp32 end to end: one-hot atom types
    embedded to 128, edge tokens Linear(256 -> 128) over [x_src || x_dst] (core/pretraining_model.py:152-198),
    then the ESA block M(8 heads) - S - PMA(1 seed) on the native packed path, against the fp64 oracle."""
    from mind_amd.edges import edge_gather
    from mind_amd.esa.packing import EdgeAdjacency
    gb, types = generators.small_molecules(seed=0)
    assert gb.num_graphs == 64
    n = nearest_multiple_of_8(gb.max_seqlen + 1)
    torch.manual_seed(0)
    emb, proj = torch.nn.Linear(16, D).to(device), torch.nn.Linear(2 * D, D).to(device)
    model = ML.ESA(num_outputs=1, dim_output=D, dim_hidden=[D, D, D], num_heads=[H, H, H], layer_types="MSP",
                   xformers_or_torch_attn="hip", use_mlps=True, mlp_hidden_size=2 * D, num_mlp_layers=2,
                   mlp_type="standard").to(device)
    onehot = torch.nn.functional.one_hot(torch.as_tensor(types), 16).float()
    ei = torch.as_tensor(gb.edge_index).to(device)
    bm = torch.as_tensor(gb.batch).to(device)
    adj = EdgeAdjacency.from_edge_index(ei, bm, gb.num_graphs, n)
    with torch.no_grad():
        tok = proj(edge_gather(emb(onehot.to(device)), ei[0].int(), ei[1].int()))
        g_emb, enc = model.forward_packed(tok, adj)
        g_pad, enc_pad = model(adj.pad(tok), ei, bm, n)
    assert torch.equal(g_pad, g_emb) and torch.equal(adj.unpad(enc_pad), enc)

    x = onehot.double() @ emb.weight.detach().cpu().double().T + emb.bias.detach().cpu().double()
    src, dst = gb.edge_index
    tok_ref = torch.cat([x[torch.as_tensor(src)], x[torch.as_tensor(dst)]], 1) @ \
        proj.weight.detach().cpu().double().T + proj.bias.detach().cpu().double()
    assert_f32_close(tok.cpu(), tok_ref, "edge tokens")
    cu = gb.cu_seqlens
    g_ref, enc_ref = OMod.esa(
        _sd(model), tok_ref, "MSP", H, 2,
        attn_m=lambda s_, p_, z: OMod.mab_packed(s_, p_, z, z, cu, cu, H, src, dst),
        attn_s=lambda s_, p_, z: OMod.mab_packed(s_, p_, z, z, cu, cu, H),
        pool=lambda s_, p_, z: OMod.pma_complete(s_, p_, z, H, 2, cu=cu, max_items=n))
    assert_f32_close(enc.cpu(), enc_ref, "token embeddings")
    assert_f32_close(g_emb.cpu(), g_ref, "graph embeddings")


def test_mab_with_the_reference_bias_tensor(device):
    """MAB / SAB given the reference's own [B, 1, N, N] mask tensors: the additive 0 / -99999 bias of
    get_adj_mask_from_edge_index_edge (fp32 and its bf16 rounding -99840), the same bias expanded over heads
    [B, H, N, N] (esa/mha.py:73), and a bool mask (True = attend); every row, padding included, against the
    oracle's padded MAB with that bias."""
    gb, n = _batch(11)
    torch.manual_seed(11)
    m = SAB(D, D, H, 0.0, "xformers").to(device)
    X, _ = _padded_tokens(gb, n, 12)
    gid = np.repeat(np.arange(gb.num_graphs), gb.edge_counts)
    bias = OM.edge_bias_padded(gb.edge_index, gid, gb.num_graphs, n, dtype=torch.float64)
    ref = OMod.mab_padded(_sd(m), "mab.", X, X, H, bias)
    xd = X.to(device)
    for what, mask in (("fp32 bias", bias.float()), ("bf16 bias", bias.to(torch.bfloat16)),
                       ("bias over heads", bias.float().expand(-1, H, -1, -1)), ("bool mask", bias == 0)):
        got = m(xd, adj_mask=mask.to(device)).cpu()
        assert_f32_close(got, ref, f"SAB with a {what}")
    mf = MABFlashVarlen(D, D, D, H).to(device)
    mf.load_state_dict(m.mab.state_dict())
    got_f = mf(xd, xd, adj_mask=bias.float().to(device)).cpu()   # the padded SDPA fallback with attn_mask
    assert_f32_close(got_f, OMod.mab_padded(_sd(mf), "", X, X, H, bias), "MABFlashVarlen padded with a bias")
    with pytest.raises(NotImplementedError):
        m(xd, adj_mask=(bias * 0.5 + 1.0).float().to(device))          # a general additive bias
    per_head = (bias == 0).expand(-1, H, -1, -1).clone()
    per_head[:, 0, 0, 0] = ~per_head[:, 0, 0, 0]
    with pytest.raises(NotImplementedError):
        m(xd, adj_mask=per_head.to(device))


def test_torch_library_ops(device):
    """The C-ABI entry points are registered torch operators: torch.ops.esa_hip.* run the same kernels."""
    from mind_amd import edges
    from mind_amd.esa import attention as A
    gb = generators.protein_like(seed=3, num_graphs=3, n_min=30, n_max=60)
    cu = torch.as_tensor(gb.cu_seqlens).to(device)
    t = int(gb.cu_seqlens[-1])
    q, k, v = (torch.randn(t, 16, 16, generator=torch.Generator().manual_seed(i)).to(torch.bfloat16).to(device)
               for i in range(3))
    out, lse = torch.ops.esa_hip.varlen_attn_fwd(q, k, v, cu, cu, gb.max_seqlen, gb.max_seqlen, 0.25, None, None,
                                                 None, None)
    ref, ref_lse = A.attn_fwd(q, k, v, cu, cu, gb.max_seqlen, gb.max_seqlen, 0.25)
    assert torch.equal(out, ref) and torch.equal(lse, ref_lse)
    x = torch.randn(100, 32, device=device)
    src = torch.randint(0, 100, (500,), device=device, dtype=torch.int32)
    dst = torch.randint(0, 100, (500,), device=device, dtype=torch.int32)
    assert torch.equal(torch.ops.esa_hip.edge_gather(x, src, dst), torch.cat([x[src.long()], x[dst.long()]], 1))
    indptr, perm = torch.ops.esa_hip.csr_build(dst, 100)
    y = torch.randn(500, 32, device=device)
    assert torch.equal(torch.ops.esa_hip.csr_segment_sum(y, indptr, perm), edges.segment_sum_csr(y, indptr, perm))
