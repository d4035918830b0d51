"""esa_varlen_attn_fwd_noalloc (the forward with the library's static per-GPU scratch, for callers that cannot
allocate) against esa_varlen_attn_fwd on the same inputs: bit-equal outputs and lse (the same kernels), on two
calls in a row, the second with a smaller input, for the dense bf16, edge-masked bf16, node-mode and fp32
paths; a shape beyond the scratch is refused before any launch."""
import numpy as np
import pytest
import torch

from mind_amd import _lib, generators
from mind_amd.esa import attention as A
from mind_amd.esa.packing import NodeAdjacency
from tests._util import node_graph, seeded_normal

pytestmark = pytest.mark.gpu

H, D = 16, 16


def _case(device, gb, seed, dtype, mask):
    cu = torch.as_tensor(gb.cu_seqlens).to(device)
    t = int(gb.cu_seqlens[-1])
    q, k, v = (seeded_normal((t, H, D), seed + i, dtype).to(device) for i in range(3))
    kw = {}
    if mask == "edge":
        kw = {"edge_src": torch.as_tensor(gb.edge_index[0].astype(np.int32)).to(device),
              "edge_dst": torch.as_tensor(gb.edge_index[1].astype(np.int32)).to(device)}
    return q, k, v, cu, int(gb.max_seqlen), kw


def _compare(device, q, k, v, cu, mx, kw):
    ref_o, ref_l = A.attn_fwd(q, k, v, cu, cu, mx, mx, 0.25, **kw)
    out = torch.full_like(q, float("nan"))
    lse = torch.full((q.shape[1], q.shape[0]), float("nan"), device=device)
    A.attn_fwd_noalloc(q, k, v, cu, cu, mx, mx, 0.25, out, lse, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_o)
    assert torch.equal(lse, ref_l)


@pytest.mark.parametrize("dtype,mask", [(torch.bfloat16, "none"), (torch.bfloat16, "edge"), (torch.float32, "none"),
                                        (torch.float32, "edge")])
def test_noalloc_forward_equals_allocating_forward(device, dtype, mask):
    big = generators.protein_like(seed=0) if mask == "none" else generators.protein_budget(seed=0, token_budget=65536)
    small = generators.protein_like(seed=3, num_graphs=5, n_min=40, n_max=150)
    for gb, seed in ((big, 11), (small, 12)):   # the second call is smaller: stale scratch must not matter
        print(f"[noalloc] {dtype} mask={mask} tokens={int(gb.cu_seqlens[-1])}", flush=True)
        _compare(device, *_case(device, gb, seed, dtype, mask))


@pytest.mark.parametrize("dtype,heads", [(torch.float32, 16), (torch.bfloat16, 32)])
def test_noalloc_edge_mask_at_the_documented_limit(device, dtype, heads):
    """131,072 edge tokens (configuration 4's batch), the size the scratch is documented to cover for every
    mask kind: the edge-masked forward fits (fp32 reserves only the plan sections its kernels read) and equals
    the allocating forward; then a small call."""
    lib = _lib.load()
    big = generators.protein_budget(seed=4, token_budget=131072)
    small = generators.protein_like(seed=5, num_graphs=4, n_min=40, n_max=120)
    for gb, seed in ((big, 21), (small, 22)):
        t = int(gb.cu_seqlens[-1])
        n = _lib.ctypes.c_size_t(0)
        _lib.check(lib.esa_varlen_attn_workspace_size(t, t, heads, D, A._dtype_code(torch.empty(0, dtype=dtype)),
                                                      _lib.ESA_MASK_EDGE, 0, 0, _lib.ctypes.byref(n)), "ws")
        assert n.value <= int(lib.esa_noalloc_scratch_bytes())
        print(f"[noalloc] {dtype} edge heads={heads} tokens={t} scratch={n.value}", flush=True)
        cu = torch.as_tensor(gb.cu_seqlens).to(device)
        q, k, v = (seeded_normal((t, heads, D), seed + i, dtype).to(device) for i in range(3))
        kw = {"edge_src": torch.as_tensor(gb.edge_index[0].astype(np.int32)).to(device),
              "edge_dst": torch.as_tensor(gb.edge_index[1].astype(np.int32)).to(device)}
        _compare(device, q, k, v, cu, int(gb.max_seqlen), kw)


@pytest.mark.parametrize("hd", [24, 32, 64])
@pytest.mark.parametrize("mask", ["none", "edge", "node"])
def test_noalloc_wide_heads(device, hd, mask):
    """Head dims 24 / 32 / 64 (the dense MFMA kernels for wide heads, the gather kernels over the edge-mask plan and
    over a node CSR): the no-allocation forward equals the allocating one, two calls in a row, the second
    smaller."""
    heads = 192 // hd if hd == 24 else 256 // hd
    cases = ((generators.protein_like(seed=1, num_graphs=6), 31), (generators.protein_like(seed=2, num_graphs=2), 32))
    for gb, seed in cases:
        t = int(gb.cu_seqlens[-1])
        print(f"[noalloc] wide hd={hd} mask={mask} tokens={t}", flush=True)
        cu = torch.as_tensor(gb.cu_seqlens).to(device)
        q, k, v = (seeded_normal((t, heads, hd), seed + i, torch.bfloat16).to(device) for i in range(3))
        kw = {}
        if mask == "edge":
            kw = {"edge_src": torch.as_tensor(gb.edge_index[0].astype(np.int32)).to(device),
                  "edge_dst": torch.as_tensor(gb.edge_index[1].astype(np.int32)).to(device)}
        elif mask == "node":
            ei, bm = node_graph(seed, [40, 70, 25])
            na = NodeAdjacency.from_edge_index(torch.as_tensor(ei).to(device), torch.as_tensor(bm).to(device), 3, 70)
            t = len(bm)
            cu = na.cu_seqlens
            q, k, v = (seeded_normal((t, heads, hd), seed + i, torch.bfloat16).to(device) for i in range(3))
            kw = {"adj_indptr": na.indptr, "adj_indices": na.indices}
        _compare(device, q, k, v, cu, int(gb.max_seqlen), kw)


@pytest.mark.parametrize("dtype,hd,mask", [(torch.bfloat16, 16, "none"), (torch.bfloat16, 24, "none"),
                                           (torch.bfloat16, 16, "edge"), (torch.float32, 16, "none")])
def test_noalloc_with_dropout(device, dtype, hd, mask):
    """Attention dropout (p = 0.08, a fixed seed) through the no-allocation forward: equal to the allocating
    forward with the same p and seed (head dim 16 with dropout runs the wide MFMA kernels, whose workspace the
    scratch also covers), two calls in a row, the second smaller."""
    heads = 8 if hd == 24 else 16
    cases = ((generators.protein_like(seed=7, num_graphs=6), 41), (generators.protein_like(seed=8, num_graphs=2), 42))
    for gb, seed in cases:
        t = int(gb.cu_seqlens[-1])
        print(f"[noalloc] dropout {dtype} hd={hd} mask={mask} tokens={t}", flush=True)
        cu = torch.as_tensor(gb.cu_seqlens).to(device)
        q, k, v = (seeded_normal((t, heads, hd), seed + i, dtype).to(device) for i in range(3))
        kw = {"dropout_p": 0.08, "dropout_seed": 1000 + seed}
        if mask == "edge":
            kw.update(edge_src=torch.as_tensor(gb.edge_index[0].astype(np.int32)).to(device),
                      edge_dst=torch.as_tensor(gb.edge_index[1].astype(np.int32)).to(device))
        _compare(device, q, k, v, cu, int(gb.max_seqlen), kw)


def test_noalloc_forward_node_mask(device):
    for sizes, seed in (([60, 45, 80], 5), ([12, 7], 6)):
        ei, bm = node_graph(seed, sizes)
        na = NodeAdjacency.from_edge_index(torch.as_tensor(ei).to(device), torch.as_tensor(bm).to(device),
                                           len(sizes), max(sizes))
        t = len(bm)
        q, k, v = (seeded_normal((t, H, D), seed + i).to(device) for i in range(3))
        _compare(device, q, k, v, na.cu_seqlens, max(sizes),
                 {"adj_indptr": na.indptr, "adj_indices": na.indices})


def test_noalloc_rejects_shapes_beyond_scratch(device):
    lib = _lib.load()
    cap = int(lib.esa_noalloc_scratch_bytes())
    assert cap == 16 << 20
    n = _lib.ctypes.c_size_t(0)
    tq = 1 << 20          # one million tokens: the forward workspace exceeds 16 MiB
    _lib.check(lib.esa_varlen_attn_workspace_size(tq, tq, H, D, _lib.ESA_BF16, _lib.ESA_MASK_NONE, 0, 0,
                                                  _lib.ctypes.byref(n)), "workspace size")
    assert n.value > cap
    # the size check comes first: with null pointers nothing can be launched
    rc = lib.esa_varlen_attn_fwd_noalloc(None, None, None, None, None, 1, tq, tq, tq, tq, H, D, _lib.ESA_BF16, 0.25,
                                         0.0, 0, _lib.ESA_MASK_NONE, None, None, 0, None, None, None)
    assert rc == -8
