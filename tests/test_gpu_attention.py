"""GPU parity of the varlen / edge-masked attention kernels against the oracle.

Kernel entry points are called through the C ABI (ctypes) by
mind_amd.esa.attention.  Inputs are seeded bf16; the oracle runs in fp64 on the
same bf16 values.  Bar (bf16 outputs): max-abs <= 2e-2 and mean-abs <= 2e-3;
gradients against the same bar scaled by max(1, max|reference gradient|).
"""
import numpy as np
import pytest
import torch

from mind_amd import generators
from mind_amd.esa import attention as A
from oracle import attention as OA
from tests._util import assert_bf16_close, cu_from_lengths, err, grad_scale, seeded_normal

pytestmark = pytest.mark.gpu

H, D = 16, 16


def _inputs(tq, tk, seed, heads=H):
    q = seeded_normal((tq, heads, D), seed)
    k = seeded_normal((tk, heads, D), seed + 1)
    v = seeded_normal((tk, heads, D), seed + 2)
    g = seeded_normal((tq, heads, D), seed + 3)
    return q, k, v, g


def _run(device, q, k, v, g, cu_q, cu_k, src=None, dst=None, scale=0.25, shared_cu=False):
    qd, kd, vd = (t.to(device).requires_grad_(True) for t in (q, k, v))
    gd = g.to(device)
    cq = torch.as_tensor(cu_q, dtype=torch.int32).to(device)
    # One cu_seqlens tensor for queries and keys (as self-attention modules pass it) or two equal ones.
    ck = cq if shared_cu else torch.as_tensor(cu_k, dtype=torch.int32).to(device)
    s = None if src is None else torch.as_tensor(src, dtype=torch.int32).to(device)
    d = None if dst is None else torch.as_tensor(dst, dtype=torch.int32).to(device)
    mq = int(np.diff(cu_q).max()) if len(cu_q) > 1 else 0
    mk = int(np.diff(cu_k).max()) if len(cu_k) > 1 else 0
    out = A.varlen_attention(qd, kd, vd, cq, ck, mq, mk, softmax_scale=scale, edge_src=s, edge_dst=d)
    out.backward(gd)
    torch.cuda.synchronize()
    return out.detach().cpu(), qd.grad.cpu(), kd.grad.cpu(), vd.grad.cpu()


def _check(device, lengths_q, lengths_k, seed, src=None, dst=None, heads=H, check_lse=True, shared_cu=False):
    cu_q, cu_k = cu_from_lengths(lengths_q), cu_from_lengths(lengths_k)
    q, k, v, g = _inputs(int(cu_q[-1]), int(cu_k[-1]), seed, heads)
    out, dq, dk, dv = _run(device, q, k, v, g, cu_q, cu_k, src, dst, shared_cu=shared_cu)
    ref, lse_ref = OA.varlen_attention(q, k, v, cu_q, cu_k, 0.25, src, dst)
    assert_bf16_close(out, ref, what="out")
    if check_lse:
        cq = torch.as_tensor(cu_q).to(device)
        _, lse = A.attn_fwd(q.to(device), k.to(device), v.to(device), cq, torch.as_tensor(cu_k).to(device),
                            0, 0, 0.25, None if src is None else torch.as_tensor(src).to(device),
                            None if dst is None else torch.as_tensor(dst).to(device))
        lse = lse.cpu().double()
        fin = torch.isfinite(lse_ref)
        assert torch.equal(torch.isfinite(lse), fin), "lse -inf pattern differs"
        if fin.any():
            # The kernel's row sum is an MFMA over the bf16-rounded probabilities
            # (the same values that weight V), so the sum carries at most the
            # bf16 unit roundoff 2^-8 relative: |d lse| <= ln(1 + 2^-8) = 3.9e-3.
            assert float((lse[fin] - lse_ref[fin]).abs().max()) < 3.9e-3
    rdq, rdk, rdv = OA.varlen_attention_bwd(g, q, k, v, cu_q, cu_k, 0.25, src, dst)
    assert_bf16_close(dq, rdq, grad_scale(rdq), "dq")
    assert_bf16_close(dk, rdk, grad_scale(rdk), "dk")
    assert_bf16_close(dv, rdv, grad_scale(rdv), "dv")


def test_dense_protein_like_small(device):
    gb = generators.protein_like(seed=1, num_graphs=4, n_min=40, n_max=120)
    L = gb.edge_counts
    _check(device, L, L, seed=11)


@pytest.mark.parametrize("lengths", [[1], [5, 0, 7], [31, 32, 33], [1, 2, 3, 64, 65, 100, 0, 17], [200]])
def test_dense_ragged(device, lengths):
    _check(device, lengths, lengths, seed=sum(lengths))


def test_dense_heads_not_multiple_of_four(device):
    _check(device, [40, 70], [40, 70], seed=5, heads=6)


@pytest.mark.parametrize("heads", [4, 8, 32])
def test_dense_xcd_line_mappings(device, heads):
    """Head counts whose blocks are mapped by 128-byte line group onto the XCDs (one XCD per line group at 32
    heads, two at 16, four at 8, eight at 4): every (group, head) work item runs once, with ragged segments
    longer than a group and an odd number of groups."""
    _check(device, [300, 1, 129, 64, 0, 257], [300, 1, 129, 64, 0, 257], seed=40 + heads, heads=heads)


@pytest.mark.parametrize("seeds", [1, 4, 32])
def test_cross_attention_pma_shape(device, seeds):
    # PMA: k seeds per graph attend over the graph's tokens.
    lk = [50, 1, 130, 77]
    lq = [seeds] * len(lk)
    _check(device, lq, lk, seed=seeds + 100)


def test_cross_attention_empty_key_segments(device):
    """Sets without keys (a graph with no edges under PMA): their queries get 0 and lse = -inf, zero dQ, and
    their row statistics (written by the dQ pass, a finite -LSE2 so that P = 0) leave the dK/dV pass of the
    neighbouring segments, whose last partial tiles read them, unchanged."""
    _check(device, [4, 4, 4, 3, 5], [50, 0, 70, 0, 33], seed=321)


def test_masked_protein_like_small(device):
    gb = generators.protein_like(seed=2, num_graphs=3, n_min=40, n_max=90)
    src, dst = gb.edge_index[0].astype(np.int32), gb.edge_index[1].astype(np.int32)
    _check(device, gb.edge_counts, gb.edge_counts, seed=21, src=src, dst=dst)


def test_masked_small_molecules(device):
    gb, _ = generators.small_molecules(seed=3, num_graphs=6)
    src, dst = gb.edge_index[0].astype(np.int32), gb.edge_index[1].astype(np.int32)
    _check(device, gb.edge_counts, gb.edge_counts, seed=31, src=src, dst=dst)


@pytest.mark.parametrize("heads", [1, 5])
def test_masked_head_counts(device, heads):
    # The edge-mask kernels take heads in groups; a last, partial group.
    gb = generators.protein_like(seed=4, num_graphs=3, n_min=30, n_max=70)
    src, dst = gb.edge_index[0].astype(np.int32), gb.edge_index[1].astype(np.int32)
    _check(device, gb.edge_counts, gb.edge_counts, seed=41 + heads, src=src, dst=dst, heads=heads)


def test_masked_segments_straddle_tiles(device):
    # Short graphs packed back to back: most 32-token tiles hold tokens of
    # several segments, and some graphs have a single edge.
    gb, _ = generators.small_molecules(seed=9, num_graphs=24)
    src, dst = gb.edge_index[0].astype(np.int32), gb.edge_index[1].astype(np.int32)
    _check(device, gb.edge_counts, gb.edge_counts, seed=91, src=src, dst=dst)


def test_masked_star_graph_far_partner_tiles(device):
    """A star graph (hub 0 and 1,200 leaves, both edge directions): every edge shares the hub, so the edge mask
    is dense over one 2,400-token segment of 75 tiles.  Every tile's partner union (2,399 tokens) is past the
    key-list capacity, so all groups take the walk kernels over the overflow list."""
    leaves = np.arange(1, 1201, dtype=np.int32)
    src = np.concatenate([np.zeros_like(leaves), leaves])
    dst = np.concatenate([leaves, np.zeros_like(leaves)])
    _check(device, [src.size], [src.size], seed=77, src=src, dst=dst)


@pytest.mark.parametrize("shared_cu", [False, True])
def test_masked_mixed_overflow(device, shared_cu):
    """Protein-like graphs around a 600-token star segment: the star's groups overflow the key lists (walk
    kernels), the others take the lists, in one call; with one cu_seqlens tensor for queries and keys the
    dK/dV pass reads the query tiles' lists (symmetric mask), with two it builds the key tiles' own."""
    gb = generators.protein_like(seed=12, num_graphs=4, n_min=64, n_max=160)
    src_p, dst_p = gb.edge_index[0].astype(np.int32), gb.edge_index[1].astype(np.int32)
    hub = int(max(src_p.max(), dst_p.max())) + 1
    leaves = np.arange(hub + 1, hub + 301, dtype=np.int32)
    star_s = np.concatenate([np.full_like(leaves, hub), leaves])
    star_d = np.concatenate([leaves, np.full_like(leaves, hub)])
    c = gb.edge_counts
    src = np.concatenate([src_p[:c[0] + c[1]], star_s, src_p[c[0] + c[1]:]])
    dst = np.concatenate([dst_p[:c[0] + c[1]], star_d, dst_p[c[0] + c[1]:]])
    lengths = [int(c[0]), int(c[1]), star_s.size, int(c[2]), int(c[3])]
    _check(device, lengths, lengths, seed=78, src=src, dst=dst, shared_cu=shared_cu)


def test_masked_shared_cu_protein(device):
    """The symmetric-mask path (one cu_seqlens tensor) on protein-like graphs with ragged segment ends."""
    gb = generators.protein_like(seed=13, num_graphs=5, n_min=40, n_max=200)
    src, dst = gb.edge_index[0].astype(np.int32), gb.edge_index[1].astype(np.int32)
    _check(device, gb.edge_counts, gb.edge_counts, seed=79, src=src, dst=dst, shared_cu=True)


def test_masked_isolated_rows_give_zero(device):
    # Two disjoint edges in one segment: neither shares a node with the other.
    src = np.array([0, 2, 4], np.int32)
    dst = np.array([1, 3, 4 + 1], np.int32)
    _check(device, [3], [3], seed=7, src=src, dst=dst)


def test_backward_is_deterministic(device):
    gb = generators.protein_like(seed=4, num_graphs=3, n_min=60, n_max=100)
    cu = gb.cu_seqlens
    q, k, v, g = _inputs(int(cu[-1]), int(cu[-1]), 41)
    r1 = _run(device, q, k, v, g, cu, cu)
    r2 = _run(device, q, k, v, g, cu, cu)
    for a, b in zip(r1, r2):
        assert torch.equal(a, b)


def test_full_config1_size(device):
    """C2 at full size: every output finite; three segments checked against the oracle."""
    gb = generators.protein_like(seed=0)
    cu = gb.cu_seqlens
    t = int(cu[-1])
    q, k, v, g = _inputs(t, t, 1234)
    out, dq, dk, dv = _run(device, q, k, v, g, cu, cu)
    for x in (out, dq, dk, dv):
        assert torch.isfinite(x.float()).all()
    for b in (0, int(np.argmax(gb.edge_counts)), gb.num_graphs - 1):
        s, e = int(cu[b]), int(cu[b + 1])
        sub = np.array([0, e - s], np.int32)
        ref, _ = OA.varlen_attention(q[s:e], k[s:e], v[s:e], sub, sub, 0.25)
        assert_bf16_close(out[s:e], ref, what=f"segment {b}")
        rdq, rdk, rdv = OA.varlen_attention_bwd(g[s:e], q[s:e], k[s:e], v[s:e], sub, sub, 0.25)
        assert_bf16_close(dq[s:e], rdq, grad_scale(rdq), f"dq segment {b}")
        assert_bf16_close(dk[s:e], rdk, grad_scale(rdk), f"dk segment {b}")
        assert_bf16_close(dv[s:e], rdv, grad_scale(rdv), f"dv segment {b}")


def test_full_config2_size_masked(device):
    """Configuration 2 (edge-masked MAB attention) at full size: the token-budgeted batch of up to 65,536
    tokens; every output finite, and three segments (first, largest, last) checked against the oracle."""
    gb = generators.protein_budget(seed=0, token_budget=65536)
    cu = gb.cu_seqlens
    t = int(cu[-1])
    src, dst = gb.edge_index[0].astype(np.int32), gb.edge_index[1].astype(np.int32)
    q, k, v, g = _inputs(t, t, 4321)
    out, dq, dk, dv = _run(device, q, k, v, g, cu, cu, src, dst)
    for x in (out, dq, dk, dv):
        assert torch.isfinite(x.float()).all()
    for b in (0, int(np.argmax(gb.edge_counts)), gb.num_graphs - 1):
        s, e = int(cu[b]), int(cu[b + 1])
        sub = np.array([0, e - s], np.int32)
        ls, ld = src[s:e], dst[s:e]
        ref, _ = OA.varlen_attention(q[s:e], k[s:e], v[s:e], sub, sub, 0.25, ls, ld)
        assert_bf16_close(out[s:e], ref, what=f"segment {b}")
        rdq, rdk, rdv = OA.varlen_attention_bwd(g[s:e], q[s:e], k[s:e], v[s:e], sub, sub, 0.25, ls, ld)
        assert_bf16_close(dq[s:e], rdq, grad_scale(rdq), f"dq segment {b}")
        assert_bf16_close(dk[s:e], rdk, grad_scale(rdk), f"dk segment {b}")
        assert_bf16_close(dv[s:e], rdv, grad_scale(rdv), f"dv segment {b}")


def test_edge_mask_dense_bits(device):
    """The on-device predicate materialised equals the oracle's global E x E mask, bit for bit."""
    from oracle import mask as OM
    gb = generators.protein_like(seed=5, num_graphs=3, n_min=30, n_max=60)
    src, dst = gb.edge_index[0].astype(np.int32), gb.edge_index[1].astype(np.int32)
    cu = gb.cu_seqlens
    n = int(np.diff(cu).max()) + 3
    m = A.edge_mask_dense(torch.as_tensor(src).to(device), torch.as_tensor(dst).to(device),
                          torch.as_tensor(cu).to(device), n).cpu().numpy().astype(bool)
    glob = OM.edge_adjacency_global(src, dst)
    for b in range(gb.num_graphs):
        s, e = int(cu[b]), int(cu[b + 1])
        ref = np.zeros((n, n), bool)
        ref[: e - s, : e - s] = glob[s:e, s:e]
        assert np.array_equal(m[b], ref)
    # cross-graph pairs never match
    gid = np.repeat(np.arange(gb.num_graphs), gb.edge_counts)
    assert not (glob & (gid[:, None] != gid[None, :])).any()


def test_argument_errors(device):
    q = torch.zeros(8, 4, 16, dtype=torch.bfloat16, device=device)
    cu = torch.tensor([0, 8], dtype=torch.int32, device=device)
    with pytest.raises(TypeError):
        A.attn_fwd(q.float(), q, q, cu, cu, 8, 8, 0.25)
    with pytest.raises(ValueError):
        A.attn_fwd(torch.zeros(8, 4, 32, dtype=torch.bfloat16, device=device), q, q, cu, cu, 8, 8, 0.25)
    with pytest.raises(TypeError):
        A.attn_fwd(q, q, q, cu.long(), cu, 8, 8, 0.25)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("seeds", [1, 4, 32])
def test_pma_seed_pooling(device, dtype, seeds):
    """esa_pma_fwd/_bwd: k shared seeds over each set's keys equal varlen attention with the seeds repeated per
    set (bit for bit: the same kernels run on the expanded queries), and against the oracle; the seed gradient
    is the sum over sets of the repeated queries' gradients."""
    lk = [50, 0, 130, 77, 1, 300]
    cu_k = cu_from_lengths(lk)
    b, tk = len(lk), int(cu_k[-1])
    qs = seeded_normal((seeds, H, D), 700 + seeds, dtype)
    k = seeded_normal((tk, H, D), 701, dtype)
    v = seeded_normal((tk, H, D), 702, dtype)
    g = seeded_normal((b * seeds, H, D), 703, dtype)
    qd, kd, vd = (t.to(device).requires_grad_(True) for t in (qs, k, v))
    ck = torch.as_tensor(cu_k).to(device)
    out = A.pma_attention(qd, kd, vd, ck, max(lk), softmax_scale=0.25)
    out.backward(g.to(device))
    qr = qs.repeat(b, 1, 1)
    cu_q = cu_from_lengths([seeds] * b)
    qrd, krd, vrd = (t.to(device).requires_grad_(True) for t in (qr, k, v))
    ref_dev = A.varlen_attention(qrd, krd, vrd, torch.as_tensor(cu_q).to(device), ck, seeds, max(lk), softmax_scale=0.25)
    ref_dev.backward(g.to(device))
    assert torch.equal(out.detach(), ref_dev.detach())
    assert torch.equal(kd.grad, krd.grad) and torch.equal(vd.grad, vrd.grad)
    ref, _ = OA.varlen_attention(qr, k, v, cu_q, cu_k, 0.25)
    rdq, rdk, rdv = OA.varlen_attention_bwd(g, qr, k, v, cu_q, cu_k, 0.25)
    rdq_seeds = rdq.reshape(b, seeds, H, D).sum(0)
    if dtype == torch.float32:
        from tests._util import assert_f32_close
        assert_f32_close(out.detach().cpu(), ref, "out")
        assert_f32_close(qd.grad.cpu(), rdq_seeds, "d seeds")
        assert_f32_close(kd.grad.cpu(), rdk, "dk")
    else:
        assert_bf16_close(out.detach().cpu(), ref, what="out")
        assert_bf16_close(qd.grad.cpu(), rdq_seeds, grad_scale(rdq_seeds), "d seeds")
        assert_bf16_close(kd.grad.cpu(), rdk, grad_scale(rdk), "dk")
        assert_bf16_close(vd.grad.cpu(), rdv, grad_scale(rdv), "dv")


@pytest.mark.parametrize("masked", [False, True])
def test_32_heads(device, masked):
    """Configuration 4's attention shape: 32 heads of head_dim 16 (dim 512), dense and edge-masked, bf16."""
    gb = generators.protein_like(seed=12, num_graphs=4, n_min=40, n_max=140)
    src = gb.edge_index[0].astype(np.int32) if masked else None
    dst = gb.edge_index[1].astype(np.int32) if masked else None
    _check(device, gb.edge_counts, gb.edge_counts, seed=1200 + masked, src=src, dst=dst, heads=32)


def test_dense_rows_after_last_segment(device):
    """cu_seqlens_q[-1] < total_q (flash-attn's varlen API allows it): the dK/dV pass stages the row statistics
    of the rows after the last segment with its last partial tile; the backward prep writes them, so a
    workspace full of NaN leaves dK / dV of every segment finite and equal to the oracle's."""
    from mind_amd import _lib
    lens = [40, 30]
    cu = cu_from_lengths(lens)
    tq = 90                                   # rows 70..89 belong to no segment
    q, _, _, g = _inputs(tq, tq, 901)
    k, v = seeded_normal((70, H, D), 905), seeded_normal((70, H, D), 906)
    dev = [t.to(device).contiguous() for t in (q, k, v, g)]
    qd, kd, vd, gd = dev
    cud = torch.as_tensor(cu).to(device)
    out, lse = A.attn_fwd(qd, kd, vd, cud, cud, 40, 40, 0.25)
    out[70:] = 0                              # rows no segment covers are not written by the forward
    lse[:, 70:] = 0
    lib = _lib.load()
    n = _lib.ctypes.c_size_t(0)
    _lib.check(lib.esa_varlen_attn_workspace_size(tq, 70, H, D, _lib.ESA_BF16, _lib.ESA_MASK_NONE, 0, 1,
                                                  _lib.ctypes.byref(n)), "workspace size")
    ws = torch.full((int(n.value),), 0xFF, dtype=torch.uint8, device=device)   # every float NaN
    dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    rc = lib.esa_varlen_attn_bwd(gd.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(),
                                 lse.data_ptr(), cud.data_ptr(), cud.data_ptr(), 2, tq, 70, 40, 40, H, D,
                                 _lib.ESA_BF16, 0.25, 0.0, 0, _lib.ESA_MASK_NONE, None, None, 0, dq.data_ptr(), dk.data_ptr(),
                                 dv.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(qd))
    _lib.check(rc, "esa_varlen_attn_bwd")
    torch.cuda.synchronize()
    assert torch.isfinite(dk.float()).all() and torch.isfinite(dv.float()).all()
    rdq, rdk, rdv = OA.varlen_attention_bwd(g[:70], q[:70], k, v, cu, cu, 0.25)
    assert_bf16_close(dk.cpu(), rdk, grad_scale(rdk), "dk")
    assert_bf16_close(dv.cpu(), rdv, grad_scale(rdv), "dv")
    assert_bf16_close(dq[:70].cpu(), rdq, grad_scale(rdq), "dq")


@pytest.mark.parametrize("shared_cu", [True, False])
def test_edge_plan_reuse_matches_per_call_mask(device, shared_cu):
    """A plan built once (esa_edge_plan_build) and passed to several forward / backward calls gives the same
    bits as the per-call edge mask (the kernels are the same); with two cu_seqlens tensors the plan carries
    the key tiles' own lists.  A group that overflows the key lists (a 600-token star) is part of the batch."""
    gb = generators.protein_like(seed=14, num_graphs=4, n_min=64, n_max=200)
    src_p, dst_p = gb.edge_index[0].astype(np.int32), gb.edge_index[1].astype(np.int32)
    hub = int(max(src_p.max(), dst_p.max())) + 1
    leaves = np.arange(hub + 1, hub + 301, dtype=np.int32)
    c = gb.edge_counts
    src = np.concatenate([src_p[:c[0]], np.full_like(leaves, hub), leaves, src_p[c[0]:]])
    dst = np.concatenate([dst_p[:c[0]], leaves, np.full_like(leaves, hub), dst_p[c[0]:]])
    lengths = [int(c[0]), 2 * leaves.size] + [int(x) for x in c[1:]]
    cu_np = cu_from_lengths(lengths)
    t = int(cu_np[-1])
    cq = torch.as_tensor(cu_np, dtype=torch.int32).to(device)
    ck = cq if shared_cu else torch.as_tensor(cu_np, dtype=torch.int32).to(device)
    s_d, d_d = torch.as_tensor(src).to(device), torch.as_tensor(dst).to(device)
    mx = int(max(lengths))
    plan = A.edge_plan(s_d, d_d, cq, ck)
    for seed in (301, 302):   # two different inputs over one plan
        q, k, v, g = (x.to(device) for x in _inputs(t, t, seed))
        o1, l1 = A.attn_fwd(q, k, v, cq, ck, mx, mx, 0.25, s_d, d_d)
        o2, l2 = A.attn_fwd(q, k, v, cq, ck, mx, mx, 0.25, edge_plan=plan)
        assert torch.equal(o1, o2) and torch.equal(l1, l2)
        g1 = A.attn_bwd(g, q, k, v, o1, l1, cq, ck, mx, mx, 0.25, s_d, d_d)
        g2 = A.attn_bwd(g, q, k, v, o1, l1, cq, ck, mx, mx, 0.25, edge_plan=plan)
        for x1, x2 in zip(g1, g2):
            assert torch.equal(x1, x2)
    torch.cuda.synchronize()
    ref, _ = OA.varlen_attention(q.cpu(), k.cpu(), v.cpu(), cu_np, cu_np, 0.25, src, dst)
    assert_bf16_close(o2.cpu(), ref, what="out")


def test_edge_plan_through_autograd_and_module_descriptor(device):
    """varlen_attention(edge_plan=...) differentiates like the edge-mask call, and the EdgeAdjacency descriptor
    builds its plan once and hands it to every masked layer."""
    from mind_amd.esa.packing import EdgeAdjacency
    gb = generators.protein_like(seed=15, num_graphs=3, n_min=50, n_max=120)
    ei = torch.as_tensor(gb.edge_index).to(device)
    bm = torch.as_tensor(gb.batch).to(device)
    adj = EdgeAdjacency.from_edge_index(ei, bm, gb.num_graphs, int(gb.max_seqlen))
    kw = adj.kernel_mask(padded=False)
    assert set(kw) == {"edge_plan"} and adj.kernel_mask(padded=False)["edge_plan"] is kw["edge_plan"]
    t = adj.num_tokens
    q, k, v, g = _inputs(t, t, 401)
    res = []
    for mask in (kw, {"edge_src": adj.edge_src, "edge_dst": adj.edge_dst}):
        qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
        out = A.varlen_attention(qd, kd, vd, adj.cu_seqlens, adj.cu_seqlens, adj.max_items, adj.max_items,
                                 softmax_scale=0.25, **mask)
        out.backward(g.to(device))
        res.append((out.detach(), qd.grad, kd.grad, vd.grad))
    for x1, x2 in zip(*res):
        assert torch.equal(x1, x2)
