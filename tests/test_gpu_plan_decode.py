"""The masks the hot path reads, bit for bit.

The attention kernels never see the reference's [B, N, N] bias: the edge-masked kernels read an edge-mask plan
(per 32-token tile a partner list with one mask bit per token and entry, plus the overflow groups the walk
kernels take) and the node-mode backward reads a node plan (the CSR's transpose by key and per-token
descriptors).  esa_edge_plan_decode expands a plan the way the kernels read it; these tests compare that, and
the node plan's sections, exactly with the oracle's mask (esa/masked_layers.py:121-142, 217-268 for the edge
mask; :79-118 for the node mask) and with a numpy transpose.
"""
import numpy as np
import pytest
import torch

from mind_amd import generators
from mind_amd.esa import attention as A
from mind_amd.esa.packing import NodeAdjacency
from oracle import mask as OM
from tests._util import node_graph

pytestmark = pytest.mark.gpu


def _oracle_edge_csr(src, dst, cu):
    """Per token, its admissible partner tokens (ascending) from the oracle's per-graph adjacency."""
    counts, cols = [], []
    for b in range(len(cu) - 1):
        s, e = int(cu[b]), int(cu[b + 1])
        m = OM.edge_adjacency_segment(src, dst, s, e)
        counts.append(m.sum(1))
        cols.append(np.nonzero(m)[1] + s)   # row-major: rows in order, each row ascending
    counts = np.concatenate(counts) if counts else np.zeros(0, np.int64)
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    return indptr, (np.concatenate(cols) if cols else np.zeros(0, np.int64))


def _check_edge_plan(device, src, dst, lengths, shared_cu, label):
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    t = int(cu[-1])
    print(f"[plan-decode] {label}: tokens={t} segments={len(lengths)} shared_cu={shared_cu}", flush=True)
    cq = torch.as_tensor(cu).to(device)
    ck = cq if shared_cu else torch.as_tensor(cu).to(device)
    plan = A.edge_plan(torch.as_tensor(src, dtype=torch.int32).to(device),
                       torch.as_tensor(dst, dtype=torch.int32).to(device), cq, ck)
    ref_ptr, ref_idx = _oracle_edge_csr(src, dst, cu)
    for direction in (0, 1):
        ptr, idx = A.edge_plan_decode(plan, t, direction)
        ptr, idx = ptr.cpu().numpy().astype(np.int64), idx.cpu().numpy().astype(np.int64)
        assert np.array_equal(ptr, ref_ptr), f"{label} dir {direction}: partner counts differ"
        assert np.array_equal(idx, ref_idx), f"{label} dir {direction}: partner ids differ"
    return plan, ref_ptr


def test_edge_plan_config2_full_size(device):
    """Configuration 2's token-budget batch (up to 65,536 edge tokens, seed 0): the plan's lists and mask words
    decode to the oracle's adjacency exactly, for the forward/dQ and the dK/dV directions."""
    gb = generators.protein_budget(seed=0, token_budget=65536)
    src, dst = gb.edge_index[0].astype(np.int64), gb.edge_index[1].astype(np.int64)
    _, ref_ptr = _check_edge_plan(device, src, dst, gb.edge_counts, True, "config2")
    assert int(ref_ptr[-1]) == OM.edge_mask_nnz(src, dst)   # nnz of the whole batch: no cross-graph pairs


def test_edge_plan_config0(device):
    """Configuration 0's 64 small molecules (seed 0): short segments packed several to a tile."""
    gb, _ = generators.small_molecules(seed=0)
    assert gb.num_graphs == 64
    src, dst = gb.edge_index[0].astype(np.int64), gb.edge_index[1].astype(np.int64)
    for shared in (True, False):
        _check_edge_plan(device, src, dst, gb.edge_counts, shared, "config0")


@pytest.mark.parametrize("shared_cu", [True, False])
def test_edge_plan_star_all_overflow(device, shared_cu):
    """A 2,400-token star segment: every tile's partner union is past the list capacity, so every group is
    on the overflow list and decodes through the walk kernels' predicate."""
    leaves = np.arange(1, 1201, dtype=np.int64)
    src = np.concatenate([np.zeros_like(leaves), leaves])
    dst = np.concatenate([leaves, np.zeros_like(leaves)])
    _check_edge_plan(device, src, dst, [src.size], shared_cu, "star")


@pytest.mark.parametrize("shared_cu", [True, False])
def test_edge_plan_mixed_overflow(device, shared_cu):
    """Protein-like graphs around a 600-token star segment: listed and overflowing groups in one plan, with
    one cu_seqlens array (symmetric plan) and with two (the key tiles' own lists and overflow groups)."""
    gb = generators.protein_like(seed=12, num_graphs=4, n_min=64, n_max=160)
    src_p, dst_p = gb.edge_index[0].astype(np.int64), gb.edge_index[1].astype(np.int64)
    hub = int(max(src_p.max(), dst_p.max())) + 1
    leaves = np.arange(hub + 1, hub + 301, dtype=np.int64)
    star_s = np.concatenate([np.full_like(leaves, hub), leaves])
    star_d = np.concatenate([leaves, np.full_like(leaves, hub)])
    c = gb.edge_counts
    src = np.concatenate([src_p[:c[0] + c[1]], star_s, src_p[c[0] + c[1]:]])
    dst = np.concatenate([dst_p[:c[0] + c[1]], star_d, dst_p[c[0] + c[1]:]])
    lengths = [int(c[0]), int(c[1]), star_s.size, int(c[2]), int(c[3])]
    _check_edge_plan(device, src, dst, lengths, shared_cu, "mixed")


def test_edge_plan_isolated_and_single_edges(device):
    """Segments of one edge, and edges sharing no node: rows without partners decode empty."""
    src = np.array([0, 2, 4, 7, 9, 9], np.int64)
    dst = np.array([1, 3, 5, 8, 10, 11], np.int64)
    _check_edge_plan(device, src, dst, [3, 1, 2], True, "isolated")


def _numpy_transpose(indptr, indices, tk):
    """Per key token, the CSR entries' query rows in ascending entry position (a stable sort by key); keys
    outside [0, tk) are not listed under any key."""
    tq = len(indptr) - 1
    row_of = np.repeat(np.arange(tq), np.diff(indptr))
    keys = indices.astype(np.int64)
    order = np.argsort(keys, kind="stable")
    inside = (keys[order] >= 0) & (keys[order] < tk)
    order = order[inside]
    t_indptr = np.concatenate([[0], np.cumsum(np.bincount(keys[order], minlength=tk))])
    return t_indptr, row_of[order]


def _descriptors(cu_own, cu_other, total_other, indptr, nnz):
    n = int(cu_own[-1])
    seg = np.searchsorted(cu_own, np.arange(n), side="right") - 1
    lo = np.maximum(cu_other[seg], 0)
    hi = np.minimum(cu_other[seg + 1], total_other)
    pa = np.clip(indptr[:-1], 0, nnz)
    pb = np.clip(indptr[1:], pa, nnz)
    return np.stack([lo, hi, pa, np.where(hi > lo, pb, pa)], 1)


@pytest.mark.parametrize("which", ["node_graph", "config2_nodes"])
def test_node_plan_sections(device, which):
    """The node plan's copy of the indices, its transposed CSR (t_indptr, t_rows) and both sides' token
    descriptors equal a numpy transpose and closed forms, bit for bit."""
    if which == "node_graph":
        ei, bm = node_graph(31, [60, 1, 45, 80, 7])
        sizes = np.bincount(bm)
    else:   # configuration 2's generator in node mode: 65,536-node budget
        gb = generators.protein_budget(seed=0, token_budget=65536, count="nodes")
        ei, bm, sizes = gb.edge_index.astype(np.int64), gb.batch.astype(np.int64), np.bincount(gb.batch)
    na = NodeAdjacency.from_edge_index(torch.as_tensor(ei).to(device), torch.as_tensor(bm).to(device),
                                       len(sizes), int(sizes.max()))
    t, nnz = len(bm), int(na.indices.numel())
    print(f"[plan-decode] node plan {which}: tokens={t} entries={nnz}", flush=True)
    plan = na.plan()
    sec = {k: v.cpu().numpy().astype(np.int64) for k, v in A.node_plan_sections(plan, t, t, nnz).items()}
    indptr = na.indptr.cpu().numpy().astype(np.int64)
    indices = na.indices.cpu().numpy().astype(np.int64)
    cu = na.cu_seqlens.cpu().numpy().astype(np.int64)
    assert np.array_equal(sec["indices"], indices)
    t_indptr, t_rows = _numpy_transpose(indptr, indices, t)
    assert np.array_equal(sec["t_indptr"], t_indptr)
    assert np.array_equal(sec["t_rows"][: int(t_indptr[-1])], t_rows)
    assert np.array_equal(sec["q_desc"], _descriptors(cu, cu, t, indptr, nnz))
    assert np.array_equal(sec["k_desc"], _descriptors(cu, cu, t, t_indptr, nnz))
    # the CSR itself against the reference's node bias: row i lists exactly the keys j with bias 0
    bias = OM.node_bias_padded(ei, bm, len(sizes), int(sizes.max()))[:, 0]
    first = np.concatenate([[0], np.cumsum(sizes)[:-1]])
    for b in range(min(len(sizes), 6)):
        s, n = int(first[b]), int(sizes[b])
        blk = OM.node_adjacency_segment(indptr, indices, s, s + n, s, s + n)
        assert np.array_equal(blk, (bias[b, :n, :n] == 0).numpy())


def _csr(rows):
    ip = np.cumsum([0] + [len(r) for r in rows]).astype(np.int32)
    ix = np.array([j for r in rows for j in r], dtype=np.int32)
    return ip, ix


@pytest.mark.parametrize("case", ["symmetric", "symmetric_repeats", "repeat_count_differs", "unsorted_row",
                                  "key_out_of_range", "one_way_edge"])
def test_node_plan_symmetric_and_general_builds(device, case):
    """A CSR that equals its own transpose (sorted rows, every entry (i, j) matched by (j, i) as often) is
    copied into the plan instead of sorted; every other CSR takes the sort.  Either way the sections equal a
    numpy transpose and the descriptors' closed forms, bit for bit: the cases below sit one entry away from
    symmetric in each way the test on the device must catch."""
    rng = np.random.default_rng(17)
    sizes = [40, 1, 23, 57]
    cu_np = np.cumsum([0] + sizes)
    t = int(cu_np[-1])
    adj = [set() for _ in range(t)]
    for b, n in enumerate(sizes):
        s = int(cu_np[b])
        for _ in range(3 * n):
            i, j = rng.integers(s, s + n, size=2)
            if i != j:
                adj[i].add(int(j))
                adj[j].add(int(i))
    rows = [sorted(a) for a in adj]
    i0 = next(i for i, r in enumerate(rows) if r)
    j0 = rows[i0][0]
    if case == "symmetric_repeats":          # the edge (i0, j0) listed twice in both directions
        rows[i0] = sorted(rows[i0] + [j0])
        rows[j0] = sorted(rows[j0] + [i0])
    elif case == "repeat_count_differs":     # twice one way, once the other
        rows[i0] = sorted(rows[i0] + [j0])
    elif case == "unsorted_row":             # symmetric as a set, one row out of order
        r = next(i for i, r in enumerate(rows) if len(r) >= 2)
        rows[r] = rows[r][::-1]
    elif case == "key_out_of_range":         # one entry naming key t (past the last token)
        rows[i0] = rows[i0] + [t]
    elif case == "one_way_edge":             # (i0, j0) without (j0, i0)
        rows[j0] = [x for x in rows[j0] if x != i0]
    ip, ix = _csr(rows)
    nnz = len(ix)
    cu = torch.as_tensor(cu_np.astype(np.int32)).to(device)
    plan = A.node_plan(torch.as_tensor(ip).to(device), torch.as_tensor(ix).to(device), cu)
    sec = {k: v.cpu().numpy().astype(np.int64) for k, v in A.node_plan_sections(plan, t, t, nnz).items()}
    t_indptr, t_rows = _numpy_transpose(ip.astype(np.int64), ix.astype(np.int64), t)
    assert np.array_equal(sec["indices"], ix)
    assert np.array_equal(sec["t_indptr"], t_indptr)
    assert np.array_equal(sec["t_rows"][: int(t_indptr[-1])], t_rows)
    assert np.array_equal(sec["q_desc"], _descriptors(cu_np, cu_np, t, ip.astype(np.int64), nnz))
    assert np.array_equal(sec["k_desc"], _descriptors(cu_np, cu_np, t, t_indptr, nnz))
    if case in ("symmetric", "symmetric_repeats"):
        assert np.array_equal(t_indptr, ip) and np.array_equal(t_rows, ix)   # its own transpose
