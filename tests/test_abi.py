"""The C-ABI library loads and exports every symbol include/esa_hip.h declares (no GPU needed)."""
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "esa_hip.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^ESA_API\s+[\w\s\*]+?\b(esa_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_entry_points():
    names = _declared()
    assert "esa_varlen_attn_fwd" in names and "esa_edge_gather" in names
    assert len(names) >= 10


def test_profile_kernel_count_matches_the_header():
    """The Python hook's buffer size is the header's ESA_PROFILE_KERNELS, and every id has a name."""
    import re
    from mind_amd import _lib
    text = (Path(__file__).resolve().parents[1] / "include" / "esa_hip.h").read_text()
    assert int(re.search(r"#define ESA_PROFILE_KERNELS (\d+)", text).group(1)) == _lib.PROFILE_KERNELS
    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    lib = _lib.load()
    names = [lib.esa_profile_kernel_name(i).decode() for i in range(_lib.PROFILE_KERNELS)]
    assert all(names) and len(set(names)) == len(names) and lib.esa_profile_kernel_name(_lib.PROFILE_KERNELS) == b""
    assert "segment_minmax" in names


def test_library_exports_every_declared_symbol():
    from mind_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built (run __graft_entry__.build())")
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (esa_\w+)", out))
    missing = [n for n in _declared() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    # nothing else leaks out of the C ABI
    assert exported == set(_declared())
    assert sorted(_lib.exported_symbols()) == _declared()


def test_library_loads_and_reports_version():
    from mind_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    assert _lib.version().startswith("esa_hip")


def test_single_hip_runtime_mapped():
    """Loading the library after torch maps exactly one libamdhip64 into the process."""
    from mind_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    import torch  # noqa: F401
    _lib.load()
    maps = Path("/proc/self/maps").read_text()
    libs = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    assert len(libs) == 1, libs


def test_argument_errors_need_no_gpu():
    """Argument validation runs before any launch: bad head_dim / workspace are errors, not faults."""
    import ctypes
    from mind_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    lib = _lib.load()
    n = ctypes.c_size_t(0)
    bf16, f32, none, edge = _lib.ESA_BF16, _lib.ESA_F32, _lib.ESA_MASK_NONE, _lib.ESA_MASK_EDGE
    for hd in (8, 12, 20, 48, 128):   # head dims outside 16, 24, 32, 64
        assert lib.esa_varlen_attn_workspace_size(100, 100, 16, hd, bf16, none, 0, 0, ctypes.byref(n)) == -3
    for hd in (24, 32, 64):
        for dt in (bf16, f32):
            for mk in (none, edge, _lib.ESA_MASK_NODE):
                assert lib.esa_varlen_attn_workspace_size(100, 100, 8, hd, dt, mk, 0, 1, ctypes.byref(n)) == 0
    assert lib.esa_varlen_attn_workspace_size(100, 90, 16, 16, bf16, edge, 0, 0, ctypes.byref(n)) == -7
    assert lib.esa_varlen_attn_workspace_size(100, 100, 16, 16, 7, none, 0, 0, ctypes.byref(n)) == -5
    assert lib.esa_varlen_attn_workspace_size(100, 100, 16, 16, bf16, 9, 0, 0, ctypes.byref(n)) == -7
    for dt in (bf16, f32):
        assert lib.esa_varlen_attn_workspace_size(100, 100, 16, 16, dt, none, 0, 1, ctypes.byref(n)) == 0
        assert n.value > 0
    # fwd with a too-small workspace is rejected before anything is launched
    rc = lib.esa_varlen_attn_fwd(16, 16, 16, 16, 16, 1, 100, 100, 100, 100, 16, 16, bf16, 0.25, 0.0, 0, none, None,
                                 None, 0, 16, 16, 256, 10, None)
    assert rc == -4
    # dropout_p outside [0, 1) is rejected before anything is launched
    for p in (-0.1, 1.0, 1.5, float("nan")):
        rc = lib.esa_varlen_attn_fwd(16, 16, 16, 16, 16, 1, 100, 100, 100, 100, 16, 16, bf16, 0.25, p, 7, none, None,
                                     None, 0, 16, 16, 1 << 20, 1 << 20, None)
        assert rc == -9, p
    assert lib.esa_edge_gather(16, 16, 16, 10, 10, 8, 7, 16, None) == -5
    assert lib.esa_csr_workspace_size(-1, 10, ctypes.byref(n)) == -2
    # segmented min / max: null, shape and dtype errors before any launch; no nodes is a no-op
    assert lib.esa_csr_segment_minmax(16, None, None, 10, 1, f32, 0, 5, 16, 16, None) == -1
    assert lib.esa_csr_segment_minmax(16, None, 16, 10, 0, f32, 0, 5, 16, 16, None) == -2
    assert lib.esa_csr_segment_minmax(16, None, 16, 10, 1, f32, 1, -1, 16, 16, None) == -2
    assert lib.esa_csr_segment_minmax(16, None, 16, 10, 1, 7, 0, 5, 16, 16, None) == -5
    assert lib.esa_csr_segment_minmax(16, None, 16, 0, 1, bf16, 1, 5, 16, None, None) == 0
    # fp32 Linear: shape, null and alignment errors before any launch; zero rows is a no-op
    vp, ci = ctypes.c_void_p, ctypes.c_int

    def lin(x, rows, k, ws, bs, ys, ns, n_out=None):
        n_out = len(ws) if n_out is None else n_out
        m = max(len(ws), 1)
        return lib.esa_linear_f32(x, rows, k, n_out, (vp * m)(*ws), (vp * m)(*bs), (vp * m)(*ys), (ci * m)(*ns),
                                  None)
    assert lin(16, 10, 128, [16], [None], [16], [64], n_out=0) == -2
    assert lin(16, 10, 128, [16] * 4, [None] * 4, [16] * 4, [64] * 4) == -2
    assert lin(16, 10, 120, [16], [None], [16], [64]) == -2          # K % 16
    assert lin(16, 10, 8, [16], [None], [16], [64]) == -2            # K < 16
    assert lin(16, 10, 128, [16], [None], [16], [96]) == -2          # N % 64
    assert lin(16, -1, 128, [16], [None], [16], [64]) == -2
    assert lin(16, 10, 128, [None], [None], [16], [64]) == -1
    assert lin(None, 10, 128, [16], [None], [16], [64]) == -1
    assert lin(16, 10, 128, [24], [None], [16], [64]) == -6
    assert lin(8, 10, 128, [16], [None], [16], [64]) == -6
    assert lib.esa_linear_f32(16, 10, 128, 1, None, None, None, None, None) == -1
    assert lin(None, 0, 128, [16, 32], [None, 16], [16, 48], [64, 128]) == 0
    assert lin(None, 0, 128, [None], [None], [None], [64]) == 0   # empty tensors may have null pointers
    # node plan: size errors, and a planned backward needs only its row statistics
    node, node_plan = _lib.ESA_MASK_NODE, _lib.ESA_MASK_NODE_PLAN
    assert lib.esa_node_plan_size(100, 100, -1, ctypes.byref(n)) == -2
    assert lib.esa_node_plan_size(100, 100, 500, ctypes.byref(n)) == 0 and n.value > 500 * 8
    m = ctypes.c_size_t(0)
    assert lib.esa_varlen_attn_workspace_size(100, 100, 16, 16, bf16, node, 500, 1, ctypes.byref(n)) == 0
    assert lib.esa_varlen_attn_workspace_size(100, 100, 16, 16, bf16, node_plan, 500, 1, ctypes.byref(m)) == 0
    assert 0 < m.value < n.value
    assert lib.esa_node_plan_build(None, None, None, None, 1, 100, 100, 0, 256, 1 << 20, None) == -1


def test_short_plans_are_refused_before_launch():
    """A plan is passed to the C ABI without its size and read at the offsets the call's token counts give:
    the Python boundary refuses a plan smaller than those counts need (one built for a smaller batch)."""
    from mind_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    import torch
    from mind_amd.esa import attention as A
    tq = 1000
    indptr = torch.zeros(tq + 1, dtype=torch.int32)
    indices = torch.zeros(50, dtype=torch.int32)
    sym, full = A.edge_plan_bytes(tq, True), A.edge_plan_bytes(tq, False)
    assert 0 < A.edge_plan_bytes(tq // 2, True) < sym < full
    with pytest.raises(ValueError, match="edge_plan holds"):
        A._mask_args(tq, None, None, None, None, edge_plan=torch.empty(sym - 1, dtype=torch.uint8))
    with pytest.raises(ValueError, match="distinct key segments"):
        A._mask_args(tq, None, None, None, None, edge_plan=torch.empty(sym, dtype=torch.uint8), symmetric=False)
    need = A.node_plan_bytes(tq, tq, indices.numel())
    with pytest.raises(ValueError, match="adj_plan holds"):
        A._mask_args(tq, None, None, indptr, indices, adj_plan=torch.empty(need - 1, dtype=torch.uint8))
    # plans of the right size get past the size check (then the device check refuses host tensors)
    with pytest.raises(ValueError, match="device tensor"):
        A._mask_args(tq, None, None, None, None, edge_plan=torch.empty(sym, dtype=torch.uint8))
    with pytest.raises(ValueError, match="device tensor"):
        A._mask_args(tq, None, None, indptr, indices, adj_plan=torch.empty(need, dtype=torch.uint8))
