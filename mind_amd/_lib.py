"""ctypes binding of ``libesa_hip.so`` (the C ABI in ``include/esa_hip.h``).

The library is loaded after ``torch`` so that it binds to the HIP runtime
torch already mapped (both carry the soname ``libamdhip64.so.7``): device
pointers and streams from torch are then valid inside the library.  There is
no fallback: if the library is missing or the process has no GPU, every entry
point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

# MIND_AMD_LIB selects another build of the library (same C ABI).
LIB_PATH = Path(os.environ.get("MIND_AMD_LIB") or Path(__file__).resolve().parent / "lib" / "libesa_hip.so")

ESA_F32 = 0
ESA_BF16 = 1
ESA_MASK_NONE = 0
ESA_MASK_EDGE = 1
ESA_MASK_NODE = 2
ESA_MASK_EDGE_PLAN = 3
ESA_MASK_NODE_PLAN = 4

ERRORS = {
    -1: "ESA_ERR_NULL (a required pointer is null)",
    -2: "ESA_ERR_SHAPE (a size or count is out of range)",
    -3: "ESA_ERR_HEAD_DIM (head_dim must be 16, 24, 32 or 64)",
    -4: "ESA_ERR_WORKSPACE (workspace too small)",
    -5: "ESA_ERR_DTYPE (unsupported dtype)",
    -6: "ESA_ERR_ALIGN (pointer not 16-byte aligned)",
    -7: "ESA_ERR_MASK (unknown mask kind, or the edge mask without total_q == total_k)",
    -8: "ESA_ERR_SCRATCH (the call needs more scratch than the no-allocation entry point's static buffer)",
    -9: "ESA_ERR_DROPOUT (dropout_p outside [0, 1))",
}

_c_int, _c_i64, _c_f, _c_sz, _vp = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p
_c_u64 = ctypes.c_ulonglong

_PROTOS = {
    "esa_version": (ctypes.c_char_p, []),
    "esa_varlen_attn_workspace_size": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                                ctypes.POINTER(_c_sz)]),
    # q k v cu_q cu_k | batch tq tk maxq maxk heads hd dtype | scale dropout_p seed | mask_kind a b n |
    # out lse ws bytes stream
    "esa_varlen_attn_fwd": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                     _c_int, _c_f, _c_f, _c_u64, _c_int, _vp, _vp, _c_int, _vp, _vp, _vp, _c_sz, _vp]),
    # dout q k v out lse cu_q cu_k | batch tq tk maxq maxk heads hd dtype | scale dropout_p seed |
    # mask_kind a b n | dq dk dv ws bytes stream
    "esa_varlen_attn_bwd": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                     _c_int, _c_int, _c_int, _c_f, _c_f, _c_u64, _c_int, _vp, _vp, _c_int, _vp, _vp,
                                     _vp, _vp, _c_sz, _vp]),
    "esa_noalloc_scratch_bytes": (_c_sz, []),
    # as esa_varlen_attn_fwd without workspace / workspace_bytes
    "esa_varlen_attn_fwd_noalloc": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                             _c_int, _c_int, _c_f, _c_f, _c_u64, _c_int, _vp, _vp, _c_int, _vp, _vp,
                                             _vp]),
    "esa_edge_mask_dense": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _vp]),
    # plan tq tk direction indptr out stream
    "esa_edge_plan_decode": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp]),
    "esa_node_plan_sections": (_c_int, [_c_int, _c_int, _c_int, ctypes.POINTER(_c_sz)]),
    # batch k_seeds total_k heads head_dim dtype backward bytes
    "esa_pma_workspace_size": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                        ctypes.POINTER(_c_sz)]),
    # q k v cu_k | batch k_seeds tk maxk heads hd dtype | scale dropout_p seed | out lse ws bytes stream
    "esa_pma_fwd": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_f,
                             _c_f, _c_u64, _vp, _vp, _vp, _c_sz, _vp]),
    # dout q k v out lse cu_k | batch k_seeds tk maxk heads hd dtype | scale dropout_p seed | dq dk dv ws bytes
    # stream
    "esa_pma_bwd": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                             _c_int, _c_f, _c_f, _c_u64, _vp, _vp, _vp, _vp, _c_sz, _vp]),
    "esa_edge_gather": (_c_int, [_vp, _vp, _vp, _c_i64, _c_int, _c_int, _c_int, _vp, _vp]),
    "esa_csr_workspace_size": (_c_int, [_c_i64, _c_int, ctypes.POINTER(_c_sz)]),
    "esa_csr_build": (_c_int, [_vp, _c_i64, _c_int, _vp, _vp, _vp, _c_sz, _vp]),
    "esa_csr_segment_sum": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _vp]),
    "esa_csr_segment_minmax": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_i64, _vp, _vp, _vp]),
    "esa_token_budget_pack_workspace_size": (_c_int, [_c_int, ctypes.POINTER(_c_sz)]),
    "esa_edge_plan_size": (_c_int, [_c_int, _c_int, _c_int, ctypes.POINTER(_c_sz)]),
    "esa_edge_plan_build": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _c_sz, _vp]),
    "esa_node_plan_size": (_c_int, [_c_int, _c_int, _c_int, ctypes.POINTER(_c_sz)]),
    "esa_node_plan_build": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _c_sz, _vp]),
    # counts num_graphs budget | batch_of_graph batch_start num_batches ws bytes stream
    "esa_token_budget_pack": (_c_int, [_vp, _c_int, _c_i64, _vp, _vp, _vp, _vp, _c_sz, _vp]),
    "esa_edge_gather_bwd": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _vp]),
    "esa_edge_gather_add": (_c_int, [_vp, _c_i64, _vp, _c_i64, _vp, _vp, _vp, _c_i64, _c_int, _c_int, _c_int, _vp,
                                     _vp]),
    "esa_mish_fwd": (_c_int, [_vp, _vp, _c_i64, _c_int, _vp, _vp]),
    "esa_mish_bwd": (_c_int, [_vp, _vp, _c_i64, _c_int, _vp, _vp]),
    # x x_dtype w b rows features eps y y_dtype y_lp mean rstd stream
    "esa_layer_norm_fwd": (_c_int, [_vp, _c_int, _vp, _vp, _c_i64, _c_int, _c_f, _vp, _c_int, _vp, _vp, _vp, _vp]),
    "esa_layer_norm_bwd_workspace_size": (_c_int, [_c_i64, _c_int, ctypes.POINTER(_c_sz)]),
    # x x_dtype w mean rstd dy dy_dtype dy_lp dx_add rows features dx dw db ws bytes stream
    "esa_layer_norm_bwd": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _c_i64, _c_int, _vp, _vp, _vp,
                                    _vp, _c_sz, _vp]),
    "esa_column_sum_workspace_size": (_c_int, [_c_i64, _c_int, ctypes.POINTER(_c_sz)]),
    "esa_column_sum": (_c_int, [_vp, _c_int, _c_i64, _c_int, _vp, _vp, _c_sz, _vp]),
    # z grad rows cols dtype dz dbias ws bytes stream
    "esa_mish_bwd_colsum": (_c_int, [_vp, _vp, _c_i64, _c_int, _c_int, _vp, _vp, _vp, _c_sz, _vp]),
    # x rows in n_out | weight[] bias[] y[] out_features[] stream
    "esa_linear_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                                ctypes.POINTER(_vp), ctypes.POINTER(_c_int), _vp]),
    "esa_mab_residual_fwd": (_c_int, [_vp, _vp, _vp, _c_i64, _c_int, _vp, _vp]),
    "esa_mab_residual_bwd": (_c_int, [_vp, _vp, _c_i64, _c_int, _vp, _vp, _vp]),
    "esa_profile_enable": (_c_int, [_c_int]),
    "esa_profile_collect": (_c_int, [ctypes.POINTER(_c_f), ctypes.POINTER(_c_int), _c_int]),
    "esa_profile_kernel_name": (ctypes.c_char_p, [_c_int]),
}

PROFILE_KERNELS = 23

_lock = threading.Lock()
_lib = None


class EsaError(RuntimeError):
    """Nonzero status from a C-ABI entry point."""


def load() -> ctypes.CDLL:
    """Load (once) and return the library with argument types set."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise EsaError(f"{LIB_PATH} is not built; run `python -m mind_amd._build` (hipcc, gfx950)")
            lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_LOCAL)
            for name, (res, args) in _PROTOS.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def exported_symbols() -> list[str]:
    return list(_PROTOS)


def check(rc: int, what: str) -> None:
    if rc != 0:
        if rc < 0:
            raise EsaError(f"{what}: {ERRORS.get(rc, rc)}")
        raise EsaError(f"{what}: HIP error {rc}")


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise EsaError("the MI355X kernels take device tensors; got a tensor on " + str(t.device))


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def version() -> str:
    return load().esa_version().decode()


_profiling = False


def profile_enable(on: bool) -> None:
    global _profiling
    check(load().esa_profile_enable(int(on)), "esa_profile_enable")
    _profiling = bool(on)


def profiling() -> bool:
    """Whether this process turned the per-kernel profiling hook on (profile_enable)."""
    return _profiling


def profile_collect() -> dict[str, tuple[float, int]]:
    """Per-kernel (total ms, launches) recorded since the last collect (synchronises)."""
    lib = load()
    ms = (_c_f * PROFILE_KERNELS)()
    n = (_c_int * PROFILE_KERNELS)()
    check(lib.esa_profile_collect(ms, n, PROFILE_KERNELS), "esa_profile_collect")
    return {lib.esa_profile_kernel_name(i).decode(): (float(ms[i]), int(n[i])) for i in range(PROFILE_KERNELS)}
