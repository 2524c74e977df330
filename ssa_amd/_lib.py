"""ctypes bindings of libssa_hip.so (the C ABI declared in include/ssa_hip.h).

The library is built in-tree by ``ssa_amd._build.build()`` (or
``__graft_entry__.build()``).  Nothing here falls back to another
implementation: a missing library or a non-HIP tensor raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
# In-tree build; SSA_HIP_LIBRARY may point at another build of the same ABI.
LIB_PATH = os.environ.get("SSA_HIP_LIBRARY") or os.path.join(_HERE, "libssa_hip.so")

SSA_OK = 0
SSA_ERR_INVALID_ARGUMENT = 1
SSA_ERR_UNSUPPORTED = 2
SSA_ERR_WORKSPACE = 3
SSA_ERR_HIP = 4

DTYPE_F32 = 0
DTYPE_BF16 = 1
INDEX_I32 = 0
INDEX_I64 = 1
MASK_NONE = 0
MASK_CAUSAL = 1
MASK_DENSE = 2
ROPE_BY_POSITION = 0
ROPE_BY_HEAD = 1

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/ssa_hip.h one to one.
SIGNATURES = {
    "ssa_version": (_int, []),
    "ssa_status_str": (ctypes.c_char_p, [_int]),
    "ssa_last_error": (ctypes.c_char_p, []),
    "ssa_rope": (
        _int, [_vp, _int, _i64, _i64, _int, _int, _i64, _i64, _i64, _vp, _vp, _int, _i64, _i64,
               _i64, _int, _int, _int, _vp, _int, _i64, _i64, _i64, _vp]),
    "ssa_route_vectors": (
        _int, [_vp, _int, _i64, _i64, _int, _int, _int, _i64, _i64, _i64, _vp, _int, _vp, _vp]),
    "ssa_normalize_rows": (_int, [_vp, _i64, _int, _vp, _vp]),
    "ssa_code_topk_workspace_bytes": (_sz, [_i64, _int, _i64, _int]),
    "ssa_code_topk": (
        _int, [_vp, _i64, _int, _i64, _vp, _int, _int, _flt, _int, _vp, _vp, _sz, _vp]),
    "ssa_route_workspace_bytes": (_sz, [_i64, _i64, _int, _int, _int]),
    "ssa_route_codes": (
        _int,
        [_vp, _vp, _int, _i64, _i64, _int, _int, _int, _i64, _i64, _i64, _i64, _i64, _i64,
         _vp, _vp, _vp, _int, _int, _int, _int, _flt, _vp, _vp, _vp, _sz, _vp]),
    "ssa_index_workspace_bytes": (_sz, [_i64, _i64, _int, _int, _int]),
    "ssa_build_index": (_int, [_vp, _i64, _i64, _int, _int, _int, _vp, _vp, _vp, _sz, _vp]),
    "ssa_query_order_workspace_bytes": (_sz, [_i64, _i64, _int, _int]),
    "ssa_query_order": (_int, [_vp, _i64, _i64, _int, _int, _int, _vp, _vp, _sz, _vp]),
    "ssa_select": (
        _int,
        [_vp, _vp, _int, _i64, _i64, _int, _int, _int, _i64, _i64, _i64, _i64, _i64, _i64,
         _vp, _int, _vp, _vp, _int, _int, _int, _int, _vp, _i64, _i64, _flt, _int, _vp, _vp,
         _int, _vp, _vp, _vp, _sz, _vp]),
    "ssa_select_workspace_bytes": (_sz, [_i64, _i64, _int, _int]),
    "ssa_select_workspace_layout": (_int, [_i64, _i64, _int, _sz, _int, _vp]),
    "ssa_select_block": (
        _int,
        [_vp, _vp, _int, _i64, _i64, _i64, _i64, _int, _int, _int, _i64, _i64, _i64, _i64, _i64,
         _i64, _vp, _int, _vp, _vp, _int, _int, _int, _int, _vp, _i64, _i64, _flt, _int, _vp, _vp,
         _int, _vp, _vp, _vp, _sz, _vp]),
    "ssa_select_noalloc_scratch_bytes": (_sz, []),
    "ssa_select_block_noalloc": (
        _int,
        [_vp, _vp, _int, _i64, _i64, _i64, _i64, _int, _int, _int, _i64, _i64, _i64, _i64, _i64,
         _i64, _vp, _int, _vp, _vp, _int, _int, _int, _int, _vp, _i64, _i64, _flt, _int, _vp, _vp,
         _int, _vp, _vp, _vp]),
    "ssa_decode_prepare_bytes": (_sz, [_int, _int, _int]),
    "ssa_decode_prepare": (_int, [_vp, _int, _int, _int, _vp, _sz, _vp]),
    "ssa_decode_workspace_bytes": (_sz, [_i64, _i64, _int, _int, _int, _int, _int, _int]),
    "ssa_decode_step": (
        _int,
        [_vp, _vp, _vp, _int, _i64, _i64, _int, _int, _int, _i64, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp,
         _vp, _int, _int, _int, _int, _flt, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _int, _flt,
         _flt, _int, _vp, _vp, _int, _i64, _i64, _i64, _vp, _sz, _vp]),
    "ssa_sparse_attention": (
        _int,
        [_vp, _vp, _vp, _int, _i64, _i64, _int, _int, _int, _i64, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _i64, _vp, _int, _int, _i64, _i64, _i64, _flt, _int, _vp, _vp, _vp, _int,
         _i64, _i64, _i64, _vp, _vp, _vp, _sz, _vp]),
    "ssa_sparse_attention_workspace_bytes": (_sz, [_int, _i64, _i64, _int, _int, _int, _int]),
    "ssa_sparse_attention_block": (
        _int,
        [_vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _int, _int, _int, _i64, _i64, _i64, _i64,
         _i64, _i64, _i64, _i64, _i64, _vp, _int, _int, _i64, _i64, _i64, _flt, _int, _vp, _vp,
         _vp, _int, _i64, _i64, _i64, _vp, _vp, _vp, _sz, _vp]),
    "ssa_block_indices": (
        _int,
        [_vp, _int, _i64, _i64, _int, _int, _i64, _i64, _i64, _int, _int, _vp, _int, _i64, _i64,
         _i64, _vp, _vp]),
    "ssa_block_sparse_attention": (
        _int,
        [_vp, _vp, _vp, _int, _i64, _i64, _int, _int, _int, _i64, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _i64, _vp, _int, _int, _int, _i64, _i64, _i64, _flt, _vp, _int, _i64, _i64,
         _i64, _vp, _vp]),
    "ssa_sparse_attention_backward": (
        _int,
        [_vp, _vp, _vp, _int, _i64, _i64, _int, _int, _int, _i64, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _i64, _vp, _int, _int, _i64, _i64, _i64, _flt, _int, _vp, _vp, _int, _i64,
         _i64, _i64, _vp, _int, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ssa_sparse_attention_backward_workspace_bytes": (_sz, [_int, _int, _i64, _i64, _int, _int, _int]),
    "ssa_sparse_attention_backward_routed": (
        _int,
        [_vp, _vp, _vp, _int, _i64, _i64, _int, _int, _int, _i64, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _i64, _vp, _int, _int, _i64, _i64, _i64, _flt, _int, _vp, _vp, _int, _i64,
         _i64, _i64, _vp, _int, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp,
         _vp, _int, _vp, _int, _vp, _vp, _int, _int, _vp, _sz, _vp]),
    "ssa_sparse_attention_backward_routed_workspace_bytes": (
        _sz, [_int, _int, _i64, _i64, _int, _int, _int, _int, _int, _int, _int, _i64]),
}

_lib = None
_lock = threading.Lock()


class SSAError(RuntimeError):
    """A libssa_hip call returned a non-zero status."""

    def __init__(self, fn: str, status: int, detail: str):
        self.status = status
        super().__init__(f"{fn}: {detail} (status {status})")


def load(path: Optional[str] = None):
    """Load libssa_hip.so once and bind every exported entry point."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise RuntimeError(
                f"libssa_hip.so is not built ({p}); run `python -c 'import __graft_entry__ as g; "
                "g.build()'` or `python ssa_amd/_build.py`")
        L = ctypes.CDLL(p)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = L
        return L


def call(name: str, *args) -> None:
    L = load()
    st = getattr(L, name)(*args)
    if st != SSA_OK:
        detail = (L.ssa_last_error() or b"").decode(errors="replace")
        if st == SSA_ERR_UNSUPPORTED:
            raise NotImplementedError(f"{name}: {detail}")
        raise SSAError(name, st, detail)


def ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_device(*tensors: torch.Tensor) -> None:
    """The product path runs on HIP devices only: no CPU fallback exists."""
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(
                f"ssa_amd runs on AMD GPUs (HIP); got a tensor on '{t.device}'. "
                "Move inputs to the GPU.")


def elem_dtype(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return DTYPE_F32
    if t.dtype == torch.bfloat16:
        return DTYPE_BF16
    raise NotImplementedError(f"dtype {t.dtype} is not supported (float32, bfloat16)")


def index_dtype(t: torch.Tensor) -> int:
    if t.dtype == torch.int64:
        return INDEX_I64
    if t.dtype == torch.int32:
        return INDEX_I32
    raise TypeError(f"indices must be int64 or int32, got {t.dtype}")
