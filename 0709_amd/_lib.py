"""ctypes binding of the gfx950 C ABI declared in include/atlas0709.h.

The shared library is loaded from ``_lib/libatlas0709_hip.so`` inside this
package.  Every public operation of the package goes through these entry
points; there is no other implementation, so a missing library or a tensor
that is not on a HIP device raises instead of computing elsewhere.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path
from typing import Sequence

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libatlas0709_hip.so"

ATLAS_OK = 0
ATLAS_EINVAL = -1
ATLAS_EUNSUPPORTED = -2
ATLAS_EHIP_BASE = -1000

DTYPE_F16 = 0
DTYPE_BF16 = 1
DTYPE_F32 = 2

MASK_NONE = 0
MASK_TREE = 1
MASK_CAUSAL = 2

MAX_LAYERS_PER_LAUNCH = 64
ATTN_SCRATCH_BYTES = 16777216  # device scratch of atlas_tree_verify_attn_noalloc
MAX_INLINE_ITEMS = 64

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_VPP = ctypes.POINTER(ctypes.c_void_p)


class AttnWork(ctypes.Structure):
    """atlas_attn_work_t (64 bytes)."""
    _fields_ = [
        ("req", _c_i32),
        ("kv_head", _c_i32),
        ("row_start", _c_i32),
        ("num_rows", _c_i32),
        ("kv_start", _c_i32),
        ("kv_end", _c_i32),
        ("partial_row", _c_i32),
        ("qo_start", _c_i32),
        ("qo_len", _c_i32),
        ("kv_len", _c_i32),
        ("mask_col_start", _c_i32),
        ("page_offset", _c_i32),
        ("pad", _c_i32 * 4),
    ]


class AttnMerge(ctypes.Structure):
    """atlas_attn_merge_t (32 bytes)."""
    _fields_ = [
        ("req", _c_i32),
        ("kv_head", _c_i32),
        ("row_start", _c_i32),
        ("num_rows", _c_i32),
        ("partial_row", _c_i32),
        ("num_splits", _c_i32),
        ("pad0", _c_i32),
        ("pad1", _c_i32),
    ]


# name -> argtypes; restype is c_int (a status) unless _RESTYPES says otherwise.
_SIGNATURES: dict[str, list] = {
    "atlas_abi_version": [],
    "atlas_kv_move_slots": [_VPP, _VPP, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp, _c_i64, _vp],
    "atlas_kv_append": [
        _VPP, _VPP, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _VPP, _VPP, _c_i64, _vp, _c_i64, _c_i64, _vp,
    ],
    "atlas_kv_commit_paged": [
        _VPP, _VPP, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _vp, _vp, _c_i64,
        ctypes.c_int, _vp, ctypes.c_size_t, _vp,
    ],
    "atlas_kv_commit_paged_host": [
        _VPP, _VPP, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp,
        ctypes.POINTER(_c_i32), ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_i64, _vp,
    ],
    "atlas_tree_verify_attn": [
        _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _vp, ctypes.c_int, _vp, _vp, ctypes.c_int,
        _vp, ctypes.c_int, _vp, _vp, ctypes.c_int, _c_i64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ctypes.c_int, ctypes.c_float, ctypes.c_int, _vp, _c_i64, _c_i64, _vp, _vp, ctypes.c_size_t, _vp,
    ],
    "atlas_tree_verify_attn_append": [
        _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _vp, ctypes.c_int, _vp, _vp, ctypes.c_int,
        _vp, ctypes.c_int, _vp, _vp, ctypes.c_int, _c_i64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ctypes.c_int, ctypes.c_float, ctypes.c_int, _vp, _c_i64, _c_i64, _vp, _vp, ctypes.c_size_t,
        _vp, _vp, _c_i64, _c_i64, _vp, _vp, _c_i64, _vp,
    ],
    "atlas_tree_verify_attn_noalloc": [
        _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _vp, ctypes.c_int, _vp, _vp, ctypes.c_int,
        _vp, ctypes.c_int, _vp, _vp, ctypes.c_int, _c_i64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ctypes.c_int, ctypes.c_float, ctypes.c_int, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp,
    ],
    "atlas_attn_page_windows": [_vp, ctypes.c_int, _vp, ctypes.c_int, _vp, _vp],
    "atlas_prune_pages": [_vp, _vp, _c_i64, _vp, _c_i64, _c_i64, _vp, _vp, _vp],
    "atlas_mark_pages": [_vp, _c_i64, _vp, _c_i64, _c_i64, _vp],
    "atlas_alloc_decode_slots": [_vp, _vp, _vp, _c_i64, ctypes.c_int, _vp, _vp],
    "atlas_alloc_extend_slots": [_vp, _vp, _vp, _vp, _c_i64, ctypes.c_int, _vp, _vp],
    "atlas_paged_metadata": [_vp, _vp, _vp, ctypes.c_int, _c_i64, _c_i64, ctypes.c_int, _vp, _vp, _vp],
    "atlas_pool_prepare_frontier": [
        _vp, ctypes.c_int, _vp, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp, _vp, _c_i64,
        _vp, _vp, _vp, _vp, _c_i64, _vp, _c_i64, _vp,
    ],
    "atlas_gather_logprobs_workspace_bytes": [_c_i64, _c_i64],
    "atlas_gather_logprobs": [
        _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i64, ctypes.c_int, _vp, _vp, _c_i64, _vp, _vp, _vp,
        ctypes.c_size_t, _vp,
    ],
    "atlas_frontier_workspace_bytes": [_c_i64, _c_i64, ctypes.c_int],
    "atlas_frontier_topk": [
        _vp, _c_i64, _c_i64, _c_i64, ctypes.c_int, _vp, _c_i64, ctypes.c_int, _vp, ctypes.c_int, _c_i64, _vp,
        _c_i64, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp,
    ],
    "atlas_candidate_select": [
        _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, ctypes.c_int, _c_i64, _vp, _c_i64, _vp, _c_i64, _vp, _vp, _vp, _vp,
    ],
}
# entry points whose return value is not an int status
_RESTYPES: dict[str, type] = {
    "atlas_frontier_workspace_bytes": ctypes.c_int64,
    "atlas_gather_logprobs_workspace_bytes": ctypes.c_int64,
}

FRONTIER_NONE = -1
FRONTIER_ORDER = 0
FRONTIER_ORDER_BY_ROOT = 1
FRONTIER_SELECT_GLOBAL = 2
FRONTIER_SELECT_PER_ROOT = 3
FRONTIER_PACK = 4
MAX_FRONTIER_K = 32
MAX_FRONTIER_CANDIDATES = 4096

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def exported_symbols() -> list[str]:
    return ["atlas_last_error", *_SIGNATURES]


def load() -> ctypes.CDLL:
    """Load the library (once) and declare the signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"HIP library {LIB_PATH} is missing; run __graft_entry__.build() "
                "(or python 0709_amd/build.py) first"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.atlas_last_error.restype = ctypes.c_char_p
        lib.atlas_last_error.argtypes = []
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
            fn.argtypes = argtypes
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    """Raise for a non-zero status using the library's last error message."""
    if rc == ATLAS_OK:
        return
    msg = load().atlas_last_error().decode("utf-8", "replace")
    if rc == ATLAS_EINVAL:
        raise ValueError(f"{what}: {msg}")
    if rc == ATLAS_EUNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: HIP error {ATLAS_EHIP_BASE - rc}: {msg}")


def require_device(*tensors: torch.Tensor | None, what: str) -> torch.device:
    """All tensors must live on one HIP device; returns it."""
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"{what} runs on the MI355X HIP kernels and needs HIP device tensors, "
                f"got a tensor on {t.device}"
            )
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f"{what}: tensors are on different devices ({device} and {t.device})")
    if device is None:
        raise ValueError(f"{what}: no tensor given")
    return device


def stream_of(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def ptr_array(values: Sequence[int]) -> ctypes.Array:
    arr = (ctypes.c_void_p * max(1, len(values)))()
    for i, v in enumerate(values):
        arr[i] = v
    return arr


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return DTYPE_F16
    if dtype == torch.bfloat16:
        return DTYPE_BF16
    if dtype == torch.float32:
        return DTYPE_F32
    raise TypeError(f"unsupported dtype {dtype}; expected float16 or bfloat16")
