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


class SlotPath(ctypes.Structure):
    """atlas_slot_path_t (16 bytes)."""
    _fields_ = [("slots", ctypes.c_void_p), ("len", _c_i64)]


PRUNE_MAX_PATHS = 64
PRUNE_PATHS_MAX_PAGES = 524288  # atlas_prune_pages_paths: one workgroup's LDS bitmap


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
        _VPP, _VPP, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _VPP, _VPP, _c_i64, _vp, _c_i64,
        _c_i64, _vp,
    ],
    "atlas_kv_commit_paged": [
        _VPP, _VPP, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _vp, _vp, _c_i64,
        ctypes.c_int, _vp, ctypes.c_size_t, _vp,
    ],
    "atlas_kv_commit_paged_host": [
        _VPP, _VPP, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp,
        ctypes.POINTER(_c_i32), ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_i64, _vp,
    ],
    "atlas_tree_verify_attn": [
        _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _vp, ctypes.c_int, _vp, _vp,
        ctypes.c_int,
        _vp, ctypes.c_int, _vp, _vp, ctypes.c_int, _c_i64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ctypes.c_int, ctypes.c_float, ctypes.c_int, _vp, _c_i64, _c_i64, _vp, _vp, ctypes.c_size_t, _vp,
    ],
    "atlas_tree_verify_attn_append": [
        _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _vp, ctypes.c_int, _vp, _vp,
        ctypes.c_int,
        _vp, ctypes.c_int, _vp, _vp, ctypes.c_int, _c_i64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ctypes.c_int, ctypes.c_float, ctypes.c_int, _vp, _c_i64, _c_i64, _vp, _vp, ctypes.c_size_t,
        _vp, _vp, _c_i64, _c_i64, _vp, _vp, _c_i64, _vp,
    ],
    "atlas_tree_verify_attn_noalloc": [
        _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _vp, ctypes.c_int, _vp, _vp,
        ctypes.c_int,
        _vp, ctypes.c_int, _vp, _vp, ctypes.c_int, _c_i64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ctypes.c_int, ctypes.c_float, ctypes.c_int, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp,
    ],
    "atlas_attn_page_windows": [_vp, ctypes.c_int, _vp, ctypes.c_int, _vp, _vp],
    "atlas_attn_plan_install": [_vp, ctypes.c_int, _vp, _c_i64, _vp, _vp, _c_i64, _vp, ctypes.c_int, _vp, _vp],
    "atlas_prune_pages": [_vp, _vp, _c_i64, _vp, _c_i64, _c_i64, _vp, _vp, _vp],
    "atlas_prune_pages_paths": [_vp, _vp, _c_i64, _vp, ctypes.c_int, ctypes.c_uint64, _c_i64, _vp, _vp, _vp],
    "atlas_mark_pages": [_vp, _c_i64, _vp, _c_i64, _c_i64, _vp],
    "atlas_alloc_decode_slots": [_vp, _vp, _vp, _c_i64, ctypes.c_int, _vp, _vp],
    "atlas_alloc_extend_slots": [_vp, _vp, _vp, _vp, _c_i64, ctypes.c_int, _vp, _vp],
    "atlas_paged_metadata": [_vp, _vp, _vp, ctypes.c_int, _c_i64, _c_i64, ctypes.c_int, _vp, _vp, _vp],
    "atlas_pool_prepare_frontier": [
        _vp, ctypes.c_int, _vp, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp, _vp, _c_i64,
        _vp, _vp, _vp, _vp, _c_i64, _vp, _vp,
    ],
    "atlas_gather_i64": [_vp, ctypes.c_int, _vp, _vp],
    "atlas_prune_pages_paths_gather": [
        _vp, _vp, _c_i64, _vp, ctypes.c_int, ctypes.c_uint64, _c_i64, _vp, _vp, _vp, ctypes.c_int, _vp, _vp,
    ],
    "atlas_pool_prepare_frontier_host": [
        _vp, _vp, _vp, ctypes.c_int, _vp, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp, _vp,
        _c_i64, _vp, _vp, _vp, _vp, _c_i64, _vp, _vp, _vp,
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
    "atlas_tree_spec_bytes": [ctypes.c_int32, ctypes.c_int32, _c_i64, ctypes.c_int32],
    "atlas_tree_mask_fill": [_vp, ctypes.c_int32, _c_i64, _vp, _vp],
    "atlas_tree_spec_upload": [_vp, _c_i64, ctypes.c_int32, _c_i64, _vp, _vp, _vp],
    "atlas_route_select": [
        _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, ctypes.c_int, _vp, _vp, _vp, _vp,
        ctypes.c_int, ctypes.c_double, ctypes.c_int, ctypes.c_double, _c_i64, _vp, _vp, _vp, _vp, _vp,
    ],
    "atlas_tree_spec_build": [
        _vp, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _c_i64, ctypes.c_int32, _vp, _c_i64, _vp, _vp, _vp,
    ],
}
# entry points whose return value is not an int status
_RESTYPES: dict[str, type] = {
    "atlas_frontier_workspace_bytes": ctypes.c_int64,
    "atlas_gather_logprobs_workspace_bytes": ctypes.c_int64,
    "atlas_tree_spec_bytes": ctypes.c_int64,
}

GATHER_MAX_SEGMENTS = 32
FRONTIER_BAD_DESCRIPTOR = 1
FRONTIER_BAD_LAYOUT = 2
FRONTIER_DUPLICATE_SLOT = 4
FRONTIER_COW_OVERLAP = 8
FRONTIER_MAX_HOST_ROUTES = 24
SELECT_MAX_ROUTES = 64
SELECT_MAX_DEPTH = 16
SELECT_MAX_ENTRIES = 512
SELECT_TARGET_BEST = 0
SELECT_FIRST_ROUTE = 1
ROUND_NONE = 0
ROUND_F16 = 1
ROUND_BF16 = 2

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


# torch's current raw stream handle, without building a Stream object
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> ctypes.c_void_p:
    """The device's current HIP stream, as a launch argument."""
    if _RAW_STREAM is not None:
        idx = device.index
        return ctypes.c_void_p(_RAW_STREAM(torch.cuda.current_device() if idx is None else idx))
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


class HostStaging:
    """Pinned host memory (``hipHostMalloc``, mapped and coherent, so kernels
    can also read it in place) for small host-to-device uploads, handed out
    from a ring of four quarters.

    A quarter is written again only after the copies queued from it have run:
    when the ring leaves a quarter it records an event on the stream that
    copied from it, and waits for that event before it enters the quarter
    again (a quarter that more than one stream copied from waits for those
    devices instead).  torch's pinned allocator records an event per copy;
    this records one per quarter, so a small upload costs one numpy write and
    one asynchronous copy."""

    def __init__(self, nbytes: int = 4 << 20) -> None:
        self.quarter = (nbytes // 4) & ~63
        self.nbytes = 4 * self.quarter
        hip = _hip_runtime()
        p = ctypes.c_void_p()
        rc = hip.hipHostMalloc(ctypes.byref(p), ctypes.c_size_t(self.nbytes), ctypes.c_uint(MappedReadback._FLAGS))
        if rc != 0 or not p.value:
            raise RuntimeError(f"hipHostMalloc of {self.nbytes} staging bytes failed ({rc})")
        self.base = p.value
        d = ctypes.c_void_p()
        rc = hip.hipHostGetDevicePointer(ctypes.byref(d), ctypes.c_void_p(p.value), ctypes.c_uint(0))
        if rc != 0 or not d.value:
            raise RuntimeError(f"hipHostGetDevicePointer of the staging ring failed ({rc})")
        self.device_base = d.value
        self.memcpy = _hip_runtime().hipMemcpyAsync
        buf = (ctypes.c_uint8 * self.nbytes).from_address(p.value)
        self.host = torch.frombuffer(buf, dtype=torch.uint8)
        self.host_np = self.host.numpy()
        self.cur = 0  # the quarter being filled; pos never leaves it but by _leave/_enter
        self.pos = 0
        self.events: list = [None] * 4
        self.users: list[set] = [set() for _ in range(4)]
        self.lock = threading.Lock()

    def _enter(self, q: int) -> None:
        ev = self.events[q]
        if isinstance(ev, torch.cuda.Event):
            ev.synchronize()
        elif ev is not None:
            for dev in ev:
                torch.cuda.synchronize(dev)
        self.events[q] = None
        self.users[q] = set()

    def _leave(self, q: int) -> None:
        users = self.users[q]
        if not users:
            return
        if len(users) == 1:
            (dev, raw), = users
            stream = torch.cuda.current_stream(dev)
            if stream.cuda_stream == raw:
                ev = torch.cuda.Event()
                ev.record(stream)
                self.events[q] = ev
                return
        self.events[q] = sorted({dev for dev, _ in users})

    def upload(self, host: "np.ndarray", device: torch.device, out: torch.Tensor | None = None) -> torch.Tensor:
        """A device copy (uint8, ``host.nbytes`` long) of a numpy array,
        queued on the device's current stream; with ``out`` (a contiguous
        device tensor of ``host.nbytes`` bytes) the bytes land there and
        ``out`` is returned."""
        import numpy as np

        nbytes = int(host.nbytes)
        src = np.ascontiguousarray(host).reshape(-1).view(np.uint8)
        if out is not None:
            if not out.is_contiguous() or out.numel() * out.element_size() != nbytes:
                raise ValueError("out must be a contiguous tensor of the array's size")
            dst = out.view(-1).view(torch.uint8)
        if nbytes > self.quarter or nbytes == 0:
            staged = torch.from_numpy(src.copy())
            if out is None:
                return staged.to(device, non_blocking=False)
            dst.copy_(staged)
            return out
        with self.lock:
            start, raw = self._place(src, nbytes, device)
            if out is None:
                out = dst = torch.empty(nbytes, dtype=torch.uint8, device=device)
            # queued on the current stream straight from the pinned bytes
            rc = self.memcpy(dst.data_ptr(), self.base + start, nbytes, _HIP_MEMCPY_H2D, raw)
            if rc != 0:
                raise RuntimeError(f"hipMemcpyAsync of {nbytes} staged bytes failed ({rc})")
        return out

    def _place(self, src, nbytes: int, device: torch.device) -> tuple[int, int]:
        """Write ``src`` (uint8, ``nbytes``) into the ring for work queued
        next on the device's current stream; returns its ring offset (64-byte
        aligned) and the raw stream.  Called with the lock held."""
        idx = torch.cuda.current_device() if device.index is None else device.index
        q = self.cur
        start = self.pos
        if start + nbytes > (q + 1) * self.quarter:
            self._leave(q)
            q = self.cur = (q + 1) % 4
            self._enter(q)
            start = q * self.quarter
        self.host_np[start : start + nbytes] = src
        raw = _RAW_STREAM(idx) if _RAW_STREAM is not None else torch.cuda.current_stream(idx).cuda_stream
        self.users[q].add((idx, raw))
        self.pos = (start + nbytes + 63) & ~63
        return start, raw

    def stage(self, host: "np.ndarray", device: torch.device, launch) -> bool:
        """Copy a numpy array's bytes into the ring and call ``launch(addr)``
        with their device address, under the ring's lock, so the kernel it
        queues on the device's current stream reads them in place (the ring
        is mapped host memory, and that part of it is not written again
        before the work queued after it has run).  False, and no call, when
        the array is empty or larger than a quarter of the ring."""
        import numpy as np

        nbytes = int(host.nbytes)
        if nbytes > self.quarter or nbytes == 0:
            return False
        src = np.ascontiguousarray(host).reshape(-1).view(np.uint8)
        with self.lock:
            start, _ = self._place(src, nbytes, device)
            launch(self.device_base + start)
        return True

    def upload_i64(self, values: Sequence[int], device: torch.device) -> torch.Tensor:
        """``torch.tensor(values, dtype=torch.int64)`` on ``device``."""
        import numpy as np

        return self.upload(np.asarray(values, dtype=np.int64), device).view(torch.int64)


class I64Segment(ctypes.Structure):
    """``atlas_i64_segment_t``: a strided run of int64 values on the device."""

    _fields_ = [("src", ctypes.c_void_p), ("count", ctypes.c_int64), ("stride", ctypes.c_int64)]


class MappedReadback:
    """Pinned host memory the device writes into directly (``hipHostMalloc``
    with the portable, mapped and coherent flags): ``np`` is the host's
    float32 view and ``device_ptr`` the address a kernel stores through.  A
    launch's stores are visible to the host once an event recorded behind the
    launch has completed.  Held until the process ends."""

    _FLAGS = 0x1 | 0x2 | 0x40000000  # hipHostMallocPortable | Mapped | Coherent

    def __init__(self, count: int) -> None:
        import numpy as np

        hip = _hip_runtime()
        self.count = int(count)
        p = ctypes.c_void_p()
        rc = hip.hipHostMalloc(ctypes.byref(p), ctypes.c_size_t(4 * self.count), ctypes.c_uint(self._FLAGS))
        if rc != 0 or not p.value:
            raise RuntimeError(f"hipHostMalloc of {4 * self.count} mapped bytes failed ({rc})")
        d = ctypes.c_void_p()
        rc = hip.hipHostGetDevicePointer(ctypes.byref(d), ctypes.c_void_p(p.value), ctypes.c_uint(0))
        if rc != 0 or not d.value:
            raise RuntimeError(f"hipHostGetDevicePointer failed ({rc})")
        self.device_ptr = ctypes.c_void_p(d.value)
        self.np = np.frombuffer((ctypes.c_float * self.count).from_address(p.value), dtype=np.float32)


_HIP = None
_HIP_MEMCPY_H2D = 1  # hipMemcpyHostToDevice
_STAGING: HostStaging | None = None


def _hip_runtime() -> ctypes.CDLL:
    """The HIP runtime torch has loaded (resolved by its soname, so no second
    copy is loaded)."""
    global _HIP
    if _HIP is None:
        hip = ctypes.CDLL("libamdhip64.so.7")
        hip.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
        hip.hipHostMalloc.restype = ctypes.c_int
        hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                       ctypes.c_void_p]
        hip.hipMemcpyAsync.restype = ctypes.c_int
        hip.hipHostGetDevicePointer.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_uint]
        hip.hipHostGetDevicePointer.restype = ctypes.c_int
        _HIP = hip
    return _HIP


def staging() -> HostStaging:
    """The process's pinned upload ring (created on first use)."""
    global _STAGING
    if _STAGING is None:
        with _lock:
            if _STAGING is None:
                _STAGING = HostStaging()
    return _STAGING


def upload_i64(values: Sequence[int], device: torch.device) -> torch.Tensor:
    """int64 values on ``device``: through the pinned ring on a HIP device,
    a plain tensor elsewhere."""
    if device.type != "cuda":
        return torch.tensor(values, dtype=torch.int64, device=device)
    return staging().upload_i64(values, device)

