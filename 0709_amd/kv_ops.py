"""All-layer KV movement on the HIP kernels: append, slot-to-slot move and
page-table commit compaction.

Three physical layouts are addressed through one slot formula (see
include/atlas0709.h):

* FlashInfer NHD paged layers ``[pages, 2, page_size, Hkv, D]`` (the
  reference's per-layer caches, ``flashinfer_full_verify.py:833-841``);
* FlashInfer HND paged layers ``[pages, 2, Hkv, page_size, D]`` (a token's row
  split by KV head, ``page_size * D`` elements apart: each head's keys of a
  page are one contiguous run);
* SGLang-style flat token pools ``[slots, Hkv, D]`` with separate K and V
  tensors per layer (the Drafter pool, addressed with ``page_size = 1``).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import torch

from . import _lib


@dataclass(frozen=True)
class SlotGeometry:
    """Byte geometry of one layer's K (or V) region.  ``head_stride`` is the
    distance between a token's KV heads, 0 when its row is contiguous."""

    page_size: int
    page_stride: int
    token_stride: int
    row_bytes: int
    head_bytes: int = 0
    head_stride: int = 0

    def as_args(self) -> tuple[int, int, int, int]:
        """(page_size, page_stride, token_stride, row_bytes): contiguous rows."""
        if self.head_stride and self.head_stride != self.head_bytes:
            raise ValueError("this call takes contiguous token rows only")
        return self.page_size, self.page_stride, self.token_stride, self.row_bytes

    def as_head_args(self) -> tuple[int, int, int, int, int, int]:
        """as_args() followed by (head_bytes, head_stride)."""
        return (self.page_size, self.page_stride, self.token_stride, self.row_bytes, self.head_bytes,
                self.head_stride)


KV_LAYOUTS = ("NHD", "HND")


def check_kv_layout(kv_layout: str) -> str:
    if kv_layout not in KV_LAYOUTS:
        raise ValueError(f"kv_layout must be one of {KV_LAYOUTS}, got {kv_layout!r}")
    return kv_layout


def paged_layer_geometry(layer_kv: torch.Tensor, kv_layout: str = "NHD") -> tuple[SlotGeometry, int]:
    """Geometry of a FlashInfer paged layer, NHD ``[pages, 2, page_size, Hkv,
    D]`` or HND ``[pages, 2, Hkv, page_size, D]``.

    Returns the slot geometry and the byte offset of the V half.
    """
    check_kv_layout(kv_layout)
    if layer_kv.ndim != 5 or int(layer_kv.shape[1]) != 2:
        raise ValueError(f"expected a paged layer [pages, 2, ...] of {kv_layout} pages, got {tuple(layer_kv.shape)}")
    es = layer_kv.element_size()
    s = layer_kv.stride()
    if kv_layout == "NHD":
        _, _, page_size, heads, dim = (int(x) for x in layer_kv.shape)
        if not rows_contiguous(layer_kv):
            raise ValueError("paged layer rows (Hkv, D) must be contiguous")
        geom = SlotGeometry(page_size, s[0] * es, s[2] * es, heads * dim * es, dim * es, s[3] * es)
    else:
        _, _, heads, page_size, dim = (int(x) for x in layer_kv.shape)
        if s[4] != 1 and dim != 1:
            raise ValueError("paged layer head rows (D) must be contiguous")
        geom = SlotGeometry(page_size, s[0] * es, s[3] * es, heads * dim * es, dim * es, s[2] * es)
    return geom, s[1] * es


def token_pool_geometry(buf: torch.Tensor) -> SlotGeometry:
    """Geometry of a flat token pool ``[slots, Hkv, D]`` (slot = row index)."""
    if buf.ndim != 3:
        raise ValueError(f"expected a token pool [slots, Hkv, D], got {tuple(buf.shape)}")
    _, heads, dim = (int(x) for x in buf.shape)
    es = buf.element_size()
    s = buf.stride()
    if not rows_contiguous(buf):
        raise ValueError("token pool rows (Hkv, D) must be contiguous")
    return SlotGeometry(1, s[0] * es, s[0] * es, heads * dim * es)


def rows_contiguous(t: torch.Tensor) -> bool:
    """The last two dims (Hkv, D) form one dense row (size-1 dims may carry
    any stride)."""
    if t.stride(-1) != 1 and int(t.shape[-1]) != 1:
        return False
    return int(t.shape[-2]) == 1 or t.stride(-2) == int(t.shape[-1])


def _layer_ptrs(layers: Sequence[torch.Tensor], v_offset: int | None = None):
    k = [int(t.data_ptr()) for t in layers]
    v = [p + v_offset for p in k] if v_offset is not None else None
    return k, v


def _layer_tables(k_layers: Sequence[torch.Tensor], v_layers: Sequence[torch.Tensor]):
    """(K pointer table, V pointer table, slot geometry) of a flat token pool."""
    if len(k_layers) != len(v_layers) or not k_layers:
        raise ValueError("k_layers and v_layers must be non-empty and of equal length")
    return (_lib.ptr_array([int(t.data_ptr()) for t in k_layers]),
            _lib.ptr_array([int(t.data_ptr()) for t in v_layers]),
            token_pool_geometry(k_layers[0]))


def _as_long(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    if t.device != device or t.dtype != torch.int64 or not t.is_contiguous():
        t = t.to(device=device, dtype=torch.int64).contiguous()
    return t


def move_slots(
    k_layers: Sequence[torch.Tensor],
    v_layers: Sequence[torch.Tensor],
    dst_slots: torch.Tensor,
    src_slots: torch.Tensor,
    *,
    layer_tables: tuple | None = None,
) -> None:
    """``K[dst] = K[src]; V[dst] = V[src]`` for every layer of a flat token pool.

    The SGLang ``move_kv_cache(tgt_loc, src_loc)`` contract used by the
    reference's tail-page copy-on-write
    (``flashinfer_paged/sglang_runtime.py:686-695``); ``dst`` and ``src`` must
    be disjoint. ``layer_tables`` = ``(k_ptrs, v_ptrs, geometry)`` built once
    by a pool whose layer buffers never move (skips rebuilding them per call).
    """
    if len(k_layers) != len(v_layers) or not k_layers:
        raise ValueError("k_layers and v_layers must be non-empty and of equal length")
    device = _lib.require_device(k_layers[0], dst_slots, src_slots, what="move_kv_cache")
    n = int(dst_slots.numel())
    if int(src_slots.numel()) != n:
        raise ValueError("move_kv_cache needs as many source as destination slots")
    if n == 0:
        return
    dst = _as_long(dst_slots.reshape(-1), device)
    src = _as_long(src_slots.reshape(-1), device)
    if layer_tables is None:
        layer_tables = _layer_tables(k_layers, v_layers)
    k_tab, v_tab, geom = layer_tables
    lib = _lib.load()
    rc = lib.atlas_kv_move_slots(
        k_tab, v_tab, len(k_layers), *geom.as_args(),
        _lib.ptr(dst), _lib.ptr(src), n, _lib.stream_of(device),
    )
    _lib.check(rc, "atlas_kv_move_slots")


def append_token_pool(
    k_layers: Sequence[torch.Tensor],
    v_layers: Sequence[torch.Tensor],
    k_src: Sequence[torch.Tensor],
    v_src: Sequence[torch.Tensor],
    dst_slots: torch.Tensor,
    *,
    layer_tables: tuple | None = None,
) -> None:
    """Scatter dense rows ``[n, Hkv, D]`` into slots of every layer of a flat pool
    (SGLang ``set_kv_buffer``, ``sglang_page_attention.py:187-194``).
    ``layer_tables`` as for :func:`move_slots`."""
    device = _lib.require_device(k_layers[0], dst_slots, k_src[0], what="set_kv_buffer")
    n = int(dst_slots.numel())
    if n == 0:
        return
    if len(k_src) != len(k_layers) or len(v_src) != len(v_layers):
        raise ValueError("one K and one V source per layer are required")
    if layer_tables is None:
        layer_tables = _layer_tables(k_layers, v_layers)
    k_tab, v_tab, geom = layer_tables
    src_stride = k_src[0].stride(0) * k_src[0].element_size()
    # each distinct source tensor is checked once (callers often pass one
    # tensor for several layers)
    for t in {id(t): t for t in (*k_src, *v_src)}.values():
        if t.dtype != k_layers[0].dtype:
            raise TypeError(f"source dtype {t.dtype} does not match the pool dtype {k_layers[0].dtype}")
        if int(t.shape[0]) < n or not rows_contiguous(t):
            raise ValueError("source rows must be [n, Hkv, D] with contiguous (Hkv, D)")
        if t.stride(0) * t.element_size() != src_stride:
            raise ValueError("every K/V source must share one row stride")
    dst = _as_long(dst_slots.reshape(-1), device)
    lib = _lib.load()
    rc = lib.atlas_kv_append(
        k_tab, v_tab, len(k_layers), *geom.as_head_args(),
        _lib.ptr_array([int(t.data_ptr()) for t in k_src]),
        _lib.ptr_array([int(t.data_ptr()) for t in v_src]),
        src_stride, _lib.ptr(dst), 0, n, _lib.stream_of(device),
    )
    _lib.check(rc, "atlas_kv_append")


def append_paged(
    layers: Sequence[torch.Tensor],
    k_src: Sequence[torch.Tensor],
    v_src: Sequence[torch.Tensor],
    *,
    start_pos: int | None = None,
    dst_slots: torch.Tensor | None = None,
    kv_layout: str = "NHD",
) -> None:
    """Write dense rows ``[n, Hkv, D]`` into paged layers (``kv_layout``
    pages) at contiguous positions ``start_pos + i`` (identity page table) or
    at physical slots."""
    if not layers or len(k_src) != len(layers) or len(v_src) != len(layers):
        raise ValueError("one K and one V source per layer are required")
    device = _lib.require_device(layers[0], k_src[0], v_src[0], dst_slots, what="write_suffix_kv")
    geom, v_off = paged_layer_geometry(layers[0], kv_layout)
    n = int(k_src[0].shape[0])
    for t in (*k_src, *v_src):
        if t.dtype != layers[0].dtype:
            raise TypeError(f"source dtype {t.dtype} does not match the KV dtype {layers[0].dtype}")
        if int(t.shape[0]) != n or t.ndim != 3 or not rows_contiguous(t):
            raise ValueError("K/V states must be [n, Hkv, D] with contiguous (Hkv, D)")
        if int(t.shape[1]) * int(t.shape[2]) * t.element_size() != geom.row_bytes:
            raise ValueError("K/V state rows do not match the cache's (Hkv, D)")
    if n == 0:
        return
    src_stride = k_src[0].stride(0) * k_src[0].element_size()
    if any(t.stride(0) * t.element_size() != src_stride for t in (*k_src, *v_src)):
        raise ValueError("all K/V sources must share one token stride")
    k_ptrs, v_ptrs = _layer_ptrs(layers, v_off)
    dst = None if dst_slots is None else _as_long(dst_slots.reshape(-1), device)
    if dst is None and (start_pos is None or start_pos < 0):
        raise ValueError("start_pos must be a non-negative position")
    lib = _lib.load()
    rc = lib.atlas_kv_append(
        _lib.ptr_array(k_ptrs), _lib.ptr_array(v_ptrs), len(layers), *geom.as_head_args(),
        _lib.ptr_array([int(t.data_ptr()) for t in k_src]),
        _lib.ptr_array([int(t.data_ptr()) for t in v_src]),
        src_stride, _lib.ptr(dst), 0 if start_pos is None else int(start_pos), n, _lib.stream_of(device),
    )
    _lib.check(rc, "atlas_kv_append")


def commit_positions_need_staging(
    src_pos: Sequence[int], dst_pos: Sequence[int], item_req: Sequence[int] | None = None
) -> bool:
    """True when some destination equals another item's source in the same
    request, i.e. a one-pass in-place copy could read an overwritten row."""
    reqs = list(item_req) if item_req is not None else [0] * len(src_pos)
    sources: dict[tuple[int, int], int] = {}
    for i, (r, s) in enumerate(zip(reqs, src_pos)):
        sources.setdefault((int(r), int(s)), i)
    for i, (r, d) in enumerate(zip(reqs, dst_pos)):
        j = sources.get((int(r), int(d)))
        if j is not None and j != i:
            return True
    return False


_LAYER_TABLES: dict = {}


def _paged_layer_tables(layers: Sequence[torch.Tensor], kv_layout: str = "NHD"):
    """(slot geometry, K pointer table, V pointer table) of a list of paged
    layers, kept for the most recent few layer sets: a Target commits into
    the same layer tensors every verify.  The key holds every layer's address
    and the first layer's shape, strides and dtype, so a changed list never
    reuses a stale table."""
    l0 = layers[0]
    key = (tuple(map(torch.Tensor.data_ptr, layers)), tuple(l0.shape), l0.stride(), l0.dtype, kv_layout)
    hit = _LAYER_TABLES.get(key)
    if hit is None:
        for t in layers[1:]:
            if t.shape != l0.shape or t.stride() != l0.stride() or t.dtype != l0.dtype:
                raise ValueError("every layer must have the first layer's shape, strides and dtype")
        geom, v_off = paged_layer_geometry(l0, kv_layout)
        k_ptrs, v_ptrs = _layer_ptrs(layers, v_off)
        hit = (geom, _lib.ptr_array(k_ptrs), _lib.ptr_array(v_ptrs))
        if len(_LAYER_TABLES) >= 8:
            _LAYER_TABLES.pop(next(iter(_LAYER_TABLES)))
        _LAYER_TABLES[key] = hit
    return hit


def _as_i32(t: torch.Tensor | None, device: torch.device) -> torch.Tensor | None:
    if t is None:
        return None
    if t.device != device or t.dtype != torch.int32 or not t.is_contiguous():
        t = t.to(device=device, dtype=torch.int32).contiguous()
    return t


def commit_paged(
    layers: Sequence[torch.Tensor],
    src_pos: Sequence[int] | torch.Tensor,
    dst_pos: Sequence[int] | torch.Tensor,
    *,
    kv_indptr: torch.Tensor | None = None,
    kv_indices: torch.Tensor | None = None,
    item_req: Sequence[int] | torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    needs_staging: bool | None = None,
    kv_layout: str = "NHD",
) -> None:
    """Route-commit compaction over paged layers (``kv_layout`` pages), every
    layer in one launch.

    Row at logical position ``src_pos[i]`` of request ``item_req[i]`` is copied
    to ``dst_pos[i]`` (positions are mapped through ``kv_indices`` starting at
    ``kv_indptr[req]``; identity when ``kv_indices`` is None).  The result
    equals the reference's gather-clone-scatter
    (``target_runtime.py:910-912``).  Host position lists travel in the kernel
    argument block (no host-to-device copy) when they fit.
    """
    if not layers:
        raise ValueError("no layers given")
    device = _lib.require_device(layers[0], kv_indptr, kv_indices, what="target_kv_commit")
    geom, k_tab, v_tab = _paged_layer_tables(layers, kv_layout)
    lib = _lib.load()
    stream = _lib.stream_of(device)
    i32_indptr = _as_i32(kv_indptr, device)
    i32_indices = _as_i32(kv_indices, device)
    host_lists = not isinstance(src_pos, torch.Tensor) and not isinstance(dst_pos, torch.Tensor) and (
        item_req is None or not isinstance(item_req, torch.Tensor)
    )
    if host_lists:
        src = [int(x) for x in src_pos]
        dst = [int(x) for x in dst_pos]
        if len(src) != len(dst):
            raise ValueError("source and destination position counts differ")
        n = len(src)
        if n == 0:
            return
        reqs = [0] * n if item_req is None else [int(x) for x in item_req]
        staging = commit_positions_need_staging(src, dst, reqs) if needs_staging is None else needs_staging
        if n <= _lib.MAX_INLINE_ITEMS and not staging:
            rc = lib.atlas_kv_commit_paged_host(
                k_tab, v_tab, len(layers), *geom.as_head_args(),
                _lib.ptr(i32_indptr), _lib.ptr(i32_indices),
                (ctypes_i32 * n)(*reqs), (ctypes_i64 * n)(*src), (ctypes_i64 * n)(*dst), n, stream,
            )
            _lib.check(rc, "atlas_kv_commit_paged_host")
            return
        src_t = torch.tensor(src, dtype=torch.int64).to(device, non_blocking=True)
        dst_t = torch.tensor(dst, dtype=torch.int64).to(device, non_blocking=True)
        req_t = torch.tensor(reqs, dtype=torch.int32).to(device, non_blocking=True)
    else:
        src_t = _as_long(torch.as_tensor(src_pos).reshape(-1), device)
        dst_t = _as_long(torch.as_tensor(dst_pos).reshape(-1), device)
        n = int(src_t.numel())
        if int(dst_t.numel()) != n:
            raise ValueError("source and destination position counts differ")
        if n == 0:
            return
        req_t = None if item_req is None else torch.as_tensor(item_req).to(device=device, dtype=torch.int32).contiguous()
        staging = True if needs_staging is None else bool(needs_staging)
    ws_bytes = 0
    if staging:
        need = n * 2 * len(layers) * geom.row_bytes
        if workspace is None or workspace.numel() * workspace.element_size() < need:
            workspace = torch.empty(need, dtype=torch.uint8, device=device)
        ws_bytes = workspace.numel() * workspace.element_size()
    rc = lib.atlas_kv_commit_paged(
        k_tab, v_tab, len(layers), *geom.as_head_args(),
        _lib.ptr(i32_indptr), _lib.ptr(i32_indices), _lib.ptr(req_t), _lib.ptr(src_t), _lib.ptr(dst_t), n,
        1 if staging else 0, _lib.ptr(workspace if staging else None), ws_bytes, stream,
    )
    _lib.check(rc, "atlas_kv_commit_paged")


import ctypes as _ctypes  # noqa: E402  (kept at the end to keep the public API at the top)

ctypes_i32 = _ctypes.c_int32
ctypes_i64 = _ctypes.c_int64
