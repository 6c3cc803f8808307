"""Drafter route pool: logical routes bound to request rows and physical KV
slots (drop-in for ``SGLangRoutePoolBridge``, reference
``flashinfer_paged/sglang_runtime.py:89-1117``).

Same fields, methods, counters, exceptions and copy-on-write rules as the
reference.  Differences (all leave the KV bytes, slot paths, request rows and
freed-page order identical):

* tail-page copy-on-write issues ONE ``move_kv_cache`` for all copied pages of
  a frontier (destinations are freshly allocated, disjoint pages), where the
  reference calls it once per copied page (``:783-797``);
* with the native allocator (``native_pool.NativePagedAllocator``) page
  ownership is a bitmap in HBM: newly handed-out pages are marked by a kernel
  at once (no deferred device-to-host flush), and ``release_unreferenced_
  node_slots`` is a mark/sweep kernel that returns the releasable pages in
  ascending order straight to the device free list.  With any other
  allocator the reference's host-set bookkeeping is kept.
"""

from __future__ import annotations

import ctypes
import operator
import sys
import threading
import time
from dataclasses import dataclass, field
from typing import Any, Sequence

import numpy as np
import torch

from .. import _lib
from .paged_metadata import build_flashinfer_paged_kv_metadata
from .kv import KVTreeStore
from .types import DraftPrefixState, FrontierDecodeOutput, PrefixKVView, RouteState


@dataclass(frozen=True)
class AtlasPagedDecodeSpec:
    """Page metadata carried to paged decode (``sglang_page_attention.py:10-17``)."""

    kv_indptr: torch.Tensor
    kv_indices: torch.Tensor
    kv_last_page_len: torch.Tensor
    page_size: int


@dataclass(frozen=True)
class SGLangRouteKVMetadata:
    """Per-frontier decode metadata (``flashinfer_backends.py:12-32``)."""

    req_pool_indices: torch.Tensor
    seq_lens: torch.Tensor
    out_cache_loc: torch.Tensor
    positions: torch.Tensor
    seq_lens_sum: int
    seq_lens_cpu: torch.Tensor
    orig_seq_lens: torch.Tensor | None = None
    attention_page_size: int = 1
    token_index_count: int = 0
    page_index_count: int = 0
    paged_decode_spec: AtlasPagedDecodeSpec | None = None


@dataclass
class SGLangRouteRow:
    route_id: int
    req_pool_index: int
    handle: Any
    written_length: int = 0
    pending_dirty_start: int | None = None


@dataclass
class _PoolReqHandle:
    rid: str
    req_pool_idx: int | None = None


class DeviceOwnedPages:
    """Set of owned page ids held as a bitmap in HBM (bit p of word p // 32).

    Supports the set operations the bridge and its callers use; reading it as
    a Python set copies the bitmap to the host (diagnostics only)."""

    def __init__(self, num_pages: int, page_size: int, device: torch.device) -> None:
        self.num_pages = int(num_pages)
        self.page_size = int(page_size)
        self.device = device
        words = (self.num_pages + 31) // 32
        self.bitmap = torch.zeros(words, dtype=torch.int32, device=device)
        self.live = torch.zeros(words, dtype=torch.int32, device=device)
        self.free_pages = torch.zeros(self.num_pages, dtype=torch.int64, device=device)
        self.free_count = torch.zeros(1, dtype=torch.int64, device=device)

    # -- device operations ---------------------------------------------
    def mark_slots(self, slots: torch.Tensor) -> None:
        s = slots.reshape(-1).to(device=self.device, dtype=torch.int64).contiguous()
        if int(s.numel()) == 0:
            return
        lib = _lib.load()
        rc = lib.atlas_mark_pages(_lib.ptr(self.bitmap), self.num_pages, _lib.ptr(s), int(s.numel()), self.page_size,
                                  _lib.stream_of(self.device))
        _lib.check(rc, "atlas_mark_pages")

    def sweep(self, live_slots: torch.Tensor) -> torch.Tensor:
        """owned -= pages not reachable from live_slots; returns the released
        pages (ascending, on the device)."""
        self.sweep_launch(live_slots)
        n = int(self.free_count.item())
        return self.free_pages[:n]

    def sweep_launch(self, live_slots: torch.Tensor) -> None:
        """The sweep without reading its count back: the released pages land
        in ``free_pages[:free_count]`` on the device."""
        s = live_slots.reshape(-1).to(device=self.device, dtype=torch.int64).contiguous()
        lib = _lib.load()
        rc = lib.atlas_prune_pages(_lib.ptr(self.bitmap), _lib.ptr(self.live), self.num_pages, _lib.ptr(s),
                                   int(s.numel()), self.page_size, _lib.ptr(self.free_pages),
                                   _lib.ptr(self.free_count), _lib.stream_of(self.device))
        _lib.check(rc, "atlas_prune_pages")

    def sweep_paths_launch(self, paths: Sequence[torch.Tensor], with_last: Sequence[bool], gather=None) -> bool:
        """``sweep_launch`` whose live slots are sampled from slot paths in
        the launch (path p: its page-start slots, plus its last slot when
        ``with_last[p]``), with no sample list built first.  ``gather``:
        (segments, count, out) the same launch then copies to ``out`` (see
        ``atlas_gather_i64``).  Returns False, launching nothing, when the
        paths are not contiguous int64 device tensors or exceed the launch's
        limits (then use ``sweep_launch``)."""
        n = len(paths)
        if n > _lib.PRUNE_MAX_PATHS or self.num_pages > _lib.PRUNE_PATHS_MAX_PAGES:
            return False
        arr = (_lib.SlotPath * max(n, 1))()
        mask = 0
        for i, (t, last) in enumerate(zip(paths, with_last)):
            if t.dtype != torch.int64 or not t.is_contiguous() or t.device != self.device:
                return False
            arr[i].slots = t.data_ptr()
            arr[i].len = t.numel()
            if last:
                mask |= 1 << i
        lib = _lib.load()
        if gather is None:
            rc = lib.atlas_prune_pages_paths(_lib.ptr(self.bitmap), _lib.ptr(self.live), self.num_pages, arr, n,
                                             mask, self.page_size, _lib.ptr(self.free_pages),
                                             _lib.ptr(self.free_count), _lib.stream_of(self.device))
        else:
            rc = lib.atlas_prune_pages_paths_gather(_lib.ptr(self.bitmap), _lib.ptr(self.live), self.num_pages, arr,
                                                    n, mask, self.page_size, _lib.ptr(self.free_pages),
                                                    _lib.ptr(self.free_count), *gather, _lib.stream_of(self.device))
        _lib.check(rc, "atlas_prune_pages_paths")
        return True

    # -- set protocol -----------------------------------------------------
    def to_set(self) -> set[int]:
        words = self.bitmap.cpu().numpy().view(np.uint32)
        out = set()
        for i in np.flatnonzero(words):
            w = int(words[i])
            while w:
                b = (w & -w).bit_length() - 1
                out.add(int(i) * 32 + b)
                w &= w - 1
        return out

    def _set_pages(self, pages, value: bool) -> None:
        pages = sorted({int(p) for p in pages})
        if not pages:
            return
        if pages[0] < 0 or pages[-1] >= self.num_pages:
            raise ValueError("page id outside the pool")
        words = self.bitmap.cpu().numpy().view(np.uint32).copy()
        for p in pages:
            bit = np.uint32(1 << (p % 32))
            if value:
                words[p // 32] |= bit
            else:
                words[p // 32] &= ~bit
        self.bitmap.copy_(torch.from_numpy(words.view(np.int32)))

    def update(self, pages) -> None:
        self._set_pages(pages, True)

    def add(self, page: int) -> None:
        self._set_pages([page], True)

    def difference_update(self, pages) -> None:
        self._set_pages(pages, False)

    def remove(self, page: int) -> None:
        if int(page) not in self:
            raise KeyError(page)
        self._set_pages([page], False)

    def clear(self) -> None:
        self.bitmap.zero_()

    def __contains__(self, page) -> bool:
        p = int(page)
        if not 0 <= p < self.num_pages:
            return False
        return bool((int(self.bitmap[p // 32].item()) >> (p % 32)) & 1)

    def __iter__(self):
        return iter(sorted(self.to_set()))

    def __len__(self) -> int:
        return len(self.to_set())

    def __eq__(self, other) -> bool:
        return self.to_set() == set(other)

    def __sub__(self, other):
        return self.to_set() - set(other)

    def __rsub__(self, other):
        return set(other) - self.to_set()

    def __repr__(self) -> str:
        return f"DeviceOwnedPages({sorted(self.to_set())})"


@dataclass
class SGLangRoutePoolBridge:
    """Bind logical routes to request rows and physical KV slots."""

    req_to_token_pool: Any
    token_to_kv_pool_allocator: Any
    page_size: int
    max_context_len: int | None = None
    device: str | torch.device = "cuda"
    prefix_slot_ids: torch.Tensor | None = None
    prefix_slot_count: int = 0
    prefix_page_ids: set[int] = field(default_factory=set)
    route_rows: dict[int, SGLangRouteRow] = field(default_factory=dict)
    node_slot_ids: dict[int, int | torch.Tensor] = field(default_factory=dict)
    route_slot_paths: dict[int, torch.Tensor] = field(default_factory=dict)
    route_tail_page_keys: dict[int, int] = field(default_factory=dict)
    prefix_tail_page_key: int | None = None
    prefix_partial_tail_keys: dict[int, int] = field(default_factory=dict)
    next_tail_page_key: int = 1
    owned_page_ids: Any = field(default_factory=set)
    pending_owned_slot_tensors: list[torch.Tensor] = field(default_factory=list)
    cow_pages_copied: int = 0
    cow_tokens_copied: int = 0
    attention_metadata_builds: int = 0
    attention_metadata_token_indices: int = 0
    attention_metadata_page_indices: int = 0
    req_row_write_calls: int = 0
    req_row_elements_written: int = 0
    req_row_full_rewrite_calls: int = 0
    req_row_full_rewrite_elements: int = 0
    req_row_full_init_calls: int = 0
    req_row_full_init_elements: int = 0
    req_row_append_calls: int = 0
    req_row_append_elements: int = 0
    req_row_cow_patch_calls: int = 0
    req_row_cow_patch_elements: int = 0
    hot_path_host_transfer_batches: int = 0
    hot_path_host_transfer_elements: int = 0
    use_page_attention_metadata: bool = True
    validate_page_layout: bool = True
    pending_device_checks: list[Any] = field(default_factory=list)

    def __post_init__(self) -> None:
        alloc = self.token_to_kv_pool_allocator
        num_pages = getattr(alloc, "num_pages", None)
        alloc_device = getattr(alloc, "device", None)
        if (
            isinstance(self.owned_page_ids, set)
            and not self.owned_page_ids
            and num_pages is not None
            and isinstance(alloc_device, torch.device)
            and alloc_device.type == "cuda"
            and callable(getattr(alloc, "free_pages_prepend", None))
        ):
            # Native pool: ownership in HBM (pages 0..num_pages, page 0 = padding).
            self.owned_page_ids = DeviceOwnedPages(int(num_pages) + 1, self.page_size, alloc_device)

    @property
    def _device_ownership(self) -> bool:
        return isinstance(self.owned_page_ids, DeviceOwnedPages)

    @classmethod
    def from_runner(cls, model_runner: Any, *, page_size: int, device: str | torch.device = "cuda"):
        """``sglang_runtime.py:130-171``."""
        req_pool = getattr(model_runner, "req_to_token_pool", None)
        allocator = None
        for name in ("token_to_kv_pool_allocator", "token_to_kv_pool_alloc", "kv_pool_allocator"):
            allocator = getattr(model_runner, name, None)
            if allocator is not None:
                break
        if req_pool is None:
            raise RuntimeError("SGLang ModelRunner does not expose req_to_token_pool")
        if allocator is None:
            raise RuntimeError("SGLang ModelRunner does not expose token_to_kv_pool_allocator")
        actual = getattr(model_runner, "atlas_pool_page_size", None)
        if actual is None:
            for name in ("token_to_kv_pool", "kv_pool", "kvcache"):
                pool = getattr(model_runner, name, None)
                if pool is not None:
                    actual = getattr(pool, "page_size", None)
                    break
        if actual is not None and int(actual) != int(page_size):
            raise RuntimeError(
                "ATLAS page-size argument does not match the physical SGLang KV pool: "
                f"requested={int(page_size)}, physical={int(actual)}"
            )
        max_ctx = getattr(model_runner, "atlas_max_context_len", None)
        if max_ctx is None:
            max_ctx = _req_pool_capacity(req_pool)
        return cls(
            req_to_token_pool=req_pool,
            token_to_kv_pool_allocator=allocator,
            page_size=page_size,
            max_context_len=int(max_ctx) if max_ctx is not None else None,
            device=device,
            use_page_attention_metadata=bool(getattr(model_runner, "atlas_use_page_attention_metadata", True)),
            validate_page_layout=bool(getattr(model_runner, "atlas_validate_page_layout", True)),
        )

    # ------------------------------------------------------------ prefix
    def set_prefix_slots(self, slot_ids: Sequence[int] | torch.Tensor, *, page_ids=None) -> None:
        """``sglang_runtime.py:173-187``.  ``page_ids``: the pages of the slot
        path when the caller already holds them on the host (saves reading
        the path back)."""
        self.prefix_slot_ids = _as_long(slot_ids, self.device)
        if page_ids is not None and int(self.prefix_slot_ids.numel()):
            self.prefix_slot_count = int(self.prefix_slot_ids.numel())
            self.prefix_page_ids = set(int(p) for p in page_ids)
        else:
            self._refresh_prefix_cpu_metadata()
        if self._device_ownership:
            self.owned_page_ids.clear()
            if self.prefix_slot_count:
                self.owned_page_ids.mark_slots(self.prefix_slot_ids[:: self.page_size])
        else:
            self.owned_page_ids = set(self.prefix_page_ids)
        self.pending_owned_slot_tensors.clear()
        self.prefix_partial_tail_keys.clear()
        partial = self.prefix_slot_count and self.prefix_slot_count % self.page_size
        self.prefix_tail_page_key = self._new_tail_page_key() if partial else None
        if self.prefix_tail_page_key is not None:
            self.prefix_partial_tail_keys[(self.prefix_slot_count - 1) // self.page_size] = self.prefix_tail_page_key

    def _refresh_prefix_cpu_metadata(self) -> None:
        if self.prefix_slot_ids is None or int(self.prefix_slot_ids.numel()) == 0:
            self.prefix_slot_count = 0
            self.prefix_page_ids.clear()
            return
        self.prefix_slot_count = int(self.prefix_slot_ids.numel())
        starts = torch.div(self.prefix_slot_ids[:: self.page_size], self.page_size, rounding_mode="floor")
        self.prefix_page_ids = set(_int_list(starts))

    def _new_tail_page_key(self) -> int:
        # Lease keys are negative, so they never equal a physical page id.
        key = -int(self.next_tail_page_key)
        self.next_tail_page_key += 1
        return key

    # ------------------------------------------------------------ ownership
    def _record_pending_owned_slots(self, slot_ids: torch.Tensor) -> None:
        if int(slot_ids.numel()) == 0:
            return
        if self._device_ownership:
            self.owned_page_ids.mark_slots(slot_ids.detach())
        else:
            self.pending_owned_slot_tensors.append(slot_ids.detach().reshape(-1))

    def _materialize_pending_owned_pages(self) -> None:
        """Host-set mode: fold the pending slots into ``owned_page_ids`` with
        one batched copy (``sglang_runtime.py:216-233``).  Device mode marks
        pages as they are handed out, so there is nothing pending."""
        if not self.pending_owned_slot_tensors:
            return
        slots = torch.cat(self.pending_owned_slot_tensors, dim=0)
        self.owned_page_ids.update(s // self.page_size for s in _int_list(slots))
        self.pending_owned_slot_tensors.clear()

    def owned_page_count(self) -> int:
        self._materialize_pending_owned_pages()
        return len(self.owned_page_ids)

    # ------------------------------------------------------------ rows
    def bind_existing_route_row(self, route_id: int, req_pool_index: int, handle: Any | None = None, *,
                                written_length: int = 0) -> None:
        if int(written_length) < 0:
            raise ValueError("written_length must be non-negative")
        if handle is None:
            handle = _PoolReqHandle(rid=f"atlas-{int(route_id)}", req_pool_idx=int(req_pool_index))
        self.route_rows[int(route_id)] = SGLangRouteRow(int(route_id), int(req_pool_index), handle,
                                                        written_length=int(written_length))

    def ensure_route_rows(self, routes: Sequence[RouteState]) -> torch.Tensor:
        return torch.tensor(self._route_row_indices(routes), dtype=torch.long, device=self.device)

    def _route_row_indices(self, routes: Sequence[RouteState]) -> list[int]:
        """Request rows of the routes (allocating rows for new routes)."""
        missing = [r for r in routes if int(r.route_id) not in self.route_rows]
        if missing:
            handles = [_PoolReqHandle(rid=f"atlas-{int(r.route_id)}") for r in missing]
            indices = self.req_to_token_pool.alloc(handles)
            if indices is None:
                raise RuntimeError("SGLang ReqToTokenPool.alloc returned None")
            rows = _int_list(indices)
            if len(rows) != len(missing):
                raise RuntimeError("SGLang ReqToTokenPool.alloc returned the wrong number of rows")
            for route, handle, row in zip(missing, handles, rows):
                handle.req_pool_idx = int(row)
                self.bind_existing_route_row(route.route_id, int(row), handle=handle)
        return [self.route_rows[int(r.route_id)].req_pool_index for r in routes]

    def release_route_rows(self, route_ids: Sequence[int]) -> None:
        for route_id in route_ids:
            row = self.route_rows.pop(int(route_id), None)
            if row is not None and hasattr(self.req_to_token_pool, "free"):
                self.req_to_token_pool.free(row.handle)

    def retain_route_rows(self, route_ids: Sequence[int]) -> int:
        """Keep only the given routes' rows, slot paths and leases
        (``sglang_runtime.py:284-302``); returns the number of released rows."""
        keep = {int(r) for r in route_ids}
        released = [int(r) for r in self.route_rows if int(r) not in keep]
        self.release_route_rows(released)
        self.route_slot_paths = {r: p for r, p in self.route_slot_paths.items() if r in keep}
        self.route_tail_page_keys = {r: k for r, k in self.route_tail_page_keys.items() if r in keep}
        return len(released)

    def register_node_slots(self, node_ids, slot_ids) -> None:
        nodes = _int_list(node_ids)
        if isinstance(slot_ids, torch.Tensor):
            values: list[Any] = list(slot_ids.reshape(-1).unbind(0))
        else:
            values = [int(s) for s in slot_ids]
        if len(nodes) != len(values):
            raise ValueError("node_ids and slot_ids must have the same length")
        for n, s in zip(nodes, values):
            self.node_slot_ids[int(n)] = s

    def reconcile_route_rows(self, previous_routes: Sequence[RouteState], next_routes: Sequence[RouteState]) -> None:
        """Children inherit the parent's slot path and lease; the first child
        takes over the parent's row, other rows are freed
        (``sglang_runtime.py:318-355``)."""
        children: dict[int, list[RouteState]] = {}
        for child in next_routes:
            if child.parent_route_id is not None:
                children.setdefault(int(child.parent_route_id), []).append(child)
        for parent in previous_routes:
            pid = int(parent.route_id)
            row = self.route_rows.pop(pid, None)
            kids = children.get(pid, [])
            path = self.route_slot_paths.get(pid)
            if path is not None:
                for child in kids:
                    self.route_slot_paths[int(child.route_id)] = path
                    key = self.route_tail_page_keys.get(pid)
                    if key is not None:
                        self.route_tail_page_keys[int(child.route_id)] = key
            if row is None:
                continue
            if kids:
                first = kids[0]
                self.route_rows[int(first.route_id)] = SGLangRouteRow(
                    route_id=int(first.route_id), req_pool_index=row.req_pool_index, handle=row.handle,
                    written_length=row.written_length, pending_dirty_start=row.pending_dirty_start,
                )
            elif hasattr(self.req_to_token_pool, "free"):
                self.req_to_token_pool.free(row.handle)

    # ------------------------------------------------------------ promote / prune
    def commit_route_as_prefix(self, route: RouteState, *, defer_page_ids: bool = False) -> torch.Tensor:
        """Zero-copy promotion: the route's slot path becomes the prefix and
        its tail lease carries over (``sglang_runtime.py:357-378``).  With
        ``defer_page_ids`` the prefix's host page-id set is left for the
        caller to refresh (the multi-request commit reads it back together
        with the prune's counts)."""
        old_len = 0 if self.prefix_slot_ids is None else int(self.prefix_slot_ids.numel())
        path = self._slot_path_for_route(route)
        expected = old_len + len(route.kv_view.node_ids)
        if int(path.numel()) != expected:
            raise RuntimeError(
                f"cannot promote route KV to prefix: slot_path_len={int(path.numel())}, expected={expected}"
            )
        self.prefix_slot_ids = path
        if not defer_page_ids:
            self._refresh_prefix_cpu_metadata()
        self.prefix_partial_tail_keys.clear()
        n = int(path.numel())
        self.prefix_tail_page_key = self.route_tail_page_keys.get(int(route.route_id)) if n % self.page_size else None
        if self.prefix_tail_page_key is not None:
            self.prefix_partial_tail_keys[(n - 1) // self.page_size] = self.prefix_tail_page_key
        return path

    def page_reference_counts(self) -> dict[int, int]:
        """One reference per path view reaching a page (prefix + each route),
        ``sglang_runtime.py:380-396``."""
        counts: dict[int, int] = {}
        for pages in self._page_id_sets_for_paths([self.prefix_slot_ids, *self.route_slot_paths.values()]):
            for p in pages:
                counts[p] = counts.get(p, 0) + 1
        return dict(sorted(counts.items()))

    def _page_id_sets_for_paths(self, paths: Sequence[torch.Tensor | None]) -> list[set[int]]:
        """Pages of each path from its page-start slots plus its last slot,
        fetched in one batch (``sglang_runtime.py:479-505``)."""
        counts: list[int] = []
        parts: list[torch.Tensor] = []
        for path in paths:
            if path is None or int(path.numel()) == 0:
                counts.append(0)
                continue
            sampled = torch.cat((path[:: self.page_size], path[-1:]))
            parts.append(torch.div(sampled, self.page_size, rounding_mode="floor").to(torch.long))
            counts.append(int(parts[-1].numel()))
        flat = _int_list(torch.cat(parts)) if parts else []
        out, off = [], 0
        for c in counts:
            out.append(set(flat[off : off + c]))
            off += c
        return out

    def validate_route_physical_state(self, route: RouteState) -> None:
        """``sglang_runtime.py:398-477``."""
        rid = int(route.route_id)
        path = self.route_slot_paths.get(rid)
        if path is None:
            raise RuntimeError(f"Drafter route {rid} has no physical slot path")
        committed = int(route.kv_view.prefix.committed_length)
        expected = committed + len(route.kv_view.node_ids)
        slots = _int_list(path)
        if len(slots) != expected:
            raise RuntimeError(
                f"Drafter route {rid} physical length does not match logical KV: physical={len(slots)}, "
                f"committed={committed}, nodes={len(route.kv_view.node_ids)}"
            )
        missing = [int(n) for n in route.kv_view.node_ids if int(n) not in self.node_slot_ids]
        if missing:
            raise RuntimeError(f"Drafter route {rid} has logical nodes without materialized KV: node_ids={missing}")
        ps = int(self.page_size)
        for pos, slot in enumerate(slots):
            off = pos % ps
            if slot % ps != off:
                raise RuntimeError(
                    f"Drafter route {rid} physical page layout is invalid: logical_position={pos}, slot_id={slot}, "
                    f"expected_page_offset={off}"
                )
            if off and slot != slots[pos - 1] + 1:
                raise RuntimeError(
                    f"Drafter route {rid} physical page is not contiguous: logical_position={pos}, "
                    f"previous_slot={slots[pos - 1]}, slot_id={slot}"
                )
        self._materialize_pending_owned_pages()
        owned = self.owned_page_ids.to_set() if self._device_ownership else self.owned_page_ids
        unowned = sorted({s // ps for s in slots} - owned)
        if unowned:
            raise RuntimeError(f"Drafter route {rid} references unowned KV pages: page_ids={unowned}")
        row = self.route_rows.get(rid)
        if row is None:
            return
        if int(row.written_length) != len(slots):
            raise RuntimeError(
                f"Drafter route {rid} req-row length is inconsistent: row={int(row.written_length)}, slots={len(slots)}"
            )
        table = getattr(self.req_to_token_pool, "req_to_token", None)
        if isinstance(table, torch.Tensor) and _int_list(table[int(row.req_pool_index), : len(slots)]) != slots:
            raise RuntimeError(f"Drafter route {rid} req-row slots do not match its physical path")

    def release_unreferenced_node_slots(self, live_node_ids: Sequence[int]) -> int:
        """Return every owned page that neither the committed prefix nor a
        retained route reaches, in ascending page order; forget dead node
        mappings (``sglang_runtime.py:507-539``).  Returns the page count.
        The deferred device checks run first (over native pools: with the
        sweep's count read-back, before any page returns to the free list)."""
        if self._device_ownership:
            return _sweep_bridges([self], [live_node_ids], refresh_prefix=False)[0]
        self.check_pending_device_checks()
        self._materialize_pending_owned_pages()
        live_pages = set(self.prefix_page_ids)
        for pages in self._page_id_sets_for_paths(list(self.route_slot_paths.values())):
            live_pages.update(pages)
        releasable = sorted(self.owned_page_ids - live_pages)
        self._forget_dead_nodes(live_node_ids)
        if releasable:
            self._require_allocator_free()
            self.token_to_kv_pool_allocator.free(
                torch.tensor([p * self.page_size for p in releasable], dtype=torch.long, device=self.device))
            self.owned_page_ids.difference_update(releasable)
        return len(releasable)

    def _live_paths(self) -> tuple[list[torch.Tensor], list[bool]]:
        """The slot paths ``_live_slot_samples`` samples, and whether each
        contributes its last slot: the prefix (page starts only), then each
        retained route's path."""
        paths, last = [], []
        if self.prefix_slot_ids is not None and int(self.prefix_slot_ids.numel()):
            paths.append(self.prefix_slot_ids)
            last.append(False)
        for path in self.route_slot_paths.values():
            if int(path.numel()):
                paths.append(path)
                last.append(True)
        return paths, last

    def _live_slot_samples(self) -> torch.Tensor:
        """One slot of every page the prefix and the retained routes reach:
        each path's page-start slots plus its last slot."""
        parts = []
        if self.prefix_slot_ids is not None and int(self.prefix_slot_ids.numel()):
            parts.append(self.prefix_slot_ids[:: self.page_size])
        for path in self.route_slot_paths.values():
            if int(path.numel()):
                parts.append(path[:: self.page_size])
                parts.append(path[-1:])
        return torch.cat(parts) if parts else torch.zeros(0, dtype=torch.long, device=self.device)

    def _forget_dead_nodes(self, live_node_ids: Sequence[int]) -> None:
        live_nodes = {int(n) for n in live_node_ids}
        for node in [n for n in self.node_slot_ids if n not in live_nodes]:
            del self.node_slot_ids[node]

    def _require_allocator_free(self) -> None:
        if not callable(getattr(self.token_to_kv_pool_allocator, "free", None)):
            raise RuntimeError("SGLang token-to-KV allocator does not expose free()")

    def clear_physical_state(self) -> None:
        """``sglang_runtime.py:541-576``."""
        self.prefix_slot_ids = None
        self.prefix_slot_count = 0
        self.prefix_page_ids.clear()
        self.prefix_tail_page_key = None
        self.prefix_partial_tail_keys.clear()
        self.route_rows.clear()
        self.node_slot_ids.clear()
        self.route_slot_paths.clear()
        self.route_tail_page_keys.clear()
        self.next_tail_page_key = 1
        self.owned_page_ids.clear()
        self.pending_owned_slot_tensors.clear()
        self.pending_device_checks.clear()
        for name in _COUNTERS:
            setattr(self, name, 0)
        for target in (self.req_to_token_pool, self.token_to_kv_pool_allocator):
            clear = getattr(target, "clear", None)
            if callable(clear):
                clear()

    # ------------------------------------------------------------ allocation
    def allocate_token_slots(self, count: int, *, mode: str = "decode") -> torch.Tensor:
        if count <= 0:
            raise ValueError("count must be positive")
        result = _allocate_kv_slots(self.token_to_kv_pool_allocator, int(count), mode=mode)
        slots = _slot_tensor(result, self.device)
        if int(slots.numel()) < int(count):
            raise RuntimeError(
                "SGLang token slot allocator returned too few slots: "
                f"needed={int(count)}, got_shape={tuple(slots.shape)}, mode={mode}, result_type={type(result).__name__}"
            )
        return slots[: int(count)]

    def allocate_extend_slots(self, *, prefix_lens: Sequence[int], seq_lens: Sequence[int],
                              last_locs: Sequence[int] | torch.Tensor) -> torch.Tensor:
        pre_cpu = torch.tensor(list(prefix_lens), dtype=torch.long)
        seq_cpu = torch.tensor(list(seq_lens), dtype=torch.long)
        pre = pre_cpu.to(self.device)
        seq = seq_cpu.to(self.device)
        last = _as_long(last_locs, self.device)
        if not (pre.numel() == seq.numel() == last.numel()):
            raise ValueError("prefix_lens, seq_lens, and last_locs must have the same length")
        n = sum(int(s) - int(p) for p, s in zip(prefix_lens, seq_lens))
        if n <= 0:
            raise ValueError("extend_num_tokens must be positive")
        fn = getattr(self.token_to_kv_pool_allocator, "alloc_extend", None)
        if callable(fn):
            result = fn(pre, pre_cpu, seq, seq_cpu, last, n)
            if result is not None:
                slots = _slot_tensor(result, self.device)
                if int(slots.numel()) >= n:
                    return slots[:n]
        return self.allocate_token_slots(n, mode="extend")

    def allocate_decode_slots(self, *, seq_lens: Sequence[int], last_locs: Sequence[int] | torch.Tensor) -> torch.Tensor:
        seq_cpu = torch.tensor(list(seq_lens), dtype=torch.long)
        seq = seq_cpu.to(self.device)
        last = _as_long(last_locs, self.device)
        if seq.numel() != last.numel():
            raise ValueError("seq_lens and last_locs must have the same length")
        fn = getattr(self.token_to_kv_pool_allocator, "alloc_decode", None)
        if callable(fn):
            result = fn(seq, seq_cpu, last)
            if result is not None:
                slots = _slot_tensor(result, self.device)
                if int(slots.numel()) >= int(seq.numel()):
                    return slots[: int(seq.numel())]
        return self.allocate_token_slots(int(seq.numel()), mode="decode")

    def _allocate_full_pages(self, count: int) -> torch.Tensor:
        """``count`` whole pages as a [count, page_size] slot tensor
        (``sglang_runtime.py:661-684``)."""
        if count <= 0:
            return torch.empty((0, self.page_size), dtype=torch.long, device=self.device)
        alloc = getattr(self.token_to_kv_pool_allocator, "alloc", None)
        if not callable(alloc):
            raise RuntimeError("SGLang token-to-KV allocator does not expose alloc()")
        result = alloc(int(count) * self.page_size)
        if result is None:
            raise RuntimeError(f"SGLang KV pool cannot allocate {int(count)} COW pages")
        slots = _slot_tensor(result, self.device)
        expected = int(count) * self.page_size
        if int(slots.numel()) != expected:
            raise RuntimeError(
                f"SGLang full-page allocation returned the wrong number of slots: expected={expected}, "
                f"got={int(slots.numel())}"
            )
        pages = slots.reshape(int(count), self.page_size)
        if not self._device_ownership:
            # Foreign allocators: confirm each returned page is contiguous.
            ids = torch.div(pages, self.page_size, rounding_mode="floor")
            self._check_or_defer(ids.eq(ids[:, :1]).all(), "SGLang allocator returned a non-contiguous COW page")
        self._record_pending_owned_slots(pages[:, 0])
        return pages

    def _copy_kv_slots(self, destination: torch.Tensor, source: torch.Tensor) -> None:
        get_kvcache = getattr(self.token_to_kv_pool_allocator, "get_kvcache", None)
        kv_cache = get_kvcache() if callable(get_kvcache) else None
        move = getattr(kv_cache, "move_kv_cache", None)
        if not callable(move):
            raise RuntimeError(
                "SGLang KV pool does not expose move_kv_cache(); tail-page copy-on-write cannot be performed"
            )
        destination = destination.to(dtype=torch.long)
        source = source.to(dtype=torch.long)
        # The all-layer move copies every slot independently, so a page that
        # is both written and read would race; copy-on-write destinations are
        # freshly allocated pages, which no source path can hold.
        dst_pages = torch.div(destination, self.page_size, rounding_mode="floor")
        src_pages = torch.div(source, self.page_size, rounding_mode="floor")
        self._check_or_defer(dst_pages[:, None].ne(src_pages[None, :]).all(),
                             "copy-on-write destination pages overlap its source pages")
        move(destination, source)

    # ------------------------------------------------------------ copy-on-write
    def _copy_partial_tail_pages(self, routes: Sequence[RouteState], slot_paths: Sequence[torch.Tensor]):
        return self._copy_partial_tail_pages_with_dirty_starts(routes, slot_paths)[0]

    def _copy_partial_tail_pages_with_dirty_starts(self, routes: Sequence[RouteState],
                                                   slot_paths: Sequence[torch.Tensor]):
        """Tail-page copy-on-write (``sglang_runtime.py:708-798``).

        Active writers whose slot paths end inside the same partial page
        (same lease key) form a group; the first keeps the page, every other
        gets a fresh page holding a copy of its valid tail, a new lease, and a
        dirty start at the copied tail.  All copies go in one move call.
        Returns the new paths and {route position: dirty start}.
        """
        result = list(slot_paths)
        plan = self._tail_copy_plan(routes, slot_paths)
        if not plan:
            return result, {}
        dest_pages = self._allocate_full_pages(len(plan))
        dirty: dict[int, int] = {}
        dst_parts, src_parts = [], []
        for page, (index, path, tail) in zip(dest_pages, plan):
            src = path[-tail:]
            dst = page[:tail]
            dst_parts.append(dst)
            src_parts.append(src)
            new_path = torch.cat((path[:-tail], dst))
            rid = int(routes[index].route_id)
            self.route_slot_paths[rid] = new_path
            self.route_tail_page_keys[rid] = self._new_tail_page_key()
            result[index] = new_path
            dirty[index] = int(path.numel()) - tail
            self.cow_pages_copied += 1
            self.cow_tokens_copied += tail
        self._copy_kv_slots(torch.cat(dst_parts), torch.cat(src_parts))
        return result, dirty

    def _tail_copy_plan(self, routes: Sequence[RouteState], slot_paths: Sequence[torch.Tensor]):
        """Routes whose partial tail page must be copied, as (position, path,
        tail length) in copy order: every writer of a shared tail page (same
        lease key) but the first."""
        if len(routes) != len(slot_paths):
            raise ValueError("routes and slot_paths must have the same length")
        if len(routes) <= 1:
            return []
        groups: dict[int, list[tuple[int, torch.Tensor, int]]] = {}
        unkeyed: list[tuple[int, torch.Tensor, int, int, torch.Tensor]] = []
        for index, path in enumerate(slot_paths):
            tail = int(path.numel()) % self.page_size
            if not tail:
                continue
            rid = int(routes[index].route_id)
            key = self.route_tail_page_keys.get(rid)
            if key is None:
                # Paths injected without a lease: key them by their physical
                # tail page (one batched device-to-host read).
                src = path[-tail:]
                pages = torch.div(src, self.page_size, rounding_mode="floor")
                self._check_or_defer(pages.eq(pages[:1]).all(), "route partial tail spans multiple physical pages")
                unkeyed.append((index, path, tail, rid, pages[:1]))
                continue
            groups.setdefault(key, []).append((index, path, tail))
        if unkeyed:
            keys = _int_list(torch.cat([e[4] for e in unkeyed]))
            self.hot_path_host_transfer_batches += 1
            self.hot_path_host_transfer_elements += len(keys)
            for (index, path, tail, rid, _), key in zip(unkeyed, keys):
                self.route_tail_page_keys[rid] = int(key)
                groups.setdefault(int(key), []).append((index, path, tail))
        return [entry for group in groups.values() for entry in group[1:]]

    # ------------------------------------------------------------ frontier
    def prepare_frontier(self, active_routes: Sequence[RouteState], *,
                         output_slot_ids: torch.Tensor | None = None):
        """Rows, copy-on-write, decode slots, incremental request-row writes
        and page metadata for one decode step (``sglang_runtime.py:800-959``)."""
        if not active_routes:
            raise ValueError("active_routes cannot be empty")
        req_rows = self._route_row_indices(active_routes)
        paths = [self._slot_path_for_route(r) for r in active_routes]
        paths, dirty = self._copy_partial_tail_pages_with_dirty_starts(active_routes, paths)
        for index, start in dirty.items():
            row = self.route_rows[int(active_routes[index].route_id)]
            if int(row.written_length) > 0:
                row.pending_dirty_start = int(start) if row.pending_dirty_start is None else min(
                    int(row.pending_dirty_start), int(start))
        seq_lens = [int(p.numel()) + 1 for p in paths]
        last_locs = torch.cat([
            p[-1:].to(torch.long) if int(p.numel()) else torch.full((1,), -1, dtype=torch.long, device=self.device)
            for p in paths
        ])
        if output_slot_ids is None:
            output_slot_ids = self.allocate_decode_slots(seq_lens=seq_lens, last_locs=last_locs)
        else:
            output_slot_ids = _as_long(output_slot_ids, self.device)
        if int(output_slot_ids.numel()) != len(active_routes):
            raise ValueError("output_slot_ids must have one slot per active route")
        if len(active_routes) > 1:
            dup = output_slot_ids[:, None].eq(output_slot_ids[None, :])
            dup.fill_diagonal_(False)
            self._check_or_defer(dup.logical_not().all(),
                                 "SGLang allocated duplicate output KV slots across forked routes; "
                                 "tail-page copy-on-write is not active")
        self._record_pending_owned_slots(output_slot_ids)

        # Every route's new path (its path, then its new slot) in one buffer;
        # the routes keep views of it.
        pieces: list[torch.Tensor] = []
        for i, path in enumerate(paths):
            pieces.append(path)
            pieces.append(output_slot_ids[i : i + 1])
        flat = torch.cat(pieces)
        positions: list[int] = []
        full_paths: list[torch.Tensor] = []
        segments: list[tuple[int, int, torch.Tensor, str]] = []
        off = 0
        for route, path in zip(active_routes, paths):
            rid = int(route.route_id)
            row = self.route_rows[rid]
            prev = int(path.numel())
            full = flat[off : off + prev + 1]
            off += prev + 1
            if int(row.written_length) == 0:
                start, kind = 0, "full_init"
            else:
                if int(row.written_length) != prev:
                    raise RuntimeError(
                        "SGLang route-row state does not match its physical KV path: "
                        f"route_id={rid}, written_length={int(row.written_length)}, physical_path_length={prev}"
                    )
                if row.pending_dirty_start is None:
                    start, kind = prev, "append"
                else:
                    start, kind = int(row.pending_dirty_start), "cow_patch"
            segments.append((int(row.req_pool_index), start, full[start:], kind))
            positions.append(prev)
            full_paths.append(full)

        def commit_route(i: int) -> None:
            # a route's state moves on only once its row write went through
            rid = int(active_routes[i].route_id)
            row = self.route_rows[rid]
            prev = positions[i]
            row.written_length = prev + 1
            row.pending_dirty_start = None
            self.route_slot_paths[rid] = full_paths[i]
            if prev % self.page_size == 0 or rid not in self.route_tail_page_keys:
                self.route_tail_page_keys[rid] = self._new_tail_page_key()

        # input ids, sequence lengths, positions, request rows (and, for a
        # pool that takes them, the request-row write indices) reach the
        # device in one copy
        b = len(active_routes)
        host = [int(r.pending_token_id) for r in active_routes] + seq_lens + positions + req_rows
        batched = bool(getattr(self.req_to_token_pool, "batched_row_writes", False))
        write_rows: list[int] = []
        write_pos: list[int] = []
        if batched:
            for req_row, start, values, _ in segments:
                n = int(values.numel())
                write_rows.extend([req_row] * n)
                write_pos.extend(range(start, start + n))
        on_device = torch.device(self.device).type != "cpu"
        packed = torch.tensor(host + write_rows + write_pos, dtype=torch.long, pin_memory=on_device)
        if on_device:
            packed = packed.to(self.device, non_blocking=True)
        input_ids, seq_dev, pos_dev = packed[:b], packed[b : 2 * b], packed[2 * b : 3 * b]
        req_indices = packed[3 * b : 4 * b]
        if batched:
            nw = len(write_rows)
            self._write_req_token_slices(segments, packed[4 * b : 4 * b + nw], packed[4 * b + nw :])
            for i in range(b):
                commit_route(i)
        else:
            # per-route slice writes, as a foreign pool (and the reference's
            # tests of its write log) expect them
            for i, (req_row, start, values, kind) in enumerate(segments):
                self._write_req_token_slice(req_row, start, values, write_kind=kind)
                commit_route(i)

        seq_cpu = torch.tensor(seq_lens, dtype=torch.long)
        tokens = int(sum(seq_lens))
        spec = None
        attn_ps = 1
        page_indices = tokens
        if self.use_page_attention_metadata:
            md = build_flashinfer_paged_kv_metadata(full_paths, page_size=self.page_size,
                                                    validate_layout=self.validate_page_layout)
            if md.layout_flag is not None:
                self.pending_device_checks.append(md.assert_layout_valid)
            spec = AtlasPagedDecodeSpec(md.kv_indptr, md.kv_page_indices, md.kv_last_page_len, int(md.page_size))
            attn_ps = int(md.page_size)
            page_indices = int(md.page_index_count)
        self.attention_metadata_builds += 1
        self.attention_metadata_token_indices += tokens
        self.attention_metadata_page_indices += page_indices
        meta = SGLangRouteKVMetadata(
            req_pool_indices=req_indices, seq_lens=seq_dev, out_cache_loc=output_slot_ids,
            positions=pos_dev, orig_seq_lens=seq_dev,
            seq_lens_sum=tokens, seq_lens_cpu=seq_cpu, attention_page_size=attn_ps, token_index_count=tokens,
            page_index_count=page_indices, paged_decode_spec=spec,
        )
        return input_ids, meta

    def _plan_fused_frontier(self, active_routes: Sequence[RouteState]) -> "_FusedFrontierPlan":
        """Host half of ``prepare_frontier`` for ``prepare_frontiers``: request
        rows, slot paths, the copy-on-write plan and the request-row segments,
        in the order ``prepare_frontier`` takes them; no device work.

        Planning changes nothing that a failed step would leave behind: the
        copy-on-write routes' new leases, the copy counters and the dirty
        starts are applied by ``_finish_fused_frontier`` once the step's pages
        are known to exist and its launch went through.  (Path inheritance
        and the keying of lease-less tails happen here, as in
        ``prepare_frontier`` before its own allocation can fail.)"""
        if not active_routes:
            raise ValueError("active_routes cannot be empty")
        rows = self._route_row_indices(active_routes)
        paths = [self._slot_path_for_route(r) for r in active_routes]
        n = len(paths)
        prevs = [int(p.numel()) for p in paths]
        cow_tail = [0] * n
        cow_rank = [-1] * n
        cow_order: list[int] = []
        dirty: dict[int, int] = {}
        for rank, (index, _path, tail) in enumerate(self._tail_copy_plan(active_routes, paths)):
            cow_tail[index] = tail
            cow_rank[index] = rank
            cow_order.append(index)
            dirty[index] = prevs[index] - tail
        starts: list[int] = []
        kinds: list[str] = []
        cap = _req_pool_capacity(self.req_to_token_pool)
        if cap is None:
            cap = self.max_context_len
        route_rows = self.route_rows
        for i, (route, prev, req_row) in enumerate(zip(active_routes, prevs, rows)):
            row = route_rows[int(route.route_id)]
            written = int(row.written_length)
            if written == 0:
                start, kind = 0, "full_init"
            else:
                if written != prev:
                    raise RuntimeError(
                        "SGLang route-row state does not match its physical KV path: "
                        f"route_id={int(route.route_id)}, written_length={written}, "
                        f"physical_path_length={prev}"
                    )
                pending = row.pending_dirty_start
                if i in dirty:
                    pending = dirty[i] if pending is None else min(int(pending), dirty[i])
                if pending is None:
                    start, kind = prev, "append"
                else:
                    start, kind = int(pending), "cow_patch"
            if start < 0 or start > prev or (cap is not None and prev + 1 > int(cap)):
                self._check_req_write(req_row, start, prev + 1 - start, kind)  # raises with the reason
            starts.append(start)
            kinds.append(kind)
        for i, p in enumerate(paths):
            if prevs[i] and (p.dtype != torch.int64 or not p.is_contiguous()):
                paths[i] = p.to(torch.int64).contiguous()
        return _FusedFrontierPlan(list(active_routes), rows, paths, prevs, cow_tail, cow_rank,
                                  len(cow_order), starts, kinds, cow_order)

    def _finish_fused_frontier(self, plan: "_FusedFrontierPlan", full_paths: Sequence[torch.Tensor],
                               flags: "_StepFlags", group: int) -> None:
        """Bookkeeping of ``prepare_frontier`` once the step's launch went
        through: the copy-on-write routes' leases and counters (in copy
        order, as ``prepare_frontier`` assigns them), request-row state, new
        slot paths, leases of routes that opened a page, counters and the
        step's device checks."""
        ps = self.page_size
        for index in plan.cow_order:
            self.route_tail_page_keys[int(plan.routes[index].route_id)] = self._new_tail_page_key()
            self.cow_pages_copied += 1
            self.cow_tokens_copied += plan.cow_tail[index]
        for i, route in enumerate(plan.routes):
            rid = int(route.route_id)
            row = self.route_rows[rid]
            prev = plan.prevs[i]
            self._count_req_write(prev + 1 - plan.starts[i], plan.kinds[i])
            row.written_length = prev + 1
            row.pending_dirty_start = None
            self.route_slot_paths[rid] = full_paths[i]
            if prev % ps == 0 or rid not in self.route_tail_page_keys:
                self.route_tail_page_keys[rid] = self._new_tail_page_key()
        self.attention_metadata_builds += 1
        self.attention_metadata_token_indices += sum(plan.prevs) + len(plan.prevs)
        self.attention_metadata_page_indices += sum((p + ps) // ps for p in plan.prevs)
        self.pending_device_checks.append(_StepCheck(flags, group, bool(self.validate_page_layout)))

    def _check_or_defer(self, ok: torch.Tensor, message: str) -> None:
        """A device-computed condition is checked at the next report boundary
        (prune), so the decode step does not wait on it; a host condition is
        checked now."""
        if ok.device.type == "cpu":
            _assert_true(ok, message)
        else:
            self.pending_device_checks.append(lambda: _assert_true(ok, message))

    def check_pending_device_checks(self) -> None:
        """Raise the first failed deferred condition (layout of frontier page
        metadata, distinct output slots) recorded since the last check.  The
        flags of fused frontier steps are already on their way to the host."""
        _prefetch_step_flags([self])
        pending, self.pending_device_checks = self.pending_device_checks, []
        for check in pending:
            check()

    def _slot_path_for_route(self, route: RouteState) -> torch.Tensor:
        """Existing path, else the parent's (inheriting its lease), else a
        committed-prefix slice keyed by the prefix's partial-tail lease
        (``sglang_runtime.py:961-1021``)."""
        rid = int(route.route_id)
        expected = int(route.kv_view.prefix.committed_length) + len(route.kv_view.node_ids)
        existing = self.route_slot_paths.get(rid)
        if existing is not None:
            if int(existing.numel()) != expected:
                raise RuntimeError(
                    "route-specific physical path length does not match logical KV: "
                    f"route_id={rid}, physical={int(existing.numel())}, logical={expected}"
                )
            return existing
        if route.parent_route_id is not None:
            pid = int(route.parent_route_id)
            parent = self.route_slot_paths.get(pid)
            if parent is not None:
                if int(parent.numel()) != expected:
                    raise RuntimeError(
                        "inherited physical path length does not match logical KV: "
                        f"route_id={rid}, physical={int(parent.numel())}, logical={expected}"
                    )
                self.route_slot_paths[rid] = parent
                key = self.route_tail_page_keys.get(pid)
                if key is not None:
                    self.route_tail_page_keys[rid] = key
                return parent
        committed = int(route.kv_view.prefix.committed_length)
        if committed:
            if self.prefix_slot_ids is None:
                raise RuntimeError("prefix_slot_ids must be set before decoding non-empty prefixes")
            if int(self.prefix_slot_ids.numel()) < committed:
                raise RuntimeError(
                    f"prefix_slot_ids has length {int(self.prefix_slot_ids.numel())}, "
                    f"but route requires committed_length={committed}"
                )
            prefix = self.prefix_slot_ids[:committed]
        else:
            prefix = torch.empty((0,), dtype=torch.long, device=self.device)
        if route.kv_view.node_ids:
            raise RuntimeError(
                "route has materialized logical KV nodes but no route-specific physical slot path: "
                f"route_id={rid}"
            )
        self.route_slot_paths[rid] = prefix
        if committed % self.page_size:
            tail_index = (committed - 1) // self.page_size
            key = self.prefix_partial_tail_keys.get(tail_index)
            if key is None:
                key = self._new_tail_page_key()
                self.prefix_partial_tail_keys[tail_index] = key
            if committed == self.prefix_slot_count:
                self.prefix_tail_page_key = key
            self.route_tail_page_keys[rid] = key
        return prefix

    # ------------------------------------------------------------ request rows
    def _write_req_token_row(self, req_pool_index: int, slot_path: torch.Tensor) -> None:
        self._write_req_token_slice(req_pool_index, 0, slot_path, write_kind="full_init")

    def _write_req_token_slices(self, segments, rows: torch.Tensor, positions: torch.Tensor) -> None:
        """The request-row writes of one frontier, (row, start, slot ids,
        kind) each, as one tensor-index write (rows / positions already on the
        device) into a pool that declares ``batched_row_writes``; checks and
        counters per segment as for ``_write_req_token_slice``."""
        for req_row, start, values, kind in segments:
            self._check_req_write(req_row, start, int(values.numel()), kind)
        values = torch.cat([v for _, _, v, _ in segments]) if len(segments) > 1 else segments[0][2]
        try:
            self.req_to_token_pool.write((rows, positions), values)
        except Exception as exc:
            raise RuntimeError("failed to write SGLang req_to_token_pool route row") from exc
        for _, _, values, kind in segments:
            self._count_req_write(int(values.numel()), kind)

    def _check_req_write(self, req_pool_index: int, start: int, n: int, write_kind: str) -> None:
        if write_kind not in {"full_init", "append", "cow_patch"}:
            raise ValueError(f"unknown req-row write kind: {write_kind}")
        if start < 0:
            raise ValueError("req-row write start must be non-negative")
        if n <= 0:
            raise ValueError("req-row write cannot be empty")
        end = start + n
        cap = _req_pool_capacity(self.req_to_token_pool)
        if cap is None:
            cap = self.max_context_len
        if cap is not None and end > int(cap):
            raise RuntimeError(
                "SGLang req_to_token_pool row is too short for the requested prefix. "
                f"write_end={end}, req_pool_context_capacity={int(cap)}, req_pool_index={int(req_pool_index)}. "
                "Increase --context-length or recreate the runner with a larger ReqToTokenPool."
            )

    def _count_req_write(self, n: int, write_kind: str) -> None:
        self.req_row_write_calls += 1
        self.req_row_elements_written += n
        if write_kind == "full_init":
            self.req_row_full_init_calls += 1
            self.req_row_full_init_elements += n
            self.req_row_full_rewrite_calls += 1
            self.req_row_full_rewrite_elements += n
        elif write_kind == "append":
            self.req_row_append_calls += 1
            self.req_row_append_elements += n
        else:
            self.req_row_cow_patch_calls += 1
            self.req_row_cow_patch_elements += n

    def _write_req_token_slice(self, req_pool_index: int, start: int, slot_ids: torch.Tensor, *,
                               write_kind: str) -> None:
        """Write ``slot_ids`` into a request row at ``start`` (slice API, then
        the tensor-index form); counters count successful writes only
        (``sglang_runtime.py:1031-1092``)."""
        if write_kind not in {"full_init", "append", "cow_patch"}:
            raise ValueError(f"unknown req-row write kind: {write_kind}")
        start = int(start)
        values = _as_long(slot_ids, self.device)
        n = int(values.numel())
        self._check_req_write(req_pool_index, start, n, write_kind)
        end = start + n
        try:
            self.req_to_token_pool.write((int(req_pool_index), slice(start, end)), values)
        except Exception:
            pos = torch.arange(start, end, dtype=torch.long, device=values.device)
            rows = torch.full_like(pos, int(req_pool_index))
            try:
                self.req_to_token_pool.write((rows, pos), values)
            except Exception as exc:
                raise RuntimeError("failed to write SGLang req_to_token_pool route row") from exc
        self._count_req_write(n, write_kind)

    def hot_path_counters(self) -> dict[str, int]:
        return dict(zip(_COUNTERS, map(int, _get_counters(self))))


@dataclass
class _FusedFrontierPlan:
    routes: list[RouteState]
    rows: list[int]
    paths: list[torch.Tensor]
    prevs: list[int]
    cow_tail: list[int]
    cow_rank: list[int]
    num_cow: int
    starts: list[int]
    kinds: list[str]
    cow_order: list[int]  # route positions of the copies, in copy order


class _StepCheck:
    """A deferred check of one request's group in a fused frontier step."""

    def __init__(self, step_flags: "_StepFlags", group: int, validate_layout: bool) -> None:
        self.step_flags = step_flags
        self.group = int(group)
        self.validate_layout = validate_layout

    def __call__(self) -> None:
        self.step_flags.check(self.group, self.validate_layout)


def _unread_step_flags(bridges: Sequence["SGLangRoutePoolBridge"]) -> list["_StepFlags"]:
    """Flags of the fused frontier steps with a check pending on these
    bridges that are still on the device (each step once)."""
    out: list[_StepFlags] = []
    seen: set[int] = set()
    for b in bridges:
        for c in b.pending_device_checks:
            f = getattr(c, "step_flags", None)
            if f is not None and f._host is None and id(f) not in seen:
                seen.add(id(f))
                out.append(f)
    return out


class _HostGather:
    """Mapped pinned host memory for ``atlas_gather_i64``: a read-back of up
    to ``capacity`` int64 values is one launch and one event wait (no
    concatenation on the device, no separate copy).  One per process,
    serialised by its lock."""

    capacity = 8192

    def __init__(self) -> None:
        self.lock = threading.Lock()
        self.buf: _lib.MappedReadback | None = None
        self.values: np.ndarray | None = None
        self.events: dict[int, torch.cuda.Event] = {}

    def segments(self, tensors: Sequence[torch.Tensor]):
        """(segments, count, total) of 1-D int64 device tensors, or None when
        this path does not take them (host tensors, other dtypes, more
        segments or values than it holds)."""
        dev = tensors[0].device
        if dev.type != "cuda" or len(tensors) > _lib.GATHER_MAX_SEGMENTS:
            return None
        segs = (_lib.I64Segment * len(tensors))()
        total = 0
        for i, t in enumerate(tensors):
            if t.device != dev or t.dtype != torch.int64 or t.dim() != 1:
                return None
            n = int(t.numel())
            seg = segs[i]
            seg.src, seg.count, seg.stride = t.data_ptr(), n, int(t.stride(0))
            total += n
        if total > self.capacity:
            return None
        return segs, len(tensors), total

    def run(self, launch, total: int, dev: torch.device) -> list[int]:
        """``launch(out)`` queues work that writes ``total`` values to the
        device address ``out``; the values once it has run."""
        with self.lock:
            if self.buf is None:
                self.buf = _lib.MappedReadback(2 * self.capacity)
                self.values = self.buf.np.view(np.int64)
            launch(self.buf.device_ptr)
            idx = dev.index if dev.index is not None else torch.cuda.current_device()
            ev = self.events.get(idx)
            if ev is None:
                ev = self.events[idx] = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(dev))
            ev.synchronize()
            return self.values[:total].tolist()

    def read(self, tensors: Sequence[torch.Tensor]) -> list[int] | None:
        """The values of the tensors, concatenated, through one gather
        launch, or None (see ``segments``)."""
        plan = self.segments(tensors)
        if plan is None:
            return None
        segs, n, total = plan
        dev = tensors[0].device

        def launch(out):
            _lib.check(_lib.load().atlas_gather_i64(segs, n, out, _lib.stream_of(dev)), "atlas_gather_i64")

        return self.run(launch, total, dev)


_HOST_GATHER = _HostGather()


def _read_back(parts: Sequence[torch.Tensor], bridges: Sequence["SGLangRoutePoolBridge"]) -> list[int]:
    """ONE read-back to the host of the int64 tensors ``parts`` together with
    the check words of every fused frontier step with a check pending on
    ``bridges`` (one gather launch into mapped host memory, else one copy);
    returns the values of ``parts``, concatenated."""
    flags = _unread_step_flags(bridges)
    tensors = [*parts, *(f.flags for f in flags)]
    if not tensors:
        return []
    flat = _HOST_GATHER.read(tensors)
    if flat is None:
        flat = _int_list(torch.cat(tensors) if len(tensors) > 1 else tensors[0])
    return _read_back_split(parts, flags, flat)


def _read_back_split(parts: Sequence[torch.Tensor], flags: Sequence["_StepFlags"], flat: list[int]) -> list[int]:
    """Hands the step flags their values from a read-back of ``parts`` and
    their words (in that order); returns the values of ``parts``."""
    off = sum(int(t.numel()) for t in parts)
    head = flat[:off]
    for f in flags:
        n = int(f.flags.numel())
        f._host = flat[off : off + n]
        off += n
    return head


def _prefetch_step_flags(bridges: Sequence["SGLangRoutePoolBridge"]) -> None:
    """Brings the flags of every fused frontier step with a check pending on
    these bridges to the host, in one copy."""
    _read_back([], bridges)


class _StepFlags:
    """Check words of one fused frontier step: one device int64 per route,
    the launch's ``FRONTIER_*`` bits (0 when every check passed), and each
    request's route range ``spans[group]``.  They stay on the device until a
    check needs them: the prune reads the words of every pending step back
    in the copy that brings its released-page counts, so a decode step
    queues no copy of its own."""

    def __init__(self, flags: torch.Tensor, spans: Sequence[tuple[int, int]]) -> None:
        self.flags = flags
        self.spans = spans
        self._host: list[int] | None = None
        self._groups: list[int] | None = None  # each request's words ORed, once

    def host(self) -> list[int]:
        if self._host is None:
            self._host = _int_list(self.flags)
        return self._host

    def check(self, group: int, validate_layout: bool) -> None:
        groups = self._groups
        if groups is None:
            h = self.host()
            groups = []
            for lo, hi in self.spans:
                bits = 0
                for w in h[lo:hi]:
                    bits |= w
                groups.append(bits)
            self._groups = groups
        if any(b & _lib.FRONTIER_BAD_DESCRIPTOR for b in groups):
            raise RuntimeError("frontier step: a route descriptor was out of range and the route was skipped")
        bits = groups[int(group)]
        # the order prepare_frontier records these checks in
        if bits & _lib.FRONTIER_COW_OVERLAP:
            raise RuntimeError("copy-on-write destination pages overlap its source pages")
        if bits & _lib.FRONTIER_DUPLICATE_SLOT:
            raise RuntimeError("SGLang allocated duplicate output KV slots across forked routes; "
                               "tail-page copy-on-write is not active")
        if validate_layout and bits & _lib.FRONTIER_BAD_LAYOUT:
            from .paged_metadata import LAYOUT_MESSAGE
            raise RuntimeError(LAYOUT_MESSAGE)


@dataclass(frozen=True)
class FusedFrontierStep:
    """One frontier step of several requests: the union batch the model runs
    (inputs and decode metadata of every route, request by request) and each
    request's route range ``spans[i] = (first, end)`` in it."""

    input_ids: torch.Tensor
    metadata: SGLangRouteKVMetadata
    route_ids: torch.Tensor
    spans: tuple[tuple[int, int], ...]
    prevs: tuple[int, ...] = ()  # every route's path length before the step


_ROUTE_FIELDS = 13  # int64 fields of one frontier route descriptor


# (allocator, request pool, request table, result) of the last pools checked
_NATIVE_POOLS: list = [None]


def _native_pools(alloc: Any, req: Any) -> bool:
    """A native paged allocator with a KV pool that moves rows, and a
    request pool with a dense int64 device table on the allocator's device
    (the answer for the last pools asked is kept)."""
    table = getattr(req, "req_to_token", None)
    hit = _NATIVE_POOLS[0]
    if hit is not None and hit[0] is alloc and hit[1] is req and hit[2] is table:
        return hit[3]
    ok = (callable(getattr(alloc, "consume_pages", None)) and callable(getattr(alloc, "get_kvcache", None))
          and callable(getattr(alloc.get_kvcache(), "move_kv_cache", None))
          and isinstance(table, torch.Tensor) and table.ndim == 2 and table.dtype == torch.int64
          and table.is_contiguous() and table.device == alloc.device)
    _NATIVE_POOLS[0] = (alloc, req, table, bool(ok))
    return bool(ok)


def fused_frontier_supported(bridges: Sequence[SGLangRoutePoolBridge]) -> bool:
    """True when ``prepare_frontiers`` can run these bridges in one launch:
    distinct bridges over one native paged allocator (device free list and
    page ownership), one request-row pool with a dense int64 device table,
    one KV pool with ``move_kv_cache``, one page size, page metadata on."""
    if not bridges or (len(bridges) > 1 and len({id(b) for b in bridges}) != len(bridges)):
        return False
    b0 = bridges[0]
    alloc, req = b0.token_to_kv_pool_allocator, b0.req_to_token_pool
    if not _native_pools(alloc, req):
        return False
    for b in bridges:
        if b.token_to_kv_pool_allocator is not alloc or b.req_to_token_pool is not req:
            return False
        if int(b.page_size) != int(b0.page_size) or not b._device_ownership or not b.use_page_attention_metadata:
            return False
    return True


def release_unreferenced_node_slots_many(bridges: Sequence[SGLangRoutePoolBridge],
                                         live_node_id_lists: Sequence[Sequence[int]]) -> list[int]:
    """``release_unreferenced_node_slots`` of several bridges.  Over one native
    allocator (``fused_frontier_supported``) every bridge's sweep is launched,
    the released-page counts come back in one copy and the released pages are
    prepended bridge by bridge, so the free list ends as one call per bridge in
    this order leaves it; the deferred device checks of all bridges run first.
    Otherwise one call per bridge.  Returns the page counts."""
    if len(bridges) != len(live_node_id_lists):
        raise ValueError("one live node list per bridge is required")
    if len(bridges) < 2 or not fused_frontier_supported(bridges):
        return [b.release_unreferenced_node_slots(live) for b, live in zip(bridges, live_node_id_lists)]
    return _sweep_bridges(bridges, live_node_id_lists, refresh_prefix=False)


def _sweep_bridges(bridges: Sequence[SGLangRoutePoolBridge], live_node_id_lists: Sequence[Sequence[int]], *,
                   refresh_prefix: bool) -> list[int]:
    """The native-pool prune of several bridges over one allocator: every
    sweep launched, then ONE copy to the host of the released-page counts,
    the flags of the bridges' pending fused frontier steps (and, with
    ``refresh_prefix``, each bridge's prefix page ids: the page of every
    page-start slot).  The deferred checks then run, so a failed one raises
    before any page goes back to the free list; the released pages are
    prepended bridge by bridge, so the free list ends as one call per bridge
    in this order leaves it."""
    # what comes back: the released-page counts, the prefix page starts and
    # the pending frontier steps' check words (all written by earlier launches
    # or by the sweeps below)
    parts = [b.owned_page_ids.free_count for b in bridges]
    starts: list[int] = []
    if refresh_prefix:
        for b in bridges:
            slots = b.prefix_slot_ids
            if slots is None or int(slots.numel()) == 0:
                starts.append(0)
                continue
            parts.append(slots[:: b.page_size])
            starts.append(int(parts[-1].numel()))
    flags = _unread_step_flags(bridges)
    tensors = [*parts, *(f.flags for f in flags)]
    plan = _HOST_GATHER.segments(tensors)
    fused = bridges[-1] if plan is not None else None  # its sweep also does the read-back
    for b in bridges:
        if b is fused:
            continue
        paths, last = b._live_paths()
        if not b.owned_page_ids.sweep_paths_launch(paths, last):
            b.owned_page_ids.sweep_launch(b._live_slot_samples())
    if fused is not None:
        segs, n, total = plan
        pages = fused.owned_page_ids

        def launch(out):
            paths, last = fused._live_paths()
            if not pages.sweep_paths_launch(paths, last, gather=(segs, n, out)):
                pages.sweep_launch(fused._live_slot_samples())
                _lib.check(_lib.load().atlas_gather_i64(segs, n, out, _lib.stream_of(pages.device)),
                           "atlas_gather_i64")

        flat = _read_back_split(parts, flags, _HOST_GATHER.run(launch, total, pages.device))
    else:
        flat = _read_back(parts, bridges)
    for b in bridges:
        b.check_pending_device_checks()
    counts = flat[: len(bridges)]
    if refresh_prefix:
        off = len(bridges)
        for b, c in zip(bridges, starts):
            b.prefix_slot_count = 0 if b.prefix_slot_ids is None else int(b.prefix_slot_ids.numel())
            ps = b.page_size
            b.prefix_page_ids = {s // ps for s in flat[off:off + c]}
            off += c
    alloc = bridges[0].token_to_kv_pool_allocator
    for b, live, n in zip(bridges, live_node_id_lists, counts):
        b._forget_dead_nodes(live)
        if n:
            b._require_allocator_free()
            alloc.free_pages_prepend(b.owned_page_ids.free_pages[:n])
    return counts


def prepare_frontiers(bridges: Sequence[SGLangRoutePoolBridge],
                      route_lists: Sequence[Sequence[RouteState]]) -> FusedFrontierStep:
    """``prepare_frontier`` of several requests' bridges as one step: one
    upload, one launch (copy-on-write page choice, decode slots, new slot
    paths, request-row writes, page tables, owned pages, checks), and one KV
    move for every copied tail.  Each bridge ends in the state, with the
    counters and the deferred checks, that ``prepare_frontier`` on its own
    routes leaves, taking pages from the shared free list in request order
    (its copy-on-write pages, then its decode pages), as the per-request
    calls in that order do.  The reference prepares one request per call
    (``flashinfer_paged/sglang_runtime.py:800-959``)."""
    if len(bridges) != len(route_lists) or not bridges:
        raise ValueError("one route list per bridge is required")
    if not fused_frontier_supported(bridges):
        raise ValueError("prepare_frontiers needs distinct bridges over one set of native pools "
                         "(see fused_frontier_supported)")
    return _prepare_frontiers(bridges, route_lists)


def _prepare_frontiers(bridges: Sequence[SGLangRoutePoolBridge],
                       route_lists: Sequence[Sequence[RouteState]]) -> FusedFrontierStep:
    """``prepare_frontiers`` once ``fused_frontier_supported`` holds."""
    b0 = bridges[0]
    alloc = b0.token_to_kv_pool_allocator
    table = b0.req_to_token_pool.req_to_token
    ps = int(b0.page_size)
    device = alloc.device
    plans = [b._plan_fused_frontier(rs) for b, rs in zip(bridges, route_lists)]

    desc: list[int] = []
    tokens: list[int] = []
    route_ids: list[int] = []
    seq_lens: list[int] = []
    spans: list[tuple[int, int]] = []
    flat_off = page_off = cow_off = free_idx = 0
    for g, (b, plan) in enumerate(zip(bridges, plans)):
        first = len(seq_lens)
        n = len(plan.prevs)
        bitmap = int(b.owned_page_ids.bitmap.data_ptr())
        cow_base = free_idx
        free_idx += plan.num_cow
        for i in range(n):
            prev = plan.prevs[i]
            tail = plan.cow_tail[i]
            if tail:
                cow_free, cow_at = cow_base + plan.cow_rank[i], cow_off
                cow_off += tail
            else:
                cow_free, cow_at = -1, 0
            if prev % ps == 0:
                new_free = free_idx
                free_idx += 1
            else:
                new_free = -1
            desc += (int(plan.paths[i].data_ptr()) if prev else 0, prev, tail, cow_free, cow_at, new_free,
                     flat_off, page_off, plan.rows[i], plan.starts[i], bitmap, first, n)
            flat_off += prev + 1
            page_off += (prev + ps) // ps
            seq_lens.append(prev + 1)
        tokens += [int(r.pending_token_id) for r in plan.routes]
        route_ids += [int(r.route_id) for r in plan.routes]
        spans.append((first, first + n))
    num_free = int(alloc.available_size()) // ps
    if free_idx > num_free:
        raise RuntimeError(f"SGLang KV pool cannot allocate {free_idx} pages for the frontier step "
                           f"({num_free} free)")
    R = len(seq_lens)
    F, C, P = flat_off, cow_off, page_off
    # launch arguments carry one request's descriptors; larger steps upload them
    by_value = R <= _lib.FRONTIER_MAX_HOST_ROUTES
    # one allocation: the int64 outputs (a check word per route; the model
    # inputs when the launch writes them), then the int32 ones
    n32 = 3 * R + 1 + P
    # flat paths, decode slots, check words, [copy pairs], [model inputs], the int32 outputs
    sizes = [F, R, R] + ([C, C] if C else []) + ([R] * 5 if by_value else []) + [(n32 + 1) // 2]
    out = torch.empty(sum(sizes), dtype=torch.int64, device=device)
    parts = out.split(sizes)
    flat, out_slots, flags = parts[:3]
    cow_dst, cow_src = parts[3:5] if C else (None, None)
    kv_indptr, kv_last, seq32, page_ids, _ = parts[-1].view(torch.int32).split([R + 1, R, R, P, n32 % 2])
    lib = _lib.load()
    free_ptr, table_ptr = alloc.free_pages.data_ptr(), table.data_ptr()
    cow = (cow_dst.data_ptr(), cow_src.data_ptr()) if C else (None, None)
    if by_value:
        input_ids, seq_dev, pos_dev, req_dev, rid_dev = parts[-6:-1]
        host = np.asarray(desc + tokens + route_ids, dtype=np.int64)
        base = host.ctypes.data
        rc = lib.atlas_pool_prepare_frontier_host(
            base, base + 8 * _ROUTE_FIELDS * R, base + 8 * (_ROUTE_FIELDS + 1) * R, R, free_ptr, num_free, ps,
            int(b0.owned_page_ids.num_pages), table_ptr, int(table.shape[0]), int(table.stride(0)), flat.data_ptr(),
            F, out_slots.data_ptr(), *cow, C, kv_indptr.data_ptr(), kv_last.data_ptr(), seq32.data_ptr(),
            page_ids.data_ptr(), P, flags.data_ptr(), input_ids.data_ptr(), _lib.stream_of(device),
        )
        _lib.check(rc, "atlas_pool_prepare_frontier_host")
    else:
        positions = [n - 1 for n in seq_lens]
        rows = [r for plan in plans for r in plan.rows]
        packed = _lib.upload_i64(desc + tokens + seq_lens + positions + rows + route_ids, device)
        input_ids, seq_dev, pos_dev, req_dev, rid_dev = packed[_ROUTE_FIELDS * R:].split(R)
        rc = lib.atlas_pool_prepare_frontier(
            packed.data_ptr(), R, free_ptr, num_free, ps, int(b0.owned_page_ids.num_pages), table_ptr,
            int(table.shape[0]), int(table.stride(0)), flat.data_ptr(), F, out_slots.data_ptr(), *cow, C,
            kv_indptr.data_ptr(), kv_last.data_ptr(), seq32.data_ptr(), page_ids.data_ptr(), P, flags.data_ptr(),
            _lib.stream_of(device),
        )
        _lib.check(rc, "atlas_pool_prepare_frontier")
    if C:
        alloc.get_kvcache().move_kv_cache(cow_dst, cow_src)
    alloc.consume_pages(free_idx)

    full = flat.split(seq_lens)
    step_flags = _StepFlags(flags, spans)
    for g, (b, plan) in enumerate(zip(bridges, plans)):
        lo, hi = spans[g]
        b._finish_fused_frontier(plan, full[lo:hi], step_flags, g)
    meta = SGLangRouteKVMetadata(
        req_pool_indices=req_dev, seq_lens=seq_dev, out_cache_loc=out_slots, positions=pos_dev,
        orig_seq_lens=seq_dev, seq_lens_sum=F, seq_lens_cpu=torch.tensor(seq_lens, dtype=torch.long),
        attention_page_size=ps, token_index_count=F, page_index_count=P,
        paged_decode_spec=AtlasPagedDecodeSpec(kv_indptr, page_ids, kv_last, ps),
    )
    return FusedFrontierStep(input_ids, meta, rid_dev, tuple(spans), tuple(n - 1 for n in seq_lens))


class SGLangFlashInferFrontierModelBackend:
    """Drafter frontier backend over the route pool
    (``sglang_runtime.py:1120-1346``).

    ``executor`` runs the Drafter model and must write each new token's K/V
    into the slots it is given (the model itself is outside this path):

    * ``forward_frontier(input_ids=, route_kv_metadata=) -> logits [B, V]``
      (one DECODE step: K/V of route i go to ``out_cache_loc[i]``);
    * ``forward_extend(input_ids=, out_cache_loc=, positions=,
      req_pool_indices=, seq_lens_cpu=) -> logits [n, V] or [V]``
      (one EXTEND of a known causal suffix).

    The reference's SGLang executor (``forward_frontier`` and a
    ``model_runner``, no ``forward_extend``; what ``from_runner`` builds when
    the reference is loaded) works too: the EXTEND then runs as an SGLang
    ``ForwardBatch`` on its runner, and each forward is preceded by the
    reference's runner set-up, as in its own backend.
    """

    def __init__(self, *, route_store: KVTreeStore, executor: Any, route_pool: SGLangRoutePoolBridge) -> None:
        self.route_store = route_store
        self.executor = executor
        self.route_pool = route_pool
        self.prefix_token_ids: tuple[int, ...] = ()
        self.prefix_next_token_logits: torch.Tensor | None = None
        hook = getattr(route_store, "add_route_release_hook", None)
        if callable(hook):
            hook(route_pool.reconcile_route_rows)

    @classmethod
    def from_runner(cls, *, route_store: KVTreeStore, model_runner: Any, page_size: int,
                    device: str | torch.device = "cuda", executor: Any = None) -> "SGLangFlashInferFrontierModelBackend":
        """``sglang_runtime.py:1139-1151``: a route pool over the runner's
        request and KV pools (``SGLangRoutePoolBridge.from_runner``, which
        checks the page size) and an executor that runs the Drafter model on
        the runner.  The model forward is the caller's: ``executor`` when
        given, else the reference's ``SGLangFlashInferPagedDecodeBackend``
        (after the reference's runner defaults and FlashInfer check) when the
        reference package is loaded beside this one.  Without either it
        raises ``RuntimeError`` before touching the runner."""
        if executor is None:
            ref = _reference_runtime()
            if ref is None:
                raise RuntimeError(
                    "from_runner needs the Drafter model executor: pass executor=, or load atlas_0709 (its "
                    "SGLangFlashInferPagedDecodeBackend runs the SGLang ModelRunner)")
            ref.ensure_sglang_runner_runtime_defaults(model_runner)
            ref.assert_sglang_flashinfer_active(model_runner)
            executor = ref.SGLangFlashInferPagedDecodeBackend(model_runner=model_runner, page_size=page_size)
        route_pool = SGLangRoutePoolBridge.from_runner(model_runner, page_size=page_size, device=device)
        return cls(route_store=route_store, executor=executor, route_pool=route_pool)

    def attach_prefilled_prefix(self, *, prompt_token_ids: Sequence[int], prefix_slot_ids,
                                next_token_logits: torch.Tensor) -> DraftPrefixState:
        self.prefix_token_ids = tuple(int(t) for t in prompt_token_ids)
        self.prefix_next_token_logits = next_token_logits
        self.route_pool.set_prefix_slots(prefix_slot_ids)
        n = len(self.prefix_token_ids)
        return DraftPrefixState(
            token_ids=torch.tensor(self.prefix_token_ids, dtype=torch.long, device=next_token_logits.device),
            prefix_kv_view=PrefixKVView(committed_length=n), next_token_logits=next_token_logits,
            committed_length=n)

    def set_prefix(self, token_ids: Sequence[int]) -> None:
        self.prefix_token_ids = tuple(int(t) for t in token_ids)

    @torch.inference_mode()
    def append_known_tokens_as_prefix(self, token_ids: Sequence[int]) -> torch.Tensor:
        """Fallback EXTEND: slots continuing the prefix's partial tail page,
        one request-row write, one EXTEND forward, then the extended path
        becomes the prefix with a fresh tail lease (``:1171-1251``)."""
        suffix = tuple(int(t) for t in token_ids)
        if not suffix:
            raise ValueError("known prefix extension cannot be empty")
        pool = self.route_pool
        prefix_slots = pool.prefix_slot_ids
        if prefix_slots is None or int(prefix_slots.numel()) != len(self.prefix_token_ids):
            raise RuntimeError("persistent Drafter prefix slots are not initialized")
        device = pool.device
        prefix_len = len(self.prefix_token_ids)
        seq_len = prefix_len + len(suffix)
        handle = _PoolReqHandle(rid="atlas-known-prefix-extend")
        indices = pool.req_to_token_pool.alloc([handle])
        if indices is None:
            raise RuntimeError("SGLang ReqToTokenPool.alloc returned None for known-token extend")
        row = int(_int_list(indices)[0])
        handle.req_pool_idx = row
        try:
            last = prefix_slots[-1:].to(torch.long) if prefix_len else torch.full((1,), -1, dtype=torch.long,
                                                                                 device=device)
            suffix_slots = pool.allocate_extend_slots(prefix_lens=[prefix_len], seq_lens=[seq_len], last_locs=last)
            full = torch.cat([prefix_slots, suffix_slots])
            pool._write_req_token_row(row, full)
            logits = _forward_extend(
                self.executor, input_ids=torch.tensor(suffix, dtype=torch.long, device=device),
                out_cache_loc=suffix_slots,
                positions=torch.arange(prefix_len, seq_len, dtype=torch.long, device=device),
                req_pool_indices=torch.tensor([row], dtype=torch.long, device=device),
                seq_lens_cpu=torch.tensor([seq_len], dtype=torch.long), prefix_lens=[prefix_len])
        finally:
            if hasattr(pool.req_to_token_pool, "free"):
                pool.req_to_token_pool.free(handle)
        pool.set_prefix_slots(full)
        self.prefix_token_ids = (*self.prefix_token_ids, *suffix)
        return logits if logits.ndim == 1 else logits[-1]

    def commit_stage1_and_promote(self, *, committed_route: RouteState, retained_routes: Sequence[RouteState]):
        """Promote the committed route's path to the prefix (no KV copy),
        rebase the retained routes, free the other rows, prune
        (``:1256-1297``).  Over the native pools this is the multi-request
        commit for one request (the new prefix's page ids and the pruned-page
        count come back in one copy); over other pools the per-step host
        path.  Both leave the same state."""
        if fused_frontier_supported([self.route_pool]):
            return SGLangFlashInferFrontierModelBackend.commit_stage1_and_promote_many(
                [self], [committed_route], [retained_routes])[0]
        nodes = self.route_store.node_path_for_route(committed_route)
        if not nodes:
            raise ValueError("cannot commit a stage-1 route with no materialized nodes")
        tokens = self.route_store.tokens_for_node_ids(nodes)
        self.route_pool.commit_route_as_prefix(committed_route)
        stored = self.route_store.commit_route(committed_route)
        if stored != tokens:
            raise RuntimeError("logical committed tokens changed during route promotion")
        self.prefix_token_ids = (*self.prefix_token_ids, *tokens)
        promoted = self.route_store.promote_routes_after_commit(
            committed_route, retained_routes, PrefixKVView(committed_length=len(self.prefix_token_ids)))
        released_rows = self.route_pool.retain_route_rows([r.route_id for r in promoted])
        live = sorted({int(n) for r in promoted for n in r.kv_view.node_ids})
        released_pages = self.route_pool.release_unreferenced_node_slots(live)
        return promoted, {
            "committed_kv_tokens": len(nodes),
            "retained_routes": len(promoted),
            "released_route_rows": released_rows,
            "released_kv_pages": released_pages,
        }

    @staticmethod
    def commit_stage1_and_promote_many(backends: Sequence["SGLangFlashInferFrontierModelBackend"],
                                       committed_routes: Sequence[RouteState],
                                       retained_route_lists: Sequence[Sequence[RouteState]]) -> list[tuple]:
        """``commit_stage1_and_promote`` of several requests.  When their
        bridges share native pools: the promotions and row releases run request
        by request on the host, then every request's prefix page ids come back
        in one copy and the prunes share one count read-back
        (``release_unreferenced_node_slots_many``), so the free list, the
        request rows and each request's state end as one call per request in
        this order leaves them.  Requests with no committed node are refused
        before any state changes; the deferred device checks run with the
        prunes' read-back, before any page returns to the free list.
        Otherwise one call per request.  Returns each request's
        ``(promoted routes, stats)``."""
        if not (len(backends) == len(committed_routes) == len(retained_route_lists)):
            raise ValueError("one committed route and one retained list per backend are required")
        bridges = [b.route_pool for b in backends]
        if not bridges:
            return []
        if not fused_frontier_supported(bridges):
            return [b.commit_stage1_and_promote(committed_route=c, retained_routes=k)
                    for b, c, k in zip(backends, committed_routes, retained_route_lists)]
        node_paths = [b.route_store.node_path_for_route(c) for b, c in zip(backends, committed_routes)]
        if not all(node_paths):
            raise ValueError("cannot commit a stage-1 route with no materialized nodes")
        results, lives = [], []
        for b, committed, keep, nodes in zip(backends, committed_routes, retained_route_lists, node_paths):
            tokens = b.route_store.tokens_for_node_ids(nodes)
            b.route_pool.commit_route_as_prefix(committed, defer_page_ids=True)
            stored = b.route_store.commit_route(committed)
            if stored != tokens:
                raise RuntimeError("logical committed tokens changed during route promotion")
            b.prefix_token_ids = (*b.prefix_token_ids, *tokens)
            promoted = b.route_store.promote_routes_after_commit(
                committed, keep, PrefixKVView(committed_length=len(b.prefix_token_ids)))
            released_rows = b.route_pool.retain_route_rows([r.route_id for r in promoted])
            lives.append(sorted({int(n) for r in promoted for n in r.kv_view.node_ids}))
            results.append((promoted, {"committed_kv_tokens": len(nodes), "retained_routes": len(promoted),
                                       "released_route_rows": released_rows}))
        counts = _sweep_bridges(bridges, lives, refresh_prefix=True)
        for (_, stats), n in zip(results, counts):
            stats["released_kv_pages"] = n
        return results

    @torch.inference_mode()
    def decode_frontier_one_token(self, active_routes: Sequence[RouteState],
                                  attention_backend: object = None) -> FrontierDecodeOutput:
        """One Drafter decode step of this request's routes
        (``sglang_runtime.py:1299-1346``).  Over the native pools it is the
        multi-request step for a single request (``decode_frontiers``: one
        upload and one launch for the routes' paths, slots, rows and page
        table, and deferred checks read back together at the next prune);
        over other pools the per-route host path of ``prepare_frontier``.
        Both leave the same bridge state."""
        if fused_frontier_supported([self.route_pool]):
            return SGLangFlashInferFrontierModelBackend._decode_fused(
                [self], [active_routes], None, attention_backend)[0]
        start = time.perf_counter()
        before = self.route_pool.hot_path_counters()
        new_nodes = self.route_store.reserve_node_ids(len(active_routes))
        input_ids, metadata = self.route_pool.prepare_frontier(active_routes)
        _ready_runner(self.executor)
        logits = self.executor.forward_frontier(input_ids=input_ids, route_kv_metadata=metadata)
        self.route_pool.register_node_slots(new_nodes, metadata.out_cache_loc)
        ids = [int(r.route_id) for r in active_routes]
        on_device = input_ids.device.type != "cpu"
        route_ids = torch.tensor(ids, dtype=torch.long, pin_memory=on_device).to(input_ids.device,
                                                                                 non_blocking=True)
        return self._frontier_output(route_ids, logits, new_nodes, start, before, metadata.attention_page_size,
                                     metadata.token_index_count, metadata.page_index_count, attention_backend)

    def _frontier_output(self, route_ids, logits, new_nodes, start, before, page_size, token_indices,
                         page_indices, attention_backend) -> FrontierDecodeOutput:
        after = self.route_pool.hot_path_counters()
        return FrontierDecodeOutput(
            route_ids=route_ids,
            next_token_logits=logits, new_node_ids=tuple(new_nodes), new_node_ids_cpu=tuple(new_nodes),
            model_ms=(time.perf_counter() - start) * 1000.0,
            metadata={
                "backend": "atlas_hip_paged_decode",
                "reference_only": False,
                "paged_kv": True,
                "cascade": False,
                "route_tail_page_cow": True,
                "branch_safe_page_size": True,
                "cow_pages_copied_total": int(self.route_pool.cow_pages_copied),
                "cow_tokens_copied_total": int(self.route_pool.cow_tokens_copied),
                "attention_metadata_page_size": int(page_size),
                "attention_metadata_token_indices_step": int(token_indices),
                "attention_metadata_page_indices_step": int(page_indices),
                "hot_path_counter_delta": {k: v - before.get(k, 0) for k, v in after.items()},
                "hot_path_counters_total": after,
                "attention_backend": str(attention_backend),
                **_executor_metadata(self.executor),
            },
        )

    @staticmethod
    @torch.inference_mode()
    def decode_frontiers(backends: Sequence["SGLangFlashInferFrontierModelBackend"],
                         route_lists: Sequence[Sequence[RouteState]], *, executor: Any = None,
                         attention_backend: object = None) -> list[FrontierDecodeOutput]:
        """``decode_frontier_one_token`` of several requests as one step:
        when their bridges share native pools, one ``prepare_frontiers`` and
        ONE ``forward_frontier`` of the union batch (``executor``, default the
        first backend's), whose logits rows and decode slots are handed back
        request by request; otherwise one call per request.  Each request's
        output and bridge state equal its own call's."""
        if len(backends) != len(route_lists):
            raise ValueError("one route list per backend is required")
        bridges = [b.route_pool for b in backends]
        if not fused_frontier_supported(bridges):
            return [b.decode_frontier_one_token(rs, attention_backend) for b, rs in zip(backends, route_lists)]
        return SGLangFlashInferFrontierModelBackend._decode_fused(backends, route_lists, executor, attention_backend)

    @staticmethod
    def _decode_fused(backends, route_lists, executor, attention_backend) -> list[FrontierDecodeOutput]:
        """``decode_frontiers`` once ``fused_frontier_supported`` holds."""
        if not all(route_lists):
            raise ValueError("active_routes cannot be empty")
        bridges = [b.route_pool for b in backends]
        start = time.perf_counter()
        before = [b.hot_path_counters() for b in bridges]
        new_nodes = [b.route_store.reserve_node_ids(len(rs)) for b, rs in zip(backends, route_lists)]
        step = _prepare_frontiers(bridges, route_lists)
        ex = executor if executor is not None else backends[0].executor
        _ready_runner(ex)
        logits = ex.forward_frontier(input_ids=step.input_ids, route_kv_metadata=step.metadata)
        out_slots = step.metadata.out_cache_loc
        outputs = []
        # one request whose rows are the whole batch: no slices
        whole = len(backends) == 1 and int(logits.shape[0]) == step.spans[0][1]
        for i, b in enumerate(backends):
            lo, hi = step.spans[i]
            b.route_pool.register_node_slots(new_nodes[i], out_slots if whole else out_slots[lo:hi])
            ps = int(b.route_pool.page_size)
            prevs = step.prevs[lo:hi]
            outputs.append(b._frontier_output(
                step.route_ids if whole else step.route_ids[lo:hi], logits if whole else logits[lo:hi],
                new_nodes[i], start, before[i], ps, sum(prevs) + len(prevs), sum((p + ps) // ps for p in prevs),
                attention_backend))
        return outputs

    @staticmethod
    @torch.inference_mode()
    def append_known_tokens_as_prefix_many(backends: Sequence["SGLangFlashInferFrontierModelBackend"],
                                           token_lists: Sequence[Sequence[int]], *,
                                           executor: Any = None) -> list[torch.Tensor]:
        """``append_known_tokens_as_prefix`` of several requests as one EXTEND:
        when their bridges share native pools, one request-row allocation, one
        ``alloc_extend`` for all requests (their new pages come off the free
        list in request order, as one call per request takes them), one
        request-row write and ONE ``forward_extend`` of the union batch
        (``executor``, default the first backend's; ``out_cache_loc``,
        ``positions`` and ``input_ids`` hold the requests' suffixes in order,
        ``req_pool_indices`` and ``seq_lens_cpu`` one entry per request);
        otherwise one call per request.  Each request's returned logits and
        bridge state equal its own call's (the temporary request rows aside,
        which are free again afterwards)."""
        if len(backends) != len(token_lists):
            raise ValueError("one token list per backend is required")
        suffixes = [tuple(int(t) for t in ts) for ts in token_lists]
        bridges = [b.route_pool for b in backends]
        union_ex = executor if executor is not None else (backends[0].executor if backends else None)
        if len(backends) < 2 or not fused_frontier_supported(bridges) or not hasattr(union_ex, "forward_extend"):
            # a runner-backed executor (no forward_extend) returns one logits
            # row per request, so its EXTENDs stay one per request
            return [b.append_known_tokens_as_prefix(sfx) for b, sfx in zip(backends, suffixes)]
        for b, sfx in zip(backends, suffixes):
            if not sfx:
                raise ValueError("known prefix extension cannot be empty")
            slots = b.route_pool.prefix_slot_ids
            if slots is None or int(slots.numel()) != len(b.prefix_token_ids):
                raise RuntimeError("persistent Drafter prefix slots are not initialized")
        pool = bridges[0]
        device = pool.device
        prefix_lens = [len(b.prefix_token_ids) for b in backends]
        lens = [len(sfx) for sfx in suffixes]
        seq_lens = [p + n for p, n in zip(prefix_lens, lens)]
        handles = [_PoolReqHandle(rid="atlas-known-prefix-extend") for _ in backends]
        indices = pool.req_to_token_pool.alloc(handles)
        if indices is None:
            raise RuntimeError("SGLang ReqToTokenPool.alloc returned None for known-token extend")
        rows = _int_list(indices)
        for h, row in zip(handles, rows):
            h.req_pool_idx = row
        try:
            lasts = torch.cat([b.route_pool.prefix_slot_ids[-1:].to(torch.long) if p
                               else torch.full((1,), -1, dtype=torch.long, device=device)
                               for b, p in zip(backends, prefix_lens)])
            suffix_slots = pool.allocate_extend_slots(prefix_lens=prefix_lens, seq_lens=seq_lens, last_locs=lasts)
            offs = np.concatenate(([0], np.cumsum(lens)))
            fulls = [torch.cat([b.route_pool.prefix_slot_ids, suffix_slots[int(offs[i]):int(offs[i + 1])]])
                     for i, b in enumerate(backends)]
            # every request's whole row in one tensor-index write; each bridge
            # checks and counts its own row as its own call would
            host = np.concatenate((np.repeat(np.asarray(rows, dtype=np.int64), seq_lens),
                                   np.concatenate([np.arange(n, dtype=np.int64) for n in seq_lens]),
                                   np.asarray([t for sfx in suffixes for t in sfx], dtype=np.int64),
                                   np.concatenate([np.arange(p, q, dtype=np.int64)
                                                   for p, q in zip(prefix_lens, seq_lens)]),
                                   np.asarray(rows, dtype=np.int64)))
            dev_vals = torch.from_numpy(host).to(device)
            total, ext = sum(seq_lens), int(offs[-1])
            row_idx, pos_idx = dev_vals[:total], dev_vals[total:2 * total]
            input_ids = dev_vals[2 * total:2 * total + ext]
            positions = dev_vals[2 * total + ext:2 * total + 2 * ext]
            req_idx = dev_vals[2 * total + 2 * ext:]
            for b, row, full in zip(backends, rows, fulls):
                b.route_pool._check_req_write(row, 0, int(full.numel()), "full_init")
            try:
                pool.req_to_token_pool.write((row_idx, pos_idx), torch.cat(fulls))
            except Exception as exc:
                raise RuntimeError("failed to write SGLang req_to_token_pool route row") from exc
            for b, full in zip(backends, fulls):
                b.route_pool._count_req_write(int(full.numel()), "full_init")
            logits = union_ex.forward_extend(input_ids=input_ids, out_cache_loc=suffix_slots, positions=positions,
                                       req_pool_indices=req_idx,
                                       seq_lens_cpu=torch.tensor(seq_lens, dtype=torch.long))
        finally:
            for h in handles:
                if hasattr(pool.req_to_token_pool, "free"):
                    pool.req_to_token_pool.free(h)
        # the new prefixes' pages: each old prefix's pages and those of its
        # suffix slots (one copy to the host for all suffixes)
        ps = int(pool.page_size)
        suffix_host = _int_list(suffix_slots)
        outputs = []
        for i, (b, sfx) in enumerate(zip(backends, suffixes)):
            pages = set(b.route_pool.prefix_page_ids)
            pages.update(s // ps for s in suffix_host[int(offs[i]):int(offs[i + 1])])
            b.route_pool.set_prefix_slots(fulls[i], page_ids=pages)
            b.prefix_token_ids = (*b.prefix_token_ids, *sfx)
            outputs.append(logits if logits.ndim == 1 else logits[int(offs[i + 1]) - 1])
        return outputs


# ------------------------------------------------------------------ executor glue
# The Drafter model forward is the caller's.  An executor either implements
# forward_frontier / forward_extend itself (the contract documented on
# SGLangFlashInferFrontierModelBackend), or is the reference's SGLang executor
# (``flashinfer_backends.py:64-121``: forward_frontier only, plus the
# ModelRunner it drives), in which case the reference's runner helpers run the
# forward exactly as its own backend does.

_REFERENCE_RUNTIME = "atlas_0709.flashinfer_paged.sglang_runtime"


def _reference_runtime():
    """The reference's route-pool module when it is loaded beside this
    package (the alias installed over it), else None."""
    mod = sys.modules.get(_REFERENCE_RUNTIME)
    if mod is None or mod is sys.modules.get(__name__):
        return None
    return mod


def _ready_runner(executor: Any) -> None:
    """Before a forward on a runner-backed executor: the reference's runner
    defaults and eager runner (``sglang_runtime.py:1309-1310``)."""
    runner = getattr(executor, "model_runner", None)
    ref = _reference_runtime()
    if runner is None or ref is None:
        return
    ref.ensure_sglang_runner_runtime_defaults(runner)
    ref.ensure_sglang_eager_runner(runner)


def _executor_metadata(executor: Any) -> dict:
    """The executor's own runtime metadata, when it reports any
    (``sglang_runtime.py:1344``)."""
    meta = getattr(executor, "runtime_metadata", None)
    return dict(meta(cascade_level=0, verify_backend="none")) if callable(meta) else {}


def _forward_extend(executor: Any, *, input_ids: torch.Tensor, out_cache_loc: torch.Tensor,
                    positions: torch.Tensor, req_pool_indices: torch.Tensor, seq_lens_cpu: torch.Tensor,
                    prefix_lens: Sequence[int]) -> torch.Tensor:
    """One EXTEND forward of known tokens: the executor's ``forward_extend``
    when it has one; otherwise an SGLang EXTEND ``ForwardBatch`` run on the
    executor's ModelRunner, with the fields the reference fills
    (``sglang_runtime.py:1211-1242``), one request per entry of
    ``seq_lens_cpu``."""
    fwd = getattr(executor, "forward_extend", None)
    if callable(fwd):
        return fwd(input_ids=input_ids, out_cache_loc=out_cache_loc, positions=positions,
                   req_pool_indices=req_pool_indices, seq_lens_cpu=seq_lens_cpu)
    runner = getattr(executor, "model_runner", None)
    ref = _reference_runtime()
    if runner is None or ref is None:
        raise RuntimeError("the Drafter executor has no forward_extend and no SGLang ModelRunner to run an EXTEND on")
    forward_batch_cls, forward_mode_cls = ref._sglang_forward_batch_classes()
    device = input_ids.device
    seq_cpu = [int(x) for x in seq_lens_cpu.tolist()]
    pre = [int(x) for x in prefix_lens]
    ext = [a - b for a, b in zip(seq_cpu, pre)]
    starts = [0]
    for n in ext[:-1]:
        starts.append(starts[-1] + n)
    seq_lens = seq_lens_cpu.to(device=device)
    batch = forward_batch_cls(
        forward_mode=ref._forward_mode(forward_mode_cls, ("EXTEND", "PREFILL")),
        batch_size=len(seq_cpu),
        input_ids=input_ids,
        req_pool_indices=req_pool_indices,
        seq_lens=seq_lens,
        out_cache_loc=out_cache_loc,
        seq_lens_sum=sum(seq_cpu),
        orig_seq_lens=seq_lens,
        positions=positions,
        seq_lens_cpu=seq_lens_cpu,
        capture_hidden_mode=ref._capture_hidden_mode_null(),
        is_extend_in_batch=True,
        all_extend_in_batch=True,
        extend_num_tokens=sum(ext),
        extend_seq_lens=torch.tensor(ext, device=device, dtype=torch.long),
        extend_prefix_lens=torch.tensor(pre, device=device, dtype=torch.long),
        extend_start_loc=torch.tensor(starts, device=device, dtype=torch.long),
        extend_seq_lens_cpu=ext,
        extend_prefix_lens_cpu=pre,
        extend_logprob_start_lens_cpu=[n - 1 for n in ext],
    )
    ref.ensure_sglang_runner_runtime_defaults(runner)
    ref.ensure_sglang_eager_runner(runner)
    logits = ref._extract_next_token_logits(runner.forward(batch))
    if device.type == "cuda":
        # the reference synchronises after the EXTEND forward (:1242)
        torch.cuda.synchronize(device)
    return logits


_COUNTERS = (
    "attention_metadata_builds",
    "attention_metadata_token_indices",
    "attention_metadata_page_indices",
    "cow_pages_copied",
    "cow_tokens_copied",
    "req_row_write_calls",
    "req_row_elements_written",
    "req_row_full_rewrite_calls",
    "req_row_full_rewrite_elements",
    "req_row_full_init_calls",
    "req_row_full_init_elements",
    "req_row_append_calls",
    "req_row_append_elements",
    "req_row_cow_patch_calls",
    "req_row_cow_patch_elements",
    "hot_path_host_transfer_batches",
    "hot_path_host_transfer_elements",
)
_get_counters = operator.attrgetter(*_COUNTERS)


def _allocate_kv_slots(allocator: Any, count: int, *, mode: str) -> Any:
    names = {"extend": ["alloc_extend", "alloc"], "decode": ["alloc_decode", "alloc"]}.get(mode, ["alloc"])
    errors: list[str] = []
    for name in names:
        fn = getattr(allocator, name, None)
        if not callable(fn):
            continue
        try:
            result = fn(int(count))
        except Exception as exc:
            errors.append(f"{name}({int(count)},): {exc!r}")
            continue
        if result is not None:
            return result
        errors.append(f"{name}({int(count)},): returned None")
    raise RuntimeError(
        "SGLang token_to_kv_pool_allocator could not allocate slots. "
        + ("; ".join(errors) if errors else "no supported allocation method")
    )


def _slot_tensor(result: Any, device) -> torch.Tensor:
    if isinstance(result, torch.Tensor):
        return _as_long(result, device)
    if isinstance(result, (list, tuple)):
        tensors = [x for x in result if isinstance(x, torch.Tensor)]
        if tensors:
            return _as_long(tensors[0], device)
        flat: list[int] = []
        for item in result:
            if isinstance(item, int):
                flat.append(int(item))
            elif isinstance(item, (list, tuple)) and all(isinstance(v, int) for v in item):
                flat.extend(int(v) for v in item)
        if flat:
            return _as_long(flat, device)
    return _as_long(result, device)


def _req_pool_capacity(req_pool: Any) -> int | None:
    if req_pool is None:
        return None
    for name in ("req_to_token", "req_to_token_pool", "req_to_token_table", "pool", "data"):
        value = getattr(req_pool, name, None)
        if isinstance(value, torch.Tensor) and value.ndim >= 2:
            return int(value.shape[1])
    try:
        attrs = vars(req_pool)
    except TypeError:
        return None
    for value in attrs.values():
        if isinstance(value, torch.Tensor) and value.ndim >= 2:
            return int(value.shape[1])
    return None


def _as_long(value, device) -> torch.Tensor:
    t = value if isinstance(value, torch.Tensor) else torch.tensor(list(value), dtype=torch.long)
    t = t.to(device=device, dtype=torch.long)
    if t.ndim != 1:
        raise ValueError(f"expected a 1D tensor, got shape {tuple(t.shape)}")
    return t


def _assert_true(condition: torch.Tensor, message: str) -> None:
    """Host check of a scalar tensor.  (The reference uses a device-side
    assertion on GPU tensors; a device trap is avoided here, so a GPU
    condition is read back, which synchronises -- this check runs only on
    foreign-allocator and lease-less compatibility paths.)"""
    if condition.numel() != 1:
        raise ValueError("device assertion condition must be scalar")
    if not bool(condition.item()):
        raise RuntimeError(message)


def _int_list(value) -> list[int]:
    if isinstance(value, torch.Tensor):
        return [int(x) for x in value.detach().cpu().reshape(-1).tolist()]
    return [int(x) for x in value]
