"""Physical page tables from token-slot paths (drop-in for the reference's
``flashinfer_paged/paged_metadata.py``).

One kernel launch compresses every path: page ids are the first slot of each
page divided by page_size, and the layout check (page-aligned starts,
contiguous slots inside each page) clears a device flag
(``paged_metadata.py:87-102`` of the reference).  The builder reads nothing
back to the host.  The reference raises through ``torch._assert_async``
(``:123-138``), a device-side trap; here the flag is kept in the metadata and
``assert_layout_valid()`` raises the same ``RuntimeError`` on the host at the
caller's next synchronisation point (``sync_check=True`` checks at once).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import torch

from .. import _lib

LAYOUT_MESSAGE = (
    "physical KV slot paths are not page-aligned contiguous pages; "
    "cannot safely compress token slots into FlashInfer page indices"
)


@dataclass(frozen=True)
class FlashInferPagedKVMetadata:
    """``paged_metadata.py:9-29``: ``kv_indptr`` counts pages,
    ``kv_page_indices`` holds physical page ids, ``kv_last_page_len`` the valid
    tokens of each route's last page; ``token_index_count`` is the size of the
    token-level representation the page table replaces."""

    kv_indptr: torch.Tensor
    kv_page_indices: torch.Tensor
    kv_last_page_len: torch.Tensor
    seq_lens: torch.Tensor
    page_size: int
    token_index_count: int
    layout_validated: bool
    layout_flag: torch.Tensor | None = None

    @property
    def page_index_count(self) -> int:
        return int(self.kv_page_indices.numel())

    def assert_layout_valid(self) -> None:
        """Raise ``RuntimeError`` if validation found a non page-aligned or
        non-contiguous page (reads one int32 from the device)."""
        if self.layout_flag is not None and not bool(self.layout_flag.item()):
            raise RuntimeError(LAYOUT_MESSAGE)


def build_flashinfer_paged_kv_metadata(
    slot_paths: Sequence[torch.Tensor],
    *,
    page_size: int,
    validate_layout: bool = True,
    sync_check: bool = False,
) -> FlashInferPagedKVMetadata:
    if int(page_size) <= 0:
        raise ValueError("page_size must be positive")
    if not slot_paths:
        raise ValueError("slot_paths cannot be empty")
    first = slot_paths[0]
    if first.ndim != 1:
        raise ValueError(f"slot paths must be 1-D, got {tuple(first.shape)}")
    if first.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"slot paths must be int32/int64, got {first.dtype}")
    device = first.device
    ps = int(page_size)
    lens: list[int] = []
    for path in slot_paths:
        if path.ndim != 1:
            raise ValueError(f"slot paths must be 1-D, got {tuple(path.shape)}")
        if path.dtype not in (torch.int32, torch.int64):
            raise TypeError(f"slot paths must be int32/int64, got {path.dtype}")
        if path.device != device:
            raise ValueError("all slot paths must be on the same device")
        n = int(path.numel())
        if n <= 0:
            raise ValueError("FlashInfer paged decode requires non-empty slot paths")
        lens.append(n)
    _lib.require_device(first, what="build_flashinfer_paged_kv_metadata")
    counts = [(n + ps - 1) // ps for n in lens]
    path_offsets = [0]
    page_offsets = [0]
    for n, c in zip(lens, counts):
        path_offsets.append(path_offsets[-1] + n)
        page_offsets.append(page_offsets[-1] + c)
    last = [n - (c - 1) * ps for n, c in zip(lens, counts)]
    batch = len(lens)
    # One upload carries offsets, indptr, last-page lengths and sequence
    # lengths; the int32 outputs are views of one device buffer.
    host = torch.tensor(path_offsets + page_offsets, dtype=torch.int64)
    small = torch.tensor(page_offsets + last + lens + [1], dtype=torch.int32)
    dev64 = host.to(device, non_blocking=True)
    dev32 = small.to(device, non_blocking=True)
    kv_indptr = dev32[: batch + 1]
    kv_last = dev32[batch + 1 : 2 * batch + 1]
    seq_lens = dev32[2 * batch + 1 : 3 * batch + 1]
    flag = dev32[3 * batch + 1 : 3 * batch + 2]
    slots = torch.cat([p.to(torch.int64) for p in slot_paths]) if batch > 1 else first.to(torch.int64).contiguous()
    total_pages = page_offsets[-1]
    pages = torch.empty(total_pages, dtype=torch.int32, device=device)
    lib = _lib.load()
    rc = lib.atlas_paged_metadata(
        _lib.ptr(slots), _lib.ptr(dev64), int(dev64.data_ptr()) + 8 * (batch + 1), batch, total_pages, ps,
        1 if validate_layout else 0, _lib.ptr(pages), _lib.ptr(flag), _lib.stream_of(device),
    )
    _lib.check(rc, "atlas_paged_metadata")
    meta = FlashInferPagedKVMetadata(
        kv_indptr=kv_indptr,
        kv_page_indices=pages,
        kv_last_page_len=kv_last,
        seq_lens=seq_lens,
        page_size=ps,
        token_index_count=int(sum(lens)),
        layout_validated=bool(validate_layout),
        layout_flag=flag if validate_layout else None,
    )
    if validate_layout and sync_check:
        meta.assert_layout_valid()
    return meta
