"""The reference's own torch implementation of the KV legs, restated for the
CPU baseline -- TEST INFRASTRUCTURE (see oracle/__init__.py).

These follow the reference's torch index ops line for line, so that
``bench.py`` can time, on the host cores, what the reference itself runs for
the path the HIP kernels replace.  They are pinned bit for bit against the
numpy restatements in ``paged_kv`` (``tests/test_oracle_pinning.py``).
"""

from __future__ import annotations

from typing import Sequence

import torch


def commit_torch(layers: Sequence[torch.Tensor], prefix_len: int, node_ids: Sequence[int], page_size: int) -> None:
    """DirectFlashInferMaskedTreeVerifyBackend._commit_selected_path,
    target_runtime.py:886-912: per layer, gather the selected nodes' rows
    [page, :, offset], clone, scatter them to prefix_len + i."""
    device = layers[0].device
    src = torch.tensor([prefix_len + int(n) for n in node_ids], dtype=torch.long, device=device)
    dst = torch.arange(prefix_len, prefix_len + len(node_ids), dtype=torch.long, device=device)
    sp = torch.div(src, int(page_size), rounding_mode="floor")
    so = torch.remainder(src, int(page_size))
    dp = torch.div(dst, int(page_size), rounding_mode="floor")
    do = torch.remainder(dst, int(page_size))
    for layer_kv in layers:
        selected = layer_kv[sp, :, so].clone()
        layer_kv[dp, :, do] = selected


def write_suffix_kv_torch(kv_cache: torch.Tensor, key_states: torch.Tensor, value_states: torch.Tensor,
                          prefix_len: int, page_size: int) -> None:
    """write_suffix_kv, flashinfer_full_verify.py:1027-1042."""
    n = int(key_states.shape[0])
    positions = torch.arange(int(prefix_len), int(prefix_len) + n, device=key_states.device)
    pages = torch.div(positions, int(page_size), rounding_mode="floor").to(torch.long)
    offsets = torch.remainder(positions, int(page_size)).to(torch.long)
    kv_cache[pages, 0, offsets] = key_states
    kv_cache[pages, 1, offsets] = value_states


def cow_copy_torch(k_layers: Sequence[torch.Tensor], v_layers: Sequence[torch.Tensor],
                   copies: Sequence[tuple[torch.Tensor, torch.Tensor]]) -> None:
    """Tail-page copy-on-write as the reference issues it
    (sglang_runtime.py:760-785): one move_kv_cache(dst, src) per copied page,
    each moving the page's valid tail in every layer with SGLang's
    values[dst] = values[src] (tests/test_tail_page_cow.py:14-16)."""
    for dst, src in copies:
        for k, v in zip(k_layers, v_layers):
            k[dst] = k[src]
            v[dst] = v[src]


def prune_torch(owned_pages: set[int], prefix_slots: torch.Tensor | None, route_paths: Sequence[torch.Tensor],
                page_size: int) -> list[int]:
    """release_unreferenced_node_slots, sglang_runtime.py:507-539, with the
    live page sets of _page_id_sets_for_paths (:479-505: every page_size-th
    slot of a path plus its last slot, one batched device-to-host read) and
    the prefix pages (every page_size-th prefix slot, :189-203):
    sorted(owned - live)."""
    live: set[int] = set()
    if prefix_slots is not None and int(prefix_slots.numel()):
        live.update(int(x) for x in torch.div(prefix_slots[::page_size], page_size, rounding_mode="floor").tolist())
    parts = []
    for path in route_paths:
        if int(path.numel()):
            parts.append(torch.cat((path[::page_size], path[-1:])))
    if parts:
        pages = torch.div(torch.cat(parts), page_size, rounding_mode="floor").tolist()
        live.update(int(x) for x in pages)
    return sorted(owned_pages - live)
