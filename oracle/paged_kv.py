"""Oracle: integer / byte functions of the paged-KV tree path (numpy).

Test infrastructure only (see oracle/__init__.py).  KV tensors here are numpy
arrays; values are compared bit-exactly with the HIP path by viewing the
16-bit payloads as uint16.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Sequence

import numpy as np


# --------------------------------------------------------------------- a1
@dataclass
class PagedMetadata:
    kv_indptr: list[int]
    kv_page_indices: list[int]
    kv_last_page_len: list[int]
    seq_lens: list[int]
    token_index_count: int
    layout_ok: bool


def paged_metadata(slot_paths: Sequence[Sequence[int]], page_size: int) -> PagedMetadata:
    """build_flashinfer_paged_kv_metadata, flashinfer_paged/paged_metadata.py:32-120.

    Pages per path = ceil(len / page_size); page index = floor(slot[k * ps] / ps);
    last page length = len - (pages - 1) * ps; layout valid iff every page start
    is a multiple of ps and slot[i] == start[i // ps] + i % ps (:87-99).
    """
    if page_size <= 0:
        raise ValueError("page_size must be positive")
    if not slot_paths:
        raise ValueError("slot_paths cannot be empty")
    indptr = [0]
    pages: list[int] = []
    last: list[int] = []
    lens: list[int] = []
    ok = True
    for path in slot_paths:
        arr = np.asarray(path, dtype=np.int64)
        n = int(arr.size)
        if n <= 0:
            raise ValueError("FlashInfer paged decode requires non-empty slot paths")
        npages = (n + page_size - 1) // page_size
        starts = arr[::page_size]
        pages.extend(int(x) for x in np.floor_divide(starts, page_size))
        indptr.append(indptr[-1] + npages)
        last.append(n - (npages - 1) * page_size)
        lens.append(n)
        expected = np.repeat(starts, page_size)[:n] + (np.arange(n) % page_size)
        ok = ok and bool(np.all(np.remainder(starts, page_size) == 0)) and bool(np.all(arr == expected))
    return PagedMetadata(indptr, pages, last, lens, int(sum(lens)), ok)


# --------------------------------------------------------------------- a2
def dedup_tree(paths: Sequence[Sequence[int]]) -> tuple[list[int], list[int], list[int], list[list[int]]]:
    """build_deduplicated_path_tree_tokens, flashinfer_full_verify.py:570-616.

    Prefix trie; a node is created the first time its (parent, token) pair is
    seen, so nodes are numbered route by route, depth by depth.
    """
    if not paths:
        raise ValueError("paths must not be empty")
    if len({len(p) for p in paths}) != 1:
        raise ValueError("all paths must have the same length")
    if len(paths[0]) <= 0:
        raise ValueError("paths must contain at least one token")
    tokens: list[int] = []
    parents: list[int] = []
    depths: list[int] = []
    kids: list[dict[int, int]] = []
    root: dict[int, int] = {}
    routes: list[list[int]] = []
    for path in paths:
        parent, table, nodes = -1, root, []
        for depth, tok in enumerate(path):
            tok = int(tok)
            node = table.get(tok)
            if node is None:
                node = len(tokens)
                table[tok] = node
                tokens.append(tok)
                parents.append(parent)
                depths.append(depth)
                kids.append({})
            nodes.append(node)
            parent, table = node, kids[node]
        routes.append(nodes)
    return tokens, parents, depths, routes


# --------------------------------------------------------------------- a3
def ancestor_mask(parents: Sequence[int], prefix_len: int) -> np.ndarray:
    """Dense bool mask [n, prefix + n] of build_deduplicated_tree_spec_from_paths,
    flashinfer_full_verify.py:719-724: prefix columns True, tree column j True iff
    j is an ancestor-or-self (ancestors_inclusive, :619-625)."""
    n = len(parents)
    mask = np.zeros((n, prefix_len + n), dtype=bool)
    mask[:, :prefix_len] = True
    for i in range(n):
        cur = i
        while cur >= 0:
            mask[i, prefix_len + cur] = True
            cur = int(parents[cur])
    return mask


def packbits(mask: np.ndarray, bitorder: str = "big") -> np.ndarray:
    """flashinfer.packbits (numpy.packbits semantics), used at
    flashinfer_full_verify.py:502-507, :729."""
    return np.packbits(np.asarray(mask, dtype=bool).reshape(-1), bitorder=bitorder)


# --------------------------------------------------------------------- a5
def write_suffix(kv_cache: np.ndarray, key: np.ndarray, value: np.ndarray, start: int) -> None:
    """write_suffix_kv, flashinfer_full_verify.py:1027-1042: positions
    start + i -> (page = pos // ps, offset = pos % ps); K half 0, V half 1."""
    ps = kv_cache.shape[2]
    for i in range(key.shape[0]):
        pos = start + i
        kv_cache[pos // ps, 0, pos % ps] = key[i]
        kv_cache[pos // ps, 1, pos % ps] = value[i]


def prefix_to_paged(key: np.ndarray, value: np.ndarray, prefix_len: int, node_count: int, page_size: int,
                    total_pages: int | None = None) -> np.ndarray:
    """prefix_layer_to_paged_kv, flashinfer_full_verify.py:814-849 (key/value
    [1, H, T, D] -> zero-filled [pages, 2, ps, H, D])."""
    _, h, t, d = key.shape
    if total_pages is None:
        total_pages = (prefix_len + node_count + page_size - 1) // page_size
    cache = np.zeros((total_pages, 2, page_size, h, d), dtype=key.dtype)
    write_suffix(cache, key[0].transpose(1, 0, 2), value[0].transpose(1, 0, 2), 0)
    return cache


# --------------------------------------------------------------------- a6/a7
def commit(layers: Sequence[np.ndarray], prefix_len: int, node_ids: Sequence[int],
           kv_indices: Sequence[int] | None = None) -> None:
    """_commit_selected_path KV part, target_runtime.py:885-912: for every layer,
    gather rows at src = prefix_len + node_id, clone, scatter to
    dst = prefix_len + i.  Positions map through kv_indices when given (the
    generalised paged Target); identity otherwise."""
    n = len(node_ids)
    src = [prefix_len + int(x) for x in node_ids]
    dst = list(range(prefix_len, prefix_len + n))
    for layer in layers:
        ps = layer.shape[2]

        def phys(pos: int) -> tuple[int, int]:
            page = pos // ps
            return (int(kv_indices[page]) if kv_indices is not None else page), pos % ps

        gathered = np.stack([layer[phys(s)[0], :, phys(s)[1]] for s in src]).copy()
        for i, d in enumerate(dst):
            page, off = phys(d)
            layer[page, :, off] = gathered[i]


def grow_capacity(layers: list[np.ndarray], required_pages: int) -> list[np.ndarray]:
    """_ensure_page_capacity, target_runtime.py:858-871."""
    out = []
    for layer in layers:
        if layer.shape[0] >= required_pages:
            out.append(layer)
            continue
        grown = np.zeros((required_pages, *layer.shape[1:]), dtype=layer.dtype)
        grown[: layer.shape[0]] = layer
        out.append(grown)
    return out


# --------------------------------------------------------------------- a9/a11
def move_kv(pool_k: Sequence[np.ndarray], pool_v: Sequence[np.ndarray], dst: Sequence[int],
            src: Sequence[int]) -> None:
    """SGLang move_kv_cache as pinned by the reference fake:
    values[dst] = values[src] (tests/test_tail_page_cow.py:14-16), all layers."""
    d = np.asarray(dst, dtype=np.int64)
    s = np.asarray(src, dtype=np.int64)
    for k, v in zip(pool_k, pool_v):
        k[d] = k[s].copy()
        v[d] = v[s].copy()


def set_kv(pool_k: Sequence[np.ndarray], pool_v: Sequence[np.ndarray], slots: Sequence[int],
           k_rows: Sequence[np.ndarray], v_rows: Sequence[np.ndarray]) -> None:
    """SGLang set_kv_buffer (sglang_page_attention.py:187-194): pool[loc] = rows."""
    sl = np.asarray(slots, dtype=np.int64)
    for k, v, kr, vr in zip(pool_k, pool_v, k_rows, v_rows):
        k[sl] = kr
        v[sl] = vr


# --------------------------------------------------------------------- a13
def sampled_page_ids(path: Sequence[int], page_size: int, include_last: bool = True) -> set[int]:
    """_page_id_sets_for_paths, sglang_runtime.py:479-505 (path[::ps] plus the
    last slot), or _refresh_prefix_cpu_metadata :189-203 (path[::ps] only)."""
    arr = np.asarray(path, dtype=np.int64)
    if arr.size == 0:
        return set()
    parts = [arr[::page_size]]
    if include_last:
        parts.append(arr[-1:])
    return {int(x) for x in np.floor_divide(np.concatenate(parts), page_size)}


def prune(owned: set[int], prefix_slots: Sequence[int] | None, route_paths: Sequence[Sequence[int]],
          page_size: int) -> tuple[list[int], set[int]]:
    """release_unreferenced_node_slots, sglang_runtime.py:507-539:
    releasable = sorted(owned - (prefix pages | pages of every route path))."""
    live = set() if prefix_slots is None else sampled_page_ids(prefix_slots, page_size, include_last=False)
    for path in route_paths:
        live |= sampled_page_ids(path, page_size)
    releasable = sorted(owned - live)
    return releasable, owned - set(releasable)


# --------------------------------------------------------------------- allocator
@dataclass
class PagedAllocator:
    """Paged free-list policy of SGLang's PagedTokenToKVPoolAllocator as driven
    by the reference (sglang_runtime.py:578-684, :1587-1597, need_sort=False):
    pages 1..num_pages free in ascending order (page 0 reserved for padding);
    alloc takes pages from the head; free prepends the sorted unique pages of
    the freed slots; decode continues a partial tail page, otherwise opens the
    next free page; extend fills the tail page, then opens pages in order.
    """

    num_pages: int
    page_size: int
    free_pages: list[int] = field(default_factory=list)

    def __post_init__(self) -> None:
        self.clear()

    def clear(self) -> None:
        self.free_pages = list(range(1, self.num_pages + 1))

    def alloc(self, need_size: int) -> list[int] | None:
        n = need_size // self.page_size
        if n > len(self.free_pages):
            return None
        pages, self.free_pages = self.free_pages[:n], self.free_pages[n:]
        return [p * self.page_size + o for p in pages for o in range(self.page_size)]

    def alloc_decode(self, seq_lens: Sequence[int], last_loc: Sequence[int]) -> list[int] | None:
        need = [1 if (int(s) - 1) % self.page_size == 0 else 0 for s in seq_lens]
        if sum(need) > len(self.free_pages):
            return None
        out, j = [], 0
        for s, ll, nd in zip(seq_lens, last_loc, need):
            if nd:
                out.append(self.free_pages[j] * self.page_size)
                j += 1
            else:
                out.append(int(ll) + 1)
        self.free_pages = self.free_pages[j:]
        return out

    def alloc_extend(self, prefix_lens: Sequence[int], seq_lens: Sequence[int],
                     last_loc: Sequence[int]) -> list[int] | None:
        ps = self.page_size
        need = sum((int(s) + ps - 1) // ps - (int(p) + ps - 1) // ps for p, s in zip(prefix_lens, seq_lens))
        if need > len(self.free_pages):
            return None
        out, j = [], 0
        for p, s, ll in zip(prefix_lens, seq_lens, last_loc):
            cur = int(ll)
            for t in range(int(p), int(s)):
                if t % ps == 0:
                    cur = self.free_pages[j] * ps
                    j += 1
                else:
                    cur += 1
                out.append(cur)
        self.free_pages = self.free_pages[j:]
        return out

    def free(self, slots: Sequence[int]) -> None:
        if len(slots) == 0:
            return
        pages = sorted({int(s) // self.page_size for s in slots})
        self.free_pages = pages + self.free_pages
