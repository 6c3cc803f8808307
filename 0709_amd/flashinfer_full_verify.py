"""Target-side tree construction and paged-KV helpers (drop-in for the
reference module ``atlas_0709.flashinfer_full_verify``).

Same names, keyword-only arguments, return types and exceptions as the
reference's tree / paged-KV functions.  Differences are in where the work runs:

* the ancestor mask is derived once on the host as one 64-bit bitmask per tree
  node (``TreeSpec.tree_mask``); the dense bool mask the reference builds with
  a Python double loop of single-element device writes
  (``flashinfer_full_verify.py:719-723``) is expanded from it with a handful
  of tensor ops, and the attention kernel consumes the bitmask directly;
* ``write_suffix_kv`` and ``prefix_layer_to_paged_kv`` write through the gfx950
  append kernel instead of ``index_put``.
"""

from __future__ import annotations

import threading
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np
import torch

from . import _lib, kv_ops
from .tree_attention import BatchPrefillWithPagedKVCacheWrapper, tensor_version


@dataclass(frozen=True)
class TreeSpec:
    """Reference ``TreeSpec`` (``flashinfer_full_verify.py:136-149``) plus the
    compact ancestor bitmask: ``tree_mask[i]`` has bit ``j`` set iff tree node
    ``j`` is an ancestor-or-self of node ``i``; tree node ``j`` sits at key
    position ``mask_col_start + j``.  ``packed_mask`` (the reference's
    ``packbits`` of ``bool_mask``) is built on first use: the verify passes
    ``bool_mask`` unless ``use_packed_custom_mask`` is set
    (``flashinfer_full_verify.py:963-967``)."""

    flat_token_ids: torch.Tensor
    parent_indices: list[int]
    depths: torch.Tensor
    bool_mask: torch.Tensor
    qo_indptr: torch.Tensor
    kv_indptr: torch.Tensor
    kv_indices: torch.Tensor
    kv_last_page_len: torch.Tensor
    total_pages: int
    node_count: int
    kv_len: int
    tree_mask: torch.Tensor | None = None
    mask_col_start: int = 0
    _packed: dict = field(default_factory=dict, repr=False, compare=False)

    @property
    def packed_mask(self) -> torch.Tensor:
        if "mask" not in self._packed:
            self._packed["mask"] = packbits(self.bool_mask)
        return self._packed["mask"]


@dataclass
class FullVerifyState:
    tree: TreeSpec
    paged_prefix_kv: list[torch.Tensor]


def ceil_div(value: int, divisor: int) -> int:
    return (int(value) + int(divisor) - 1) // int(divisor)


def last_page_len(length: int, page_size: int) -> int:
    rem = int(length) % int(page_size)
    return int(page_size) if rem == 0 else rem


def packbits(mask: torch.Tensor, bitorder: str = "big") -> torch.Tensor:
    """numpy.packbits semantics (FlashInfer's ``packbits`` default, big bit
    order) on the tensor's device."""
    if bitorder not in ("big", "little"):
        raise ValueError("bitorder must be 'big' or 'little'")
    flat = mask.reshape(-1).to(torch.uint8)
    pad = (-int(flat.numel())) % 8
    if pad:
        flat = torch.cat((flat, torch.zeros(pad, dtype=torch.uint8, device=flat.device)))
    shifts = torch.arange(8, dtype=torch.uint8, device=flat.device)
    if bitorder == "big":
        shifts = 7 - shifts
    return (flat.view(-1, 8) << shifts).sum(dim=1, dtype=torch.int32).to(torch.uint8)


def _validate_paths(paths: Sequence[Sequence[int]]) -> int:
    if not paths:
        raise ValueError("paths must not be empty")
    path_lengths = {len(path) for path in paths}
    if len(path_lengths) != 1:
        raise ValueError(f"all paths must have the same length, got {sorted(path_lengths)}")
    depth = next(iter(path_lengths))
    if depth <= 0:
        raise ValueError("paths must contain at least one token")
    return depth


def _path_tree_lists(paths: Sequence[Sequence[int]]) -> tuple[list[int], list[int], list[int]]:
    _validate_paths(paths)
    token_ids: list[int] = []
    parent_indices: list[int] = []
    depths: list[int] = []
    for path in paths:
        parent = -1
        for depth_idx, token_id in enumerate(path):
            token_ids.append(int(token_id))
            parent_indices.append(parent)
            depths.append(depth_idx)
            parent = len(token_ids) - 1
    return token_ids, parent_indices, depths


def build_path_tree_tokens_from_paths(
    paths: Sequence[Sequence[int]],
    *,
    device: torch.device | str,
) -> tuple[torch.Tensor, list[int], torch.Tensor]:
    """One node per path position, no sharing
    (``flashinfer_full_verify.py:541-567``)."""
    token_ids, parent_indices, depths = _path_tree_lists(paths)
    return (
        torch.tensor(token_ids, dtype=torch.long, device=device),
        parent_indices,
        torch.tensor(depths, dtype=torch.long, device=device),
    )


def _dedup_tree_lists(paths: Sequence[Sequence[int]]) -> tuple[list[int], list[int], list[int], list[list[int]]]:
    _validate_paths(paths)
    token_ids: list[int] = []
    parent_indices: list[int] = []
    depths: list[int] = []
    # children[(parent_node, token)] -> node; parent -1 is the root.
    children: dict[tuple[int, int], int] = {}
    route_nodes: list[list[int]] = []
    for path in paths:
        parent = -1
        nodes: list[int] = []
        for depth_idx, raw in enumerate(path):
            token = int(raw)
            node = children.get((parent, token))
            if node is None:
                node = len(token_ids)
                children[(parent, token)] = node
                token_ids.append(token)
                parent_indices.append(parent)
                depths.append(depth_idx)
            nodes.append(node)
            parent = node
        route_nodes.append(nodes)
    return token_ids, parent_indices, depths, route_nodes


def build_deduplicated_path_tree_tokens(
    paths: Sequence[Sequence[int]],
    *,
    device: torch.device | str,
) -> tuple[torch.Tensor, list[int], torch.Tensor, list[list[int]]]:
    """Prefix trie over the routes: one node per unique token prefix, numbered
    in insertion order (route by route, depth by depth), and the route -> node
    paths (``flashinfer_full_verify.py:570-616``)."""
    token_ids, parent_indices, depths, route_nodes = _dedup_tree_lists(paths)
    return (
        torch.tensor(token_ids, dtype=torch.long, device=device),
        parent_indices,
        torch.tensor(depths, dtype=torch.long, device=device),
        route_nodes,
    )


def ancestors_inclusive(node_idx: int, parent_indices: Sequence[int]) -> list[int]:
    out: list[int] = []
    cur = int(node_idx)
    while cur >= 0:
        out.append(cur)
        cur = int(parent_indices[cur])
    return out


def ancestor_bitmasks(parent_indices: Sequence[int]) -> list[int]:
    """bits[i] = OR of 1 << a over the ancestors-or-self a of node i.  Parents
    precede children in the trie numbering, so one forward pass suffices."""
    bits: list[int] = []
    for i, parent in enumerate(parent_indices):
        parent = int(parent)
        if parent >= i:
            # Arbitrary parent order: walk the chain.
            value = 0
            for a in ancestors_inclusive(i, parent_indices):
                value |= 1 << a
            bits.append(value)
        else:
            bits.append((bits[parent] if parent >= 0 else 0) | (1 << i))
    return bits


def _signed64(value: int) -> int:
    value &= (1 << 64) - 1
    return value - (1 << 64) if value >= 1 << 63 else value


def with_host_values(t: torch.Tensor, values: Sequence[int]) -> torch.Tensor:
    """Attach the host copy of a small index tensor's values (and its version
    counter), so a plan that reads them back skips the device-to-host copy
    while the tensor is unchanged.  An inference tensor has no counter, and a
    plan ignores the copy attached to it."""
    t._atlas_host_values = (list(values), tensor_version(t))
    return t


class _SpecScratch(threading.local):
    """Per-thread host buffers of the native tree builder, grown on demand
    (their contents are copied out before a build returns)."""

    def __init__(self):
        self.out = np.empty(0, dtype=np.uint8)
        self.parents = np.empty(0, dtype=np.int32)
        self.routes = np.empty(0, dtype=np.int32)
        self.info = np.zeros(8, dtype=np.int64)
        self.ptrs = (0, 0, 0, self.info.ctypes.data)

    def reserve(self, nbytes: int, nodes: int) -> None:
        if self.out.nbytes >= nbytes and self.parents.size >= nodes:
            return
        if self.out.nbytes < nbytes:
            self.out = np.empty(max(nbytes, 2 * self.out.nbytes), dtype=np.uint8)
        if self.parents.size < nodes:
            self.parents = np.empty(max(nodes, 2 * self.parents.size), dtype=np.int32)
            self.routes = np.empty_like(self.parents)
        self.ptrs = (self.out.ctypes.data, self.parents.ctypes.data, self.routes.ctypes.data, self.ptrs[3])


_SCRATCH = _SpecScratch()


def _native_tree_spec(paths, *, prefix_len: int, page_size: int, device, dedup: bool):
    """The spec of ``paths`` from the library's host builder
    (``atlas_tree_spec_build``: trie, ancestor sets, packed upload buffer in
    one call) and, for ``dedup``, the route -> node paths."""
    if isinstance(paths, (torch.Tensor, np.ndarray)):
        paths = paths.tolist()
    depth = _validate_paths(paths)
    arr = np.asarray(paths, dtype=np.int64)
    k = int(arr.shape[0])
    prefix_len, page_size = int(prefix_len), int(page_size)
    lib = _lib.load()
    need = lib.atlas_tree_spec_bytes(k, depth, prefix_len, page_size)
    if need < 0:
        raise ValueError(f"invalid tree shape: {k} paths of depth {depth}, prefix_len {prefix_len}, "
                         f"page_size {page_size}")
    sc = _SCRATCH
    sc.reserve(need, k * depth)
    out_p, par_p, rt_p, info_p = sc.ptrs
    rc = lib.atlas_tree_spec_build(arr.ctypes.data, k, depth, 1 if dedup else 0, prefix_len, page_size, out_p,
                                   sc.out.nbytes, par_p, rt_p, info_p)
    _lib.check(rc, "atlas_tree_spec_build")
    n, kv_len, total_pages, last, n_words, tiles, n32, nbytes = sc.info.tolist()
    parents = sc.parents[:n].tolist()
    route_nodes = sc.routes[: k * depth].reshape(k, depth).tolist() if dedup else None
    args = (sc.out[:nbytes], 2 * n + n_words, n32)
    kw = dict(node_count=n, kv_len=kv_len, total_pages=total_pages, last=last, prefix_len=prefix_len,
              compact=n <= 64, device=torch.device(device), parent_indices=parents,
              tile_shape=(n, tiles) if tiles else None)
    if not torch.is_inference_mode_enabled():
        return _tree_spec_tensors(*args, **kw), route_nodes
    # Normal tensors even under torch.inference_mode (the Target verify runs
    # in it): their version counters let a plan trust the attached host
    # values only while the tensors are unchanged.
    with torch.inference_mode(False):
        return _tree_spec_tensors(*args, **kw), route_nodes


_TRUE: dict = {}


def _true(device: torch.device) -> torch.Tensor:
    """A [1, 1] bool True on ``device`` (kept per device) to expand."""
    t = _TRUE.get(device)
    if t is None:
        t = _TRUE[device] = torch.ones((1, 1), dtype=torch.bool, device=device)
    return t


def _tree_spec_tensors(host, n64, n32, *, node_count, kv_len, total_pages, last, prefix_len, compact, device,
                       parent_indices, tile_shape=None) -> TreeSpec:
    """The spec's tensors as views of one device copy of ``host``: ``n64``
    int64 (token ids, depths, mask words), ``n32`` int32 (indptrs, last page
    length, page table, pad), then the n x n tree block of the mask."""
    dense = None
    if device.type == "cuda":
        # One allocation: the spec buffer, then the dense mask.  One launch
        # copies the spec from the pinned ring (mapped host memory) and fills
        # the mask (prefix columns visible, tree column j visible iff bit j of
        # the row's ancestor bitmask).
        nbytes = int(host.nbytes)
        head = (nbytes + 15) & ~15
        alloc = torch.empty(head + node_count * kv_len, dtype=torch.uint8, device=device)
        buf = alloc[:nbytes]
        dense = alloc[head:]
        lib, dst, mask, stream = _lib.load(), _lib.ptr(buf), _lib.ptr(dense), _lib.stream_of(device)

        def launch(src):
            _lib.check(lib.atlas_tree_spec_upload(src, nbytes, node_count, prefix_len, dst, mask, stream),
                       "atlas_tree_spec_upload")

        staging = _lib.staging()
        if not staging.stage(host, device, launch):
            # larger than the ring takes: a plain copy, then the mask from it
            staging.upload(host, device, out=buf)
            launch(dst)
    else:
        buf = torch.from_numpy(host.copy()).to(device)
    nb = 8 * node_count
    (tok_b, dep_b, words_b, qo_b, kvp_b, last_b, idx_b, _, block_b) = buf.split(
        [nb, nb, 8 * n64 - 2 * nb, 8, 8, 4, 4 * total_pages, 4 * n32 - 20 - 4 * total_pages,
         node_count * node_count])
    flat_token_ids = tok_b.view(torch.int64)
    depths_t = dep_b.view(torch.int64)
    tree_mask = words_b.view(torch.int64) if compact else None
    tile_words = words_b.view(torch.int64).view(tile_shape) if tile_shape else None
    qo_indptr = with_host_values(qo_b.view(torch.int32), [0, node_count])
    kv_indptr = with_host_values(kvp_b.view(torch.int32), [0, total_pages])
    kv_last = with_host_values(last_b.view(torch.int32), [last])
    kv_indices = idx_b.view(torch.int32)
    if dense is not None:
        flat_mask = dense.view(torch.bool)
    else:
        block_t = block_b.view(torch.bool).view(node_count, node_count)
        mask = torch.cat((_true(device).expand(node_count, prefix_len), block_t), dim=1) if prefix_len \
            else block_t.clone()
        flat_mask = mask.flatten()
    if tree_mask is not None:
        # Lets the attention plan skip re-deriving the bitmask from the mask.
        # The version counter lets plan() notice an in-place change of the mask.
        flat_mask._atlas_tree_window = (prefix_len, tree_mask, tensor_version(flat_mask))
    elif tile_words is not None:
        flat_mask._atlas_tree_tiles = (prefix_len, tile_words, tensor_version(flat_mask))
    return TreeSpec(
        flat_token_ids=flat_token_ids,
        parent_indices=list(parent_indices),
        depths=depths_t,
        bool_mask=flat_mask,
        qo_indptr=qo_indptr,
        kv_indptr=kv_indptr,
        kv_indices=kv_indices,
        kv_last_page_len=kv_last,
        total_pages=total_pages,
        node_count=node_count,
        kv_len=kv_len,
        tree_mask=tree_mask,
        mask_col_start=prefix_len,
    )


def build_tree_spec_from_paths(
    *,
    paths: Sequence[Sequence[int]],
    prefix_len: int,
    page_size: int,
    device: torch.device | str,
) -> TreeSpec:
    """Undeduplicated tree (``flashinfer_full_verify.py:655-701``)."""
    return _native_tree_spec(paths, prefix_len=prefix_len, page_size=page_size, device=device, dedup=False)[0]


def build_deduplicated_tree_spec_from_paths(
    *,
    paths: Sequence[Sequence[int]],
    prefix_len: int,
    page_size: int,
    device: torch.device | str,
) -> tuple[TreeSpec, list[list[int]]]:
    """Deduplicated tree and its route -> node paths
    (``flashinfer_full_verify.py:704-739``)."""
    return _native_tree_spec(paths, prefix_len=prefix_len, page_size=page_size, device=device, dedup=True)


def prefix_layer_to_paged_kv(
    *,
    key: torch.Tensor,
    value: torch.Tensor,
    prefix_len: int,
    node_count: int,
    page_size: int,
    total_pages: int | None = None,
    kv_layout: str = "NHD",
) -> torch.Tensor:
    """HF ``[1, Hkv, T, D]`` prefix K/V -> zero-initialised paged layer
    ``[pages, 2, page_size, Hkv, D]`` with token t at page t // page_size,
    offset t % page_size (``flashinfer_full_verify.py:814-849``);
    ``kv_layout="HND"`` lays the pages out ``[pages, 2, Hkv, page_size, D]``."""
    kv_ops.check_kv_layout(kv_layout)
    if key.shape[0] != 1 or value.shape[0] != 1:
        raise ValueError("full masked verify expects batch-1 prefix KV")
    if key.ndim != 4 or value.ndim != 4:
        raise ValueError(f"expected key/value shape [1, H, T, D], got {tuple(key.shape)} and {tuple(value.shape)}")
    _, kv_heads, key_len, head_dim = key.shape
    if int(key_len) != int(prefix_len):
        raise ValueError(f"prefix cache length mismatch: expected {prefix_len}, got {key_len}")
    if total_pages is None:
        total_pages = ceil_div(int(prefix_len) + int(node_count), int(page_size))
    page = (int(page_size), int(kv_heads)) if kv_layout == "NHD" else (int(kv_heads), int(page_size))
    kv_cache = torch.zeros(int(total_pages), 2, *page, int(head_dim), dtype=key.dtype, device=key.device)
    if int(prefix_len) > 0:
        key_tokens = key[0].permute(1, 0, 2).contiguous()
        value_tokens = value[0].permute(1, 0, 2).contiguous()
        kv_ops.append_paged([kv_cache], [key_tokens], [value_tokens], start_pos=0, kv_layout=kv_layout)
    return kv_cache


def write_suffix_kv(
    kv_cache: torch.Tensor,
    *,
    key_states: torch.Tensor,
    value_states: torch.Tensor,
    prefix_len: int,
    page_size: int,
    start_pos: int | None = None,
    kv_layout: str = "NHD",
) -> None:
    """Write node K/V ``[n, Hkv, D]`` at positions ``start + i`` of one paged
    layer (``flashinfer_full_verify.py:1027-1042``) of ``kv_layout`` pages."""
    cache_ps = int(kv_cache.shape[2 if kv_ops.check_kv_layout(kv_layout) == "NHD" else 3])
    if cache_ps != int(page_size):
        raise ValueError(f"page_size {page_size} does not match the cache's {cache_ps}")
    start = int(prefix_len) if start_pos is None else int(start_pos)
    node_count = int(key_states.shape[0])
    if start < 0 or start + node_count > int(kv_cache.shape[0]) * int(page_size):
        raise IndexError(
            f"positions [{start}, {start + node_count}) exceed the cache's "
            f"{int(kv_cache.shape[0]) * int(page_size)} slots"
        )
    kv_ops.append_paged([kv_cache], [key_states], [value_states], start_pos=start, kv_layout=kv_layout)


def first_tensor(value) -> torch.Tensor:
    if isinstance(value, torch.Tensor):
        return value
    if isinstance(value, (tuple, list)):
        for item in value:
            if isinstance(item, torch.Tensor):
                return item
    raise TypeError(f"expected tensor output, got {type(value).__name__}")


from .decode_attention import make_decode_wrapper, plan_decode_wrapper  # noqa: E402  (decode wrapper helpers)


def make_prefill_wrapper(*, args, flashinfer=None, kv_layout: str | None = None) -> BatchPrefillWithPagedKVCacheWrapper:
    """Workspace-backed wrapper (``flashinfer_full_verify.py:877-879``) for
    ``kv_layout`` pages (default: ``args.kv_layout`` when set, else NHD, the
    reference's)."""
    workspace = torch.empty(int(args.workspace_mb) * 1024 * 1024, dtype=torch.uint8, device=args.device)
    layout = kv_layout or getattr(args, "kv_layout", None) or "NHD"
    return BatchPrefillWithPagedKVCacheWrapper(workspace, layout, backend=getattr(args, "flashinfer_backend", "auto"))


def plan_prefill_wrapper(wrapper, tree: TreeSpec, *, args, config, dtype: torch.dtype) -> None:
    """Masked, non-causal plan with the reference's keyword retry ladder
    (``flashinfer_full_verify.py:953-985``)."""
    head_dim = getattr(config, "head_dim", int(config.hidden_size) // int(config.num_attention_heads))
    attempts = [
        {"q_data_type": dtype, "kv_data_type": dtype},
        {"q_data_type": str(dtype).replace("torch.", ""), "kv_data_type": str(dtype).replace("torch.", "")},
        {},
    ]
    last_error: Exception | None = None
    for kwargs in attempts:
        try:
            mask_kwargs = (
                {"packed_custom_mask": tree.packed_mask}
                if getattr(args, "use_packed_custom_mask", False)
                else {"custom_mask": tree.bool_mask}
            )
            wrapper.plan(
                tree.qo_indptr,
                tree.kv_indptr,
                tree.kv_indices,
                tree.kv_last_page_len,
                int(config.num_attention_heads),
                int(config.num_key_value_heads),
                int(head_dim),
                int(args.page_size),
                causal=False,
                pos_encoding_mode="NONE",
                **mask_kwargs,
                **kwargs,
            )
            return
        except (AttributeError, TypeError) as exc:
            last_error = exc
    raise RuntimeError(f"BatchPrefillWithPagedKVCacheWrapper.plan failed: {last_error!r}")
