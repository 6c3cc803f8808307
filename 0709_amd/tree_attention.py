"""Ancestor-masked paged tree / forest verify attention (FlashInfer-shaped API).

``BatchPrefillWithPagedKVCacheWrapper`` keeps the plan/run protocol the
reference drives (``flashinfer_full_verify.py:877-879``, ``:953-985``,
``:1223``): ``plan`` receives the page-table metadata, head counts, page size,
``causal`` and ``custom_mask`` / ``packed_custom_mask``; ``run(q, kv_cache)``
returns ``[nnz, Hq, D]`` (optionally with the LSE).  ``plan`` does the host
work once per verify (the reference re-plans per verify and runs per layer):
it reads the index arrays, derives a per-query 64-bit ancestor bitmask for the
tree columns, splits every (request, KV head, row block) along its keys so a
launch fills the 256 CUs, and uploads the work list in one copy.  ``run`` is a
single kernel launch (plus a merge launch when rows are split).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib

TILE_KEYS = 64
MAX_ROWS_PER_ITEM = 256  # 8 waves x 2 row tiles of 16 (head_dim 128, pages of >= 16 tokens)
MAX_ROWS_PER_ITEM_OTHER = 192  # 4 waves x 3 row tiles of 16 (other shapes)
DEFAULT_ROWS_PER_ITEM = 64  # 4 waves x 1 row tile
MAX_TREE_WIDTH = 64  # tree columns one ancestor word per row covers
MAX_WIDE_TREE_WIDTH = 4096  # tree columns of the per-tile word layout
MAX_SPLITS = 1024
DEFAULT_CU_COUNT = 256


def _partial_row_bytes(head_dim: int) -> int:
    """Workspace bytes of one split partial row: the normalised O in the output
    dtype (16-bit) and its fp32 base-2 LSE."""
    return 2 * head_dim + 4


@dataclass
class AttentionPlan:
    batch: int
    num_qo_heads: int
    num_kv_heads: int
    head_dim: int
    page_size: int
    sm_scale: float
    q_dtype: torch.dtype
    kv_dtype: torch.dtype
    nnz: int
    mask_mode: int
    qo_indptr: torch.Tensor
    kv_indptr: torch.Tensor
    kv_indices: torch.Tensor
    tree_mask: torch.Tensor | None
    meta: torch.Tensor  # int32: [work | merge | kv_len | mask_col_start]
    num_work: int
    num_merge: int
    work_offset: int
    merge_offset: int
    kv_len_offset: int
    col_offset: int
    max_rows: int
    partial_rows: int
    kv_lens: list[int]
    qo_lens: list[int]
    tiles_per_split: int  # most key tiles any work item streams
    page_windows: torch.Tensor | None = None  # int32 [num_work * 64]: first page ids of each item
    # run(append_key_states=...) can write the newest rows inside the launch:
    # head_dim-128 kernel, one row block per (request, KV head)
    fused_append: bool = False
    # tree mask words per query row (1: one ancestor word; more: one word per
    # 64-key tile of the tree region, for trees wider than 64 columns)
    mask_words: int = 1

    def device_view(self, offset: int) -> int:
        return int(self.meta.data_ptr()) + 4 * offset


def tensor_version(t: torch.Tensor) -> int | None:
    """The tensor's in-place version counter, or None for an inference tensor
    (created under torch.inference_mode, which keeps no counter)."""
    try:
        return t._version
    except RuntimeError:
        return None


def _cached_host_values(t: torch.Tensor) -> list[int] | None:
    """The host copy a tree builder attached to a small index tensor, if the
    tensor has not been modified in place since (version counter unchanged).
    An inference tensor keeps no counter, so its copy cannot be trusted and
    its values are read back."""
    cached = getattr(t, "_atlas_host_values", None)
    if cached is None:
        return None
    values, version = cached
    if version is None or version != tensor_version(t) or len(values) != int(t.numel()):
        return None
    return values


def _host_lists(*items: torch.Tensor | list | tuple) -> list[list[int]]:
    """Host int lists of index arrays: lists and CPU tensors directly, device
    tensors from their attached host copy when valid, the rest with one
    device-to-host copy for all of them."""
    out: list[list[int] | None] = []
    pending: list[tuple[int, torch.Tensor]] = []
    for i, t in enumerate(items):
        if not isinstance(t, torch.Tensor):
            out.append([int(x) for x in t])
        elif t.device.type == "cpu":
            out.append([int(x) for x in t.reshape(-1).tolist()])
        else:
            cached = _cached_host_values(t)
            out.append(cached)
            if cached is None:
                pending.append((i, t.detach().reshape(-1)))
    if pending:
        flat = torch.cat([t.to(torch.int64) for _, t in pending]).cpu().tolist()
        off = 0
        for i, t in pending:
            n = int(t.numel())
            out[i] = [int(x) for x in flat[off:off + n]]
            off += n
    return out  # type: ignore[return-value]


def _dtype_from(value, default: torch.dtype) -> torch.dtype:
    if value is None:
        return default
    if isinstance(value, torch.dtype):
        return value
    name = str(value).replace("torch.", "")
    table = {"float16": torch.float16, "half": torch.float16, "bfloat16": torch.bfloat16}
    if name not in table:
        raise TypeError(f"unsupported data type {value!r}")
    return table[name]


def tree_mask_from_dense(mask2d: torch.Tensor) -> tuple[int, torch.Tensor] | None:
    """(col0, bits) such that columns < col0 are visible to every row and row
    q sees column col0 + j iff bit j of bits[q]; None if no window of at most
    64 columns describes the mask."""
    qo, kv = (int(x) for x in mask2d.shape)
    if qo == 0:
        return kv, torch.zeros(0, dtype=torch.int64, device=mask2d.device)
    m = mask2d.to(torch.bool)
    all_true = m.all(dim=0)
    # col0 = first column that is not visible to every row.
    false_cols = torch.nonzero(~all_true)
    col0 = kv if false_cols.numel() == 0 else int(false_cols[0])
    if kv - col0 > MAX_TREE_WIDTH:
        return None
    window = m[:, col0:kv].to(torch.int64)
    shifts = torch.arange(kv - col0, device=m.device, dtype=torch.int64)
    bits = (window << shifts).sum(dim=1) if kv > col0 else torch.zeros(qo, dtype=torch.int64, device=m.device)
    return col0, bits


def tree_tile_words_from_dense(mask2d: torch.Tensor, max_width: int = MAX_WIDE_TREE_WIDTH):
    """(col0, words) of a wide tree mask: col0 as for ``tree_mask_from_dense``
    and, per query row, one visibility word per 64-key tile from the tile
    holding col0 to the last key (bit b of word j: key 64 (col0 // 64 + j) +
    b; columns below col0 are visible); None when the non-visible region
    spans more than ``max_width`` columns."""
    qo, kv = (int(x) for x in mask2d.shape)
    m = mask2d.to(torch.bool)
    false_cols = torch.nonzero(~m.all(dim=0)) if qo else torch.zeros((0, 1), dtype=torch.long)
    col0 = kv if false_cols.numel() == 0 else int(false_cols[0])
    if kv - col0 > max_width:
        return None
    t0 = col0 // 64
    ntiles = max(0, (kv - 1) // 64 - t0 + 1) if kv else 0
    window = torch.zeros((qo, ntiles * 64), dtype=torch.int64, device=m.device)
    if ntiles:
        window[:, : kv - t0 * 64] = m[:, t0 * 64 : kv].to(torch.int64)
    shifts = torch.arange(64, device=m.device, dtype=torch.int64)
    words = (window.view(qo, ntiles, 64) << shifts).sum(dim=2)
    return col0, words


def _cached_tree_window(custom_mask, qo_lens: list[int], kv_lens: list[int]):
    """The (col0, bits) window the tree builder attached to a single-request
    dense mask, if it still describes this plan: one request, one ancestor
    word per query row, col0 within the keys and at most 64 tree columns, and
    the mask not modified in place since (its version counter unchanged; an
    inference tensor keeps no counter, so its window is not trusted).
    Otherwise None, and the plan derives the window from the mask itself."""
    cached = getattr(custom_mask, "_atlas_tree_window", None) if custom_mask is not None else None
    if cached is None or len(qo_lens) != 1 or len(cached) != 3:
        return None
    col0, bits, version = cached
    if version is None or version != tensor_version(custom_mask) or \
            int(custom_mask.numel()) != qo_lens[0] * kv_lens[0]:
        return None
    if int(bits.numel()) != qo_lens[0] or not (0 <= int(col0) <= kv_lens[0]):
        return None
    if kv_lens[0] - int(col0) > MAX_TREE_WIDTH:
        return None
    return int(col0), bits


def _cached_tree_tiles(custom_mask, qo_lens: list[int], kv_lens: list[int]):
    """The per-tile words (``tree_tile_words_from_dense``) the tree builder
    attached to a single-request dense mask of a wide tree, if they still
    describe this plan and the mask is unchanged since (version counter);
    otherwise None."""
    cached = getattr(custom_mask, "_atlas_tree_tiles", None) if custom_mask is not None else None
    if cached is None or len(qo_lens) != 1 or len(cached) != 3:
        return None
    col0, words, version = cached
    if version is None or version != tensor_version(custom_mask) or \
            int(custom_mask.numel()) != qo_lens[0] * kv_lens[0]:
        return None
    ntiles = max(0, (kv_lens[0] - 1) // 64 - int(col0) // 64 + 1) if kv_lens[0] else 0
    if words.ndim != 2 or int(words.shape[0]) != qo_lens[0] or int(words.shape[1]) != ntiles:
        return None
    if not (0 <= int(col0) <= kv_lens[0]) or kv_lens[0] - int(col0) > MAX_WIDE_TREE_WIDTH:
        return None
    return int(col0), words


def unpack_bits_little(packed: torch.Tensor, count: int) -> torch.Tensor:
    """Inverse of a little-bit-order packbits over ``count`` booleans."""
    b = packed.to(torch.uint8).reshape(-1).to(torch.int32)
    bits = (b[:, None] >> torch.arange(8, device=b.device, dtype=torch.int32)) & 1
    return bits.reshape(-1)[:count].to(torch.bool)


def _rope_table(t: torch.Tensor, name: str, plan: AttentionPlan, dtype: torch.dtype) -> torch.Tensor:
    """A rotary cos or sin table as [rows, D] with contiguous, 16-byte aligned rows."""
    if t.shape[-1] != plan.head_dim or t.stride(-1) != 1:
        raise ValueError(f"rope {name} rows must be contiguous [.., {plan.head_dim}], got {tuple(t.shape)}")
    t = t.reshape(-1, plan.head_dim)
    if int(t.shape[0]) < plan.nnz:
        raise ValueError(f"rope {name} has {int(t.shape[0])} rows for {plan.nnz} query tokens")
    if t.dtype != dtype:
        raise TypeError(f"rope {name} must have q's dtype {dtype}, got {t.dtype}")
    if t.stride(0) % 8 != 0 or int(t.data_ptr()) % 16 != 0:
        t = t.contiguous()
    return t


def pack_plan(*, work, merge, partial_rows, max_rows, direct, fused_append, kv_lens, cols, qo, kvp) -> dict:
    """A planned work list as the kernels read it: one int32 array of [work
    items (16 ints) | merge items (8 ints) | kv_len | mask_col_start |
    qo_indptr | kv_indptr] and the offsets of its parts.  ``fused_append``:
    every (request, KV head) is a single row block (the launch may write the
    newest rows itself)."""
    meta_vals: list[int] = []
    for item in work:
        meta_vals.extend(item)
    merge_off = len(meta_vals)
    for item in merge:
        meta_vals.extend(item)
    kvlen_off = len(meta_vals)
    meta_vals.extend(kv_lens)
    col_off = len(meta_vals)
    meta_vals.extend(cols)
    qo_off = len(meta_vals)
    meta_vals.extend(qo)
    kvp_off = len(meta_vals)
    meta_vals.extend(kvp)
    return dict(
        work=work, num_merge=len(merge), partial_rows=partial_rows, max_rows=max_rows, direct=direct,
        fused_append=fused_append, meta=np.asarray(meta_vals, dtype=np.int32), merge_off=merge_off,
        kvlen_off=kvlen_off, col_off=col_off, qo_off=qo_off, kvp_off=kvp_off, qo=qo, kvp=kvp,
        tiles_per_split=max((math.ceil((it[5] - it[4]) / TILE_KEYS) for it in work), default=0))


class BatchPrefillWithPagedKVCacheWrapper:
    """Paged prefill attention with a custom (tree) mask on the gfx950 kernel.

    ``float_workspace_buffer`` holds the split-KV partial states (like
    FlashInfer's workspace: the partial O in the output dtype and an fp32 LSE
    per row); its size bounds how finely keys are split.
    """

    def __init__(
        self,
        float_workspace_buffer: torch.Tensor,
        kv_layout: str = "NHD",
        backend: str = "auto",
        **_unused,
    ) -> None:
        if kv_layout not in ("NHD", "HND"):
            raise NotImplementedError(f"paged layout {kv_layout!r}: NHD and HND are supported")
        self._workspace = float_workspace_buffer
        self._kv_layout = kv_layout
        self._backend = backend
        self._plan: AttentionPlan | None = None
        # None: chosen per plan (see plan())
        self.split_target_items: int | None = None
        # Plan-time page-id windows for the head_dim-128 kernel (off: the
        # kernel reads them from the page table after its work item).
        self.use_page_windows: bool = True
        self.min_tiles_per_split = 1
        self.max_rows_per_item: int | None = None
        # Key granule of the split boundaries (None: whole 64-key tiles).  The
        # head_dim-128 kernel accepts splits starting at any multiple of
        # min(page_size, 64) keys; other shapes always split at whole tiles.
        self.split_granule_keys: int | None = None
        self._decomp_cache: tuple | None = None
        self._meta_uploaded: tuple | None = None
        self._plan_cache: tuple | None = None
        self._meta_buf: torch.Tensor | None = None
        self._indices_buf: torch.Tensor | None = None
        self._bits_buf: torch.Tensor | None = None

    @property
    def device(self) -> torch.device:
        return self._workspace.device

    # ------------------------------------------------------------------ plan
    def plan(
        self,
        qo_indptr: torch.Tensor,
        paged_kv_indptr: torch.Tensor,
        paged_kv_indices: torch.Tensor,
        paged_kv_last_page_len: torch.Tensor,
        num_qo_heads: int,
        num_kv_heads: int,
        head_dim_qk: int,
        page_size: int,
        head_dim_vo: int | None = None,
        custom_mask: torch.Tensor | None = None,
        packed_custom_mask: torch.Tensor | None = None,
        causal: bool = False,
        pos_encoding_mode: str = "NONE",
        use_fp16_qk_reduction: bool = False,
        sm_scale: float | None = None,
        window_left: int = -1,
        logits_soft_cap: float | None = None,
        rope_scale: float | None = None,
        rope_theta: float | None = None,
        q_data_type=torch.float16,
        kv_data_type=None,
        non_blocking: bool = True,
    ) -> None:
        device = self.device
        _lib.require_device(self._workspace, what="BatchPrefillWithPagedKVCacheWrapper")
        if pos_encoding_mode != "NONE":
            raise NotImplementedError("only pos_encoding_mode='NONE' is supported (RoPE is applied by the caller)")
        if head_dim_vo is not None and int(head_dim_vo) != int(head_dim_qk):
            raise NotImplementedError("head_dim_vo must equal head_dim_qk")
        if window_left != -1 or logits_soft_cap not in (None, 0.0):
            raise NotImplementedError("sliding windows and logit soft-capping are not supported")
        hq, hkv, d, ps = int(num_qo_heads), int(num_kv_heads), int(head_dim_qk), int(page_size)
        if hq <= 0 or hkv <= 0 or hq % hkv != 0:
            raise ValueError("num_qo_heads must be a positive multiple of num_kv_heads")
        if d not in (64, 128):
            raise NotImplementedError(f"head_dim {d} is not supported (64 or 128)")
        if ps <= 0:
            raise ValueError("page_size must be positive")
        q_dtype = _dtype_from(q_data_type, torch.float16)
        kv_dtype = _dtype_from(kv_data_type, q_dtype)
        if q_dtype != kv_dtype:
            raise NotImplementedError("q and kv data types must match")

        qo, kvp, last = _host_lists(qo_indptr, paged_kv_indptr, paged_kv_last_page_len)
        batch = len(qo) - 1
        if batch <= 0 or len(kvp) != batch + 1 or len(last) != batch:
            raise ValueError("qo_indptr / kv_indptr / kv_last_page_len sizes are inconsistent")
        qo_lens = [qo[b + 1] - qo[b] for b in range(batch)]
        pages = [kvp[b + 1] - kvp[b] for b in range(batch)]
        if any(x < 0 for x in qo_lens) or any(x < 0 for x in pages):
            raise ValueError("indptr arrays must be non-decreasing")
        kv_lens = [0 if pages[b] == 0 else (pages[b] - 1) * ps + last[b] for b in range(batch)]
        for b in range(batch):
            if pages[b] and not (1 <= last[b] <= ps):
                raise ValueError(f"kv_last_page_len[{b}]={last[b]} outside [1, page_size]")

        # ---- mask ----
        mask_mode = _lib.MASK_CAUSAL if causal else _lib.MASK_NONE
        tree_bits = None
        mask_words = 1
        cols = [0] * batch
        if custom_mask is not None or packed_custom_mask is not None:
            if causal:
                raise ValueError("custom masks require causal=False")
            mask_mode = _lib.MASK_TREE
            cached = _cached_tree_window(custom_mask, qo_lens, kv_lens)
            cached_tiles = None if cached is not None else _cached_tree_tiles(custom_mask, qo_lens, kv_lens)
            if cached is not None:
                col0, bits = cached
                cols = [int(col0)]
                tree_bits = bits.to(device=device, dtype=torch.int64)
            elif cached_tiles is not None:
                col0, words = cached_tiles
                cols = [int(col0)]
                mask_words = max(1, int(words.shape[1]))
                tree_bits = words.to(device=device, dtype=torch.int64)
                if mask_words == 1:
                    # a one-tile window still uses the per-tile layout (two words)
                    mask_words = 2
                    tree_bits = torch.cat((tree_bits, torch.zeros_like(tree_bits)), dim=1)
                tree_bits = tree_bits.reshape(-1)
            else:
                total = sum(qo_lens[b] * kv_lens[b] for b in range(batch))
                if custom_mask is not None:
                    flat = custom_mask.reshape(-1).to(device=device, dtype=torch.bool)
                else:
                    flat = self._unpack_segments(packed_custom_mask.to(device), qo_lens, kv_lens)
                if int(flat.numel()) != total:
                    raise ValueError(f"custom mask has {int(flat.numel())} entries, expected {total}")
                parts = []
                segs = []
                off = 0
                for b in range(batch):
                    seg = flat[off : off + qo_lens[b] * kv_lens[b]].view(qo_lens[b], kv_lens[b])
                    off += qo_lens[b] * kv_lens[b]
                    segs.append(seg)
                    res = tree_mask_from_dense(seg) if parts is not None else None
                    if res is None:
                        parts = None  # some request is wide: every request takes the per-tile layout
                        continue
                    cols[b] = res[0]
                    parts.append(res[1])
                if parts is not None:
                    tree_bits = torch.cat(parts) if parts else torch.zeros(0, dtype=torch.int64, device=device)
                else:
                    # a tree wider than 64 columns: one word per 64-key tile
                    # of every request's tree region
                    tiles = []
                    for b, seg in enumerate(segs):
                        res = tree_tile_words_from_dense(seg)
                        if res is None:
                            raise NotImplementedError(
                                f"request {b}: the mask's non-visible region spans more than "
                                f"{MAX_WIDE_TREE_WIDTH} key columns; only prefix + tree masks are supported"
                            )
                        cols[b] = res[0]
                        tiles.append(res[1])
                    mask_words = max(2, max(int(t.shape[1]) for t in tiles))
                    tree_bits = torch.cat([torch.nn.functional.pad(t, (0, mask_words - int(t.shape[1])))
                                           for t in tiles]).reshape(-1)

        # ---- work decomposition (the same inputs give the same work list) ----
        ws_rows_cap = self._workspace.numel() * self._workspace.element_size() // _partial_row_bytes(d)
        key = (tuple(qo), tuple(kvp), tuple(kv_lens), tuple(cols), hq, hkv, d, ps, self.max_rows_per_item,
               self.split_target_items, self.min_tiles_per_split, self.split_granule_keys, ws_rows_cap, mask_words)
        if self._decomp_cache is None or self._decomp_cache[0] != key:
            self._decomp_cache = (key, self._decompose(batch=batch, qo=qo, kvp=kvp, qo_lens=qo_lens,
                                                       kv_lens=kv_lens, cols=cols, hq=hq, hkv=hkv, d=d, ps=ps,
                                                       ws_rows_cap=ws_rows_cap, whole_tiles=mask_words > 1))
        dec = self._decomp_cache[1]
        self._install(
            batch=batch, hq=hq, hkv=hkv, d=d, ps=ps, sm_scale=sm_scale, q_dtype=q_dtype, kv_dtype=kv_dtype,
            mask_mode=mask_mode, dec=dec, kv_lens=kv_lens, qo_lens=qo_lens,
            indices_src=paged_kv_indices.reshape(-1), tree_bits=tree_bits, mask_words=mask_words,
            non_blocking=non_blocking)

    def _decompose(self, *, batch, qo, kvp, qo_lens, kv_lens, cols, hq, hkv, d, ps, ws_rows_cap,
                   whole_tiles=False) -> dict:
        """Work and merge items of a plan, and the int32 metadata the kernels
        read: [work items | merge items | kv_len | mask_col_start | qo_indptr |
        kv_indptr]."""
        group = hq // hkv
        direct = d == 128 and ps >= 16 and (ps & (ps - 1)) == 0
        if self.max_rows_per_item is None:
            # head_dim-128 kernel: up to 160 rows (10 row tiles: two per wave on
            # waves 0..3, leftovers split by keys over waves 4..7) in one block,
            # so the keys are streamed once; more rows split into equal blocks.
            rows_max = max((qo_lens[b] * (hq // hkv) for b in range(batch)), default=1)
            cap = 160 if direct else DEFAULT_ROWS_PER_ITEM
            nblk = max(1, math.ceil(rows_max / cap))
            row_block = 16 * math.ceil(math.ceil(rows_max / nblk) / 16)
        else:
            row_block = int(self.max_rows_per_item)
        row_block = max(16, min(MAX_ROWS_PER_ITEM if direct else MAX_ROWS_PER_ITEM_OTHER, row_block))
        split_target = self.split_target_items
        if split_target is None:
            # One 8-wave workgroup per CU for the head_dim-128 kernel, leaving a
            # sixteenth of the CUs free (the previous launch's tail still holds
            # some; measured 27.2-27.4 us/layer at 232-240 items against 28.3 at
            # 256 on the forest headline); a batch of unequal requests gets two
            # items per CU, dispatched longest first.
            split_target = DEFAULT_CU_COUNT * 15 // 16 if (direct and batch == 1) else 2 * DEFAULT_CU_COUNT
        blocks = []  # (req, row_start, num_rows)
        for b in range(batch):
            rows = qo_lens[b] * group
            nblk = max(1, math.ceil(rows / row_block))
            # equal-sized blocks, each a multiple of 16 rows where possible
            size = min(row_block, 16 * math.ceil(math.ceil(rows / nblk) / 16)) if rows else 0
            for r0 in range(0, rows, max(size, 1)):
                blocks.append((b, r0, min(size, rows - r0)))
            if rows == 0:
                blocks.append((b, 0, 0))
        gran = TILE_KEYS
        # (wide tree masks are read per 64-key tile: their splits start on tiles)
        if direct and self.split_granule_keys is not None and not whole_tiles:
            gran = int(self.split_granule_keys)
            if gran <= 0 or gran > TILE_KEYS or gran % min(ps, TILE_KEYS) != 0 or TILE_KEYS % gran != 0:
                raise ValueError(f"split_granule_keys must divide {TILE_KEYS} and be a multiple of "
                                 f"min(page_size, {TILE_KEYS}) = {min(ps, TILE_KEYS)}, got {gran}")
        unit_tiles = sum(hkv * math.ceil(kv_lens[b] / TILE_KEYS) for (b, _, _) in blocks)
        # Tiles per split as a fraction, so the split count per request rounds
        # down and the items do not exceed the target (one per CU when a single
        # request fills the device).
        tiles_per_split = max(float(self.min_tiles_per_split), unit_tiles / max(1, split_target))
        # the merge kernel combines at most MAX_SPLITS states per row
        max_tiles = max((math.ceil(kv_lens[b] / TILE_KEYS) for (b, _, _) in blocks), default=0)
        tiles_per_split = max(tiles_per_split, max_tiles / MAX_SPLITS)
        while True:
            work, merge = [], []
            partial_rows = 0
            for (b, r0, nr) in blocks:
                tiles = math.ceil(kv_lens[b] / TILE_KEYS)
                splits = max(1, min(tiles, int(tiles / tiles_per_split + 1e-9)))
                # balanced splits of the request's key granules: `per` granules
                # each, one more for the first `extra` splits, so the last
                # split, which holds the request's masked tail tile (the
                # costliest to compute), has one granule less
                units = math.ceil(kv_lens[b] / gran)
                per = units // splits if units else 0
                extra = units - per * splits
                # request values every item repeats (qo_start, qo_len, kv_len,
                # mask column start, page offset) and padding to 16 ints
                req_vals = (qo[b], qo_lens[b], kv_lens[b], cols[b], kvp[b], 0, 0, 0, 0)
                for h in range(hkv):
                    if splits == 1:
                        work.append((b, h, r0, nr, 0, kv_lens[b], -1) + req_vals)
                        continue
                    base = partial_rows
                    for s in range(splits):
                        t0 = s * per + min(s, extra)
                        t1 = t0 + per + (1 if s < extra else 0)
                        k0 = t0 * gran
                        k1 = min(kv_lens[b], t1 * gran)
                        work.append((b, h, r0, nr, k0, k1, base + s * nr) + req_vals)
                    merge.append((b, h, r0, nr, base, splits, 0, 0))
                    partial_rows += splits * nr
            if partial_rows <= ws_rows_cap:
                break
            tiles_per_split *= 2
        max_rows = max((nr for (_, _, nr) in blocks), default=1)
        # Largest items first: workgroups are dispatched in order, so the
        # long ones start early and the short ones fill in behind them.  Equal
        # items cycle through the KV heads, so with workgroups spread over the
        # 8 XCDs round-robin each KV head's splits share one XCD's L2 (and
        # their queries) when there are 8 KV heads.
        work.sort(key=lambda it: (-(it[5] - it[4]), it[0], it[2], it[4], it[1]))

        return pack_plan(work=work, merge=merge, partial_rows=partial_rows, max_rows=max_rows, direct=direct,
                         fused_append=direct and all(r0 == 0 for (_, r0, _) in blocks), kv_lens=kv_lens,
                         cols=cols, qo=qo, kvp=kvp)

    def _install(self, *, batch, hq, hkv, d, ps, sm_scale, q_dtype, kv_dtype, mask_mode, dec, kv_lens, qo_lens,
                 indices_src, tree_bits, non_blocking, mask_words=1) -> None:
        """Write a planned work list (``dec``, from ``_decompose``) into the
        persistent device buffers and make it the current plan."""
        device = self.device
        meta_np = dec["meta"]
        # Persistent device buffers keep their addresses across plans, so a
        # HIP graph captured over run() stays valid after a re-plan of the
        # same (or a smaller) shape.  Metadata equal to what the buffer already
        # holds is not uploaded again.
        meta = self._persistent("_meta_buf", len(meta_np), torch.int32)
        if self._meta_uploaded is None or self._meta_uploaded[0] is not meta or \
                (self._meta_uploaded[1] is not meta_np and not np.array_equal(self._meta_uploaded[1], meta_np)):
            if device.type == "cuda":
                _lib.staging().upload(meta_np, device, out=meta[: len(meta_np)])
            else:
                meta[: len(meta_np)].copy_(torch.from_numpy(meta_np))
            self._meta_uploaded = (meta, meta_np)
        work = dec["work"]
        n_idx = int(indices_src.numel())
        indices = self._persistent("_indices_buf", n_idx, torch.int32)
        src_idx = indices_src
        if src_idx.dtype != torch.int32 or src_idx.device != device or not src_idx.is_contiguous():
            src_idx = src_idx.to(device=device, dtype=torch.int32).contiguous()
        bits_buf = src_bits = None
        nb = 0
        if tree_bits is not None:
            nb = int(tree_bits.numel())
            bits_buf = self._persistent("_bits_buf", nb, torch.int64)
            src_bits = tree_bits.to(device=device, dtype=torch.int64).contiguous()
        # The page table and mask words go into the plan's own buffers, and
        # the first page-id window of every work item is gathered (the page
        # table is fixed until the next plan, so the head_dim-128 kernel
        # requests its first page ids with its work item): one launch.
        windows = None
        if dec["direct"] and work and self.use_page_windows:
            windows = self._persistent("_windows_buf", 64 * len(work), torch.int32)
        rc = _lib.load().atlas_attn_plan_install(
            int(meta.data_ptr()), len(work) if windows is not None else 0, _lib.ptr(src_idx), n_idx,
            _lib.ptr(indices), _lib.ptr(src_bits), nb, _lib.ptr(bits_buf), ps, _lib.ptr(windows),
            _lib.stream_of(device))
        _lib.check(rc, "atlas_attn_plan_install")

        # The same work list over the same buffers and arguments is the same
        # plan object (kv_lens and qo_lens are part of the work list's key).
        plan_key = (dec, meta, indices, bits_buf, windows, sm_scale, q_dtype, kv_dtype, mask_mode, mask_words,
                    batch, hq, hkv, d, ps)
        cached = self._plan_cache
        if cached is not None and len(cached[0]) == len(plan_key) and \
                all(a is b or (type(a) in (int, float, str) and a == b) for a, b in zip(cached[0], plan_key)):
            self._plan = cached[1]
            return
        self._plan = AttentionPlan(
            batch=batch, num_qo_heads=hq, num_kv_heads=hkv, head_dim=d, page_size=ps,
            sm_scale=float(sm_scale) if sm_scale is not None else 1.0 / math.sqrt(d),
            q_dtype=q_dtype, kv_dtype=kv_dtype, nnz=dec["qo"][-1] - dec["qo"][0] if batch else 0,
            mask_mode=mask_mode, qo_indptr=meta[dec["qo_off"]:], kv_indptr=meta[dec["kvp_off"]:],
            kv_indices=indices, tree_mask=bits_buf, mask_words=int(mask_words), meta=meta, num_work=len(work),
            num_merge=dec["num_merge"],
            work_offset=0, merge_offset=dec["merge_off"], kv_len_offset=dec["kvlen_off"],
            col_offset=dec["col_off"], max_rows=dec["max_rows"], partial_rows=dec["partial_rows"],
            kv_lens=kv_lens, qo_lens=qo_lens, tiles_per_split=dec["tiles_per_split"], page_windows=windows,
            fused_append=dec["fused_append"],
        )
        self._plan_cache = (plan_key, self._plan)

    @property
    def kv_layout(self) -> str:
        """The paged layout run() reads: "NHD" or "HND"."""
        return self._kv_layout

    def _persistent(self, name: str, count: int, dtype: torch.dtype) -> torch.Tensor:
        buf = getattr(self, name, None)
        if buf is None or int(buf.numel()) < count or buf.dtype != dtype:
            buf = torch.empty(max(count, 1024), dtype=dtype, device=self.device)
            setattr(self, name, buf)
        return buf

    @staticmethod
    def _unpack_segments(packed: torch.Tensor, qo_lens: list[int], kv_lens: list[int]) -> torch.Tensor:
        # Each request's segment is packed separately and padded to whole bytes.
        parts = []
        byte_off = 0
        for ql, kl in zip(qo_lens, kv_lens):
            count = ql * kl
            nbytes = (count + 7) // 8
            parts.append(unpack_bits_little(packed[byte_off : byte_off + nbytes], count))
            byte_off += nbytes
        return torch.cat(parts) if parts else torch.zeros(0, dtype=torch.bool, device=packed.device)

    begin_forward = plan

    # ------------------------------------------------------------------- run
    def run(
        self,
        q: torch.Tensor,
        paged_kv_cache,
        *args,
        out: torch.Tensor | None = None,
        lse: torch.Tensor | None = None,
        return_lse: bool = False,
        append_key_states: torch.Tensor | None = None,
        append_value_states: torch.Tensor | None = None,
        rope_cos_sin: tuple[torch.Tensor, torch.Tensor] | None = None,
    ):
        """Attention of the planned batch.  With ``append_key_states`` and
        ``append_value_states`` ([nnz, Hkv, D], one row per query token), each
        request's rows are first written to its last qo_len key positions,
        inside the same launch: ``write_suffix_kv`` followed by ``run`` as one
        kernel (``flashinfer_full_verify.py:1216-1223``).  Needs a head_dim-128
        plan with one row block per (request, KV head)
        (``current_plan.fused_append``); otherwise NotImplementedError.

        ``rope_cos_sin=(cos, sin)`` ([nnz, D] in q's dtype, row = query token,
        as ``rope_cos_sin`` returns them, ``flashinfer_full_verify.py:259-301``)
        goes with the fused append: ``q`` and ``append_key_states`` are then
        the projections before the rotary embedding, and the launch applies
        ``apply_rope_with_cos_sin`` (``:324-333``, called at ``:1213``) itself,
        with the same rounding, so the cache receives the K rows the reference
        writes, bit for bit."""
        plan = self._plan
        if plan is None:
            raise RuntimeError("plan() must be called before run()")
        hnd = self._kv_layout == "HND"
        # (token, head) dims of a page: NHD pages [.., page_size, Hkv, D],
        # HND pages [.., Hkv, page_size, D]
        td, hd = (-2, -3) if hnd else (-3, -2)
        if isinstance(paged_kv_cache, (tuple, list)):
            k_cache, v_cache = paged_kv_cache
            if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
                raise ValueError("K and V caches must have the same shape and strides")
            if k_cache.ndim != 4:
                raise ValueError(f"tuple KV caches must be [pages, {'Hkv, page_size' if hnd else 'page_size, Hkv'}, D]")
            base = k_cache
            v_offset = int(v_cache.data_ptr()) - int(k_cache.data_ptr())
        else:
            kv = paged_kv_cache
            if kv.ndim != 5 or int(kv.shape[1]) != 2:
                raise ValueError(f"kv cache must be [pages, 2, {'Hkv, page_size' if hnd else 'page_size, Hkv'}, D], "
                                 f"got {tuple(kv.shape)}")
            base = kv
            v_offset = kv.stride(1) * kv.element_size()
        es = base.element_size()
        page_stride = base.stride(0) * es
        token_stride = base.stride(td) * es
        head_stride = base.stride(hd) * es
        shape_tail = (int(base.shape[td]), int(base.shape[hd]), int(base.shape[-1]))
        device = _lib.require_device(q, base, what="tree verify attention")
        if shape_tail != (plan.page_size, plan.num_kv_heads, plan.head_dim):
            raise ValueError(
                f"kv cache (page_size, Hkv, D) {shape_tail} does not match the plan "
                f"({plan.page_size}, {plan.num_kv_heads}, {plan.head_dim})"
            )
        if base.stride(-1) != 1 or (not hnd and plan.num_kv_heads > 1 and base.stride(-2) != plan.head_dim):
            raise ValueError("kv cache rows must be contiguous: (Hkv, D) for NHD pages, D for HND pages")
        if q.dtype != plan.q_dtype or base.dtype != plan.kv_dtype:
            raise TypeError(f"dtype mismatch: q {q.dtype}, kv {base.dtype}, planned {plan.q_dtype}")
        if q.ndim != 3 or tuple(q.shape[1:]) != (plan.num_qo_heads, plan.head_dim) or int(q.shape[0]) < plan.nnz:
            raise ValueError(f"q must be [nnz, {plan.num_qo_heads}, {plan.head_dim}], got {tuple(q.shape)}")
        if q.stride(-1) != 1:
            raise ValueError("q rows must be contiguous")
        if out is None:
            out = torch.empty((int(q.shape[0]), plan.num_qo_heads, plan.head_dim), dtype=q.dtype, device=device)
        if out.stride(-1) != 1 or out.dtype != q.dtype:
            raise ValueError("out must have q's dtype and contiguous rows")
        want_lse = return_lse or lse is not None
        if want_lse and lse is None:
            lse = torch.empty((int(q.shape[0]), plan.num_qo_heads), dtype=torch.float32, device=device)
        if lse is not None and (lse.dtype != torch.float32 or not lse.is_contiguous()):
            raise ValueError("lse must be a contiguous float32 tensor")
        ws_bytes = plan.partial_rows * _partial_row_bytes(plan.head_dim)
        lib = _lib.load()
        common = (
            _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(base), page_stride, v_offset, token_stride, head_stride,
            _lib.ptr(plan.qo_indptr), _lib.ptr(plan.kv_indptr), _lib.ptr(plan.kv_indices),
            plan.device_view(plan.kv_len_offset), plan.mask_mode, _lib.ptr(plan.tree_mask),
            plan.device_view(plan.col_offset), plan.mask_words, plan.device_view(plan.work_offset), plan.num_work,
            _lib.ptr(plan.page_windows) if plan.page_windows is not None else None,
            plan.device_view(plan.merge_offset) if plan.num_merge else None, plan.num_merge,
            plan.partial_rows if plan.num_merge else 0, plan.max_rows,
            plan.num_qo_heads, plan.num_kv_heads, plan.head_dim, plan.page_size, plan.sm_scale,
            _lib.dtype_code(q.dtype), _lib.ptr(out), out.stride(0), out.stride(1),
            _lib.ptr(lse) if lse is not None else None, _lib.ptr(self._workspace) if ws_bytes else None,
            ws_bytes,
        )
        if append_key_states is None and append_value_states is None:
            if rope_cos_sin is not None:
                raise NotImplementedError("rope_cos_sin is applied only together with the fused append")
            rc = lib.atlas_tree_verify_attn(*common, _lib.stream_of(device))
            _lib.check(rc, "atlas_tree_verify_attn")
        else:
            k_new, v_new = append_key_states, append_value_states
            if k_new is None or v_new is None:
                raise ValueError("append_key_states and append_value_states go together")
            if not plan.fused_append:
                raise NotImplementedError(
                    "the fused append needs a head_dim-128 plan with one row block per (request, KV head); "
                    "call write_suffix_kv, then run()")
            _lib.require_device(k_new, v_new, what="fused append")
            want = (plan.nnz, plan.num_kv_heads, plan.head_dim)
            for name, t in (("append_key_states", k_new), ("append_value_states", v_new)):
                if t.ndim != 3 or tuple(t.shape[1:]) != want[1:] or int(t.shape[0]) < plan.nnz:
                    raise ValueError(f"{name} must be [nnz, {plan.num_kv_heads}, {plan.head_dim}], got {tuple(t.shape)}")
                if t.dtype != plan.kv_dtype or t.stride(-1) != 1:
                    raise ValueError(f"{name} must have the cache dtype and contiguous rows")
            if k_new.stride() != v_new.stride():
                raise ValueError("append_key_states and append_value_states must have the same strides")
            cos = sin = None
            if rope_cos_sin is not None:
                cos, sin = (_rope_table(t, name, plan, q.dtype) for t, name in zip(rope_cos_sin, ("cos", "sin")))
                _lib.require_device(cos, sin, what="rotary tables")
                if cos.stride(0) != sin.stride(0):
                    raise ValueError("rope cos and sin must have the same row stride")
            rc = lib.atlas_tree_verify_attn_append(*common, _lib.ptr(k_new), _lib.ptr(v_new), k_new.stride(0),
                                                   k_new.stride(1), _lib.ptr(cos), _lib.ptr(sin),
                                                   cos.stride(0) if cos is not None else 0, _lib.stream_of(device))
            _lib.check(rc, "atlas_tree_verify_attn_append")
        if want_lse:
            return out, lse
        return out

    forward = run

    @property
    def current_plan(self) -> AttentionPlan | None:
        return self._plan
