"""Paged decode attention (one query per request) on the gfx950 kernels.

``BatchDecodeWithPagedKVCacheWrapper`` keeps FlashInfer's decode interface as
the reference drives it:

* ``make_decode_wrapper`` / ``plan_decode_wrapper`` create and plan it
  (src/atlas_0709/flashinfer_full_verify.py:882-927, with the keyword retry
  ladder of :901-927);
* the Drafter's SGLang backend calls ``begin_forward(kv_indptr, kv_indices,
  kv_last_page_len, Hq, Hkv, D, page_size, data_type=, q_data_type=,
  non_blocking=True, ...)`` per decode batch and then ``forward(q, (k_cache,
  v_cache), sm_scale=, logits_soft_cap=, k_scale=, v_scale=)`` per layer
  (src/atlas_0709/flashinfer_paged/sglang_page_attention.py:121-140, :171-209).

A decode batch runs on the same paged kernels as the verify attention, with
no mask.  Forked Drafter routes list the same prefix pages (each route owns
only its copy-on-write tail page), so the plan reads the page table once on the
host and builds a cascade: consecutive routes whose page lists begin with the
same full pages form a group.
* One set of work items streams the group's shared pages for all of its routes'
  query rows together (GQA rows of every route packed as the rows of one
  request).
* One small item per route and KV head streams the route's own pages.
* The split merge combines the two states of every row exactly (log-sum-exp
  weights), as it combines key splits.

The shared prefix is then read once per group instead of once per route.
Routes that share nothing are planned one request each (qo_indptr =
0, 1, ..., B), exactly like a prefill batch of single-query requests.

Not supported (raise NotImplementedError): RoPE inside the kernel, sliding
windows, logit soft-capping, and k_scale / v_scale other than 1.
"""

from __future__ import annotations

import dataclasses
import math

import torch

from . import _lib
from .tree_attention import (
    DEFAULT_CU_COUNT,
    DEFAULT_ROWS_PER_ITEM,
    MAX_ROWS_PER_ITEM,
    TILE_KEYS,
    BatchPrefillWithPagedKVCacheWrapper,
    _dtype_from,
    _partial_row_bytes,
    _host_lists,
    pack_plan,
)

# Routes whose page lists begin with at least this many identical full pages
# share one cascade prefix pass.
CASCADE_MIN_SHARED_PAGES = 2
# Shortest key split of a cascade's long streams, in 64-key tiles.
CASCADE_MIN_TILES_PER_SPLIT = 2


def _unit_scale(value, name: str) -> None:
    if value is None:
        return
    if isinstance(value, torch.Tensor):
        if value.numel() != 1:
            raise NotImplementedError(f"{name} must be a scalar")
        value = float(value.item())
    if float(value) != 1.0:
        raise NotImplementedError(f"{name} other than 1 is not supported (fp16/bf16 KV only)")


class BatchDecodeWithPagedKVCacheWrapper:
    """FlashInfer ``BatchDecodeWithPagedKVCacheWrapper`` over the gfx950 paged
    attention kernels (NHD or HND pages, head_dim 64 or 128, fp16 / bf16)."""

    def __init__(
        self,
        float_workspace_buffer: torch.Tensor,
        kv_layout: str = "NHD",
        use_cuda_graph: bool = False,
        use_tensor_cores: bool = False,
        backend: str = "auto",
        **_unused,
    ) -> None:
        self._prefill = BatchPrefillWithPagedKVCacheWrapper(float_workspace_buffer, kv_layout, backend=backend)
        self._use_cuda_graph = bool(use_cuda_graph)
        self._batch = 0
        # Group routes with shared leading pages into a cascade (off: every
        # route streams its whole page list).
        self.use_cascade = True
        self.cascade_groups = 0
        # Work items to aim for when splitting keys (None: the planner's
        # default); plan(disable_split_kv=True) keeps every request whole.
        self.split_target_items: int | None = None

    @property
    def is_cuda_graph_enabled(self) -> bool:
        return self._use_cuda_graph

    @property
    def kv_layout(self) -> str:
        """The paged layout run() reads: "NHD" or "HND"."""
        return self._prefill.kv_layout

    @property
    def current_plan(self):
        return self._prefill.current_plan

    @property
    def prefill_wrapper(self) -> BatchPrefillWithPagedKVCacheWrapper:
        """The wrapper holding the plan (its split and page-window knobs)."""
        return self._prefill

    # ------------------------------------------------------------------ plan
    def plan(
        self,
        indptr: torch.Tensor,
        indices: torch.Tensor,
        last_page_len: torch.Tensor,
        num_qo_heads: int,
        num_kv_heads: int,
        head_dim: int,
        page_size: int,
        pos_encoding_mode: str = "NONE",
        window_left: int = -1,
        logits_soft_cap: float | None = None,
        q_data_type=None,
        kv_data_type=None,
        data_type=None,
        sm_scale: float | None = None,
        rope_scale: float | None = None,
        rope_theta: float | None = None,
        non_blocking: bool = True,
        fixed_split_size: int | None = None,
        disable_split_kv: bool = False,
        **_unused,
    ) -> None:
        if pos_encoding_mode != "NONE":
            raise NotImplementedError("only pos_encoding_mode='NONE' is supported (RoPE is applied by the caller)")
        if window_left != -1 or logits_soft_cap not in (None, 0.0):
            raise NotImplementedError("sliding windows and logit soft-capping are not supported")
        # FlashInfer: data_type is the older name of the KV (and q) type.
        q_dtype = _dtype_from(q_data_type if q_data_type is not None else data_type, torch.float16)
        kv_dtype = _dtype_from(kv_data_type if kv_data_type is not None else data_type, q_dtype)
        if isinstance(indptr, torch.Tensor):
            batch = int(indptr.numel()) - 1
        else:
            batch = len(indptr) - 1
        if batch <= 0:
            raise ValueError("indptr must describe at least one request")
        self._prefill.split_target_items = 1 if disable_split_kv else self.split_target_items
        self.cascade_groups = 0
        if self.use_cascade and batch > 1 and not disable_split_kv:
            if self._plan_cascade(indptr, indices, last_page_len, int(num_qo_heads), int(num_kv_heads),
                                  int(head_dim), int(page_size), q_dtype, kv_dtype, sm_scale, non_blocking):
                self._batch = batch
                return
        qo = torch.arange(batch + 1, dtype=torch.int32)
        self._prefill.plan(
            qo, indptr, indices, last_page_len, num_qo_heads, num_kv_heads, head_dim, page_size,
            causal=False, pos_encoding_mode="NONE", sm_scale=sm_scale, q_data_type=q_dtype, kv_data_type=kv_dtype,
            non_blocking=non_blocking,
        )
        self._batch = batch

    begin_forward = plan

    def _plan_cascade(self, indptr, indices, last_page_len, hq, hkv, d, ps, q_dtype, kv_dtype, sm_scale,
                      non_blocking) -> bool:
        """Cascade plan over groups of routes sharing leading full pages.
        Returns False (nothing planned) when no two neighbouring routes share
        CASCADE_MIN_SHARED_PAGES pages."""
        pf = self._prefill
        if hq <= 0 or hkv <= 0 or hq % hkv != 0:
            raise ValueError("num_qo_heads must be a positive multiple of num_kv_heads")
        if d not in (64, 128):
            raise NotImplementedError(f"head_dim {d} is not supported (64 or 128)")
        if ps <= 0:
            raise ValueError("page_size must be positive")
        if q_dtype != kv_dtype:
            raise NotImplementedError("q and kv data types must match")
        kvp, last, idx = _host_lists(indptr, last_page_len, indices)
        batch = len(kvp) - 1
        if len(last) != batch or any(b < a for a, b in zip(kvp, kvp[1:])) or kvp[-1] > len(idx):
            raise ValueError("indptr / indices / last_page_len sizes are inconsistent")
        kv_lens = []
        for b in range(batch):
            n = kvp[b + 1] - kvp[b]
            if n and not (1 <= last[b] <= ps):
                raise ValueError(f"last_page_len[{b}]={last[b]} outside [1, page_size]")
            kv_lens.append((n - 1) * ps + last[b] if n else 0)
        group = hq // hkv
        direct = d == 128 and ps >= 16 and (ps & (ps - 1)) == 0
        max_routes = max(1, (MAX_ROWS_PER_ITEM if direct else 3 * DEFAULT_ROWS_PER_ITEM) // group)

        def full_pages(b):  # every page but the route's last (which holds its newest token)
            return idx[kvp[b]: max(kvp[b], kvp[b + 1] - 1)]

        # (first route, route count, shared pages)
        groups: list[tuple[int, int, int]] = []
        b = 0
        while b < batch:
            first = full_pages(b)
            shared, n = len(first), 1
            while b + n < batch and n < max_routes:
                other = full_pages(b + n)
                c = 0
                lim = min(shared, len(other))
                while c < lim and other[c] == first[c]:
                    c += 1
                if c < CASCADE_MIN_SHARED_PAGES:
                    break
                shared, n = c, n + 1
            if n < 2 or shared < CASCADE_MIN_SHARED_PAGES:
                groups.append((b, 1, 0))
                b += 1
            else:
                groups.append((b, n, shared))
                b += n
        if not any(n > 1 for _, n, _ in groups):
            return False

        def tiles(keys):
            return math.ceil(keys / TILE_KEYS)

        def split_bounds(t, splits):
            per, extra = t // splits, t - (t // splits) * splits
            for s_ in range(splits):
                t0 = s_ * per + min(s_, extra)
                yield t0, t0 + per + (1 if s_ < extra else 0)

        # Split the long streams (shared prefixes, and whole routes outside
        # groups) so that they alone fill the device about twice, in splits of
        # at least CASCADE_MIN_TILES_PER_SPLIT tiles: the per-route tails are
        # short and add their own items; shorter splits cost more merge work
        # than they gain.
        tail_items = sum(hkv * n for _, n, _ in groups if n > 1)
        long_tiles = sum(hkv * tiles(c * ps if n > 1 else kv_lens[g0]) for g0, n, c in groups)
        if pf.split_target_items is not None:
            tiles_per_split = max(1.0, long_tiles / max(1, pf.split_target_items - tail_items))
        else:
            tiles_per_split = max(float(CASCADE_MIN_TILES_PER_SPLIT), long_tiles / (2 * DEFAULT_CU_COUNT))
        ws_rows_cap = pf._workspace.numel() * pf._workspace.element_size() // _partial_row_bytes(d)
        while True:
            work, merge, qo, qo_lens, plan_kv_lens = [], [], [0], [], []
            partial_rows = 0
            for gi, (g0, n, c) in enumerate(groups):
                rows = n * group
                qo.append(qo[-1] + n)
                qo_lens.append(n)
                # a route of its own streams its whole page list; a group
                # streams the shared pages, then each route its own pages
                keys = kv_lens[g0] if n == 1 else c * ps
                plan_kv_lens.append(keys)
                t = tiles(keys)
                splits = max(1, min(t, int(t / tiles_per_split + 1e-9))) if t else 1
                vals = (g0, n, keys, 0, kvp[g0], 0, 0, 0, 0)
                for h in range(hkv):
                    if n == 1 and splits == 1:
                        work.append((gi, h, 0, rows, 0, keys, -1) + vals)
                        continue
                    base = partial_rows
                    for s_, (t0, t1) in enumerate(split_bounds(t, splits)):
                        work.append((gi, h, 0, rows, t0 * TILE_KEYS, min(keys, t1 * TILE_KEYS), base + s_ * rows)
                                    + vals)
                    nsplit = splits
                    if n > 1:
                        tail_base = base + splits * rows
                        for k in range(n):
                            r = g0 + k
                            tl = kv_lens[r] - keys
                            work.append((gi, h, k * group, group, 0, tl, tail_base + k * group,
                                         g0, n, tl, 0, kvp[r] + c, 0, 0, 0, 0))
                        nsplit += 1
                    merge.append((gi, h, 0, rows, base, nsplit, 0, 0))
                    partial_rows += nsplit * rows
            if partial_rows <= ws_rows_cap or tiles_per_split > float(1 << 20):
                break
            tiles_per_split *= 2
        if partial_rows > ws_rows_cap:
            raise ValueError("workspace too small for the decode plan's partial states")
        # Longest streams first: workgroups are dispatched in order.
        work.sort(key=lambda it: -(it[5] - it[4]))
        src = indices.reshape(-1) if isinstance(indices, torch.Tensor) else torch.tensor(idx, dtype=torch.int32)
        dec = pack_plan(work=work, merge=merge, partial_rows=partial_rows, max_rows=max(it[3] for it in work),
                        direct=direct, fused_append=False, kv_lens=plan_kv_lens, cols=[0] * len(groups), qo=qo,
                        kvp=kvp)
        pf._install(
            batch=len(groups), hq=hq, hkv=hkv, d=d, ps=ps, sm_scale=sm_scale, q_dtype=q_dtype, kv_dtype=kv_dtype,
            mask_mode=_lib.MASK_NONE, dec=dec, kv_lens=plan_kv_lens, qo_lens=qo_lens, indices_src=src,
            tree_bits=None, non_blocking=non_blocking)
        self.cascade_groups = sum(1 for _, n, _ in groups if n > 1)
        return True

    # ------------------------------------------------------------------- run
    def run(
        self,
        q: torch.Tensor,
        paged_kv_cache,
        *args,
        q_scale=None,
        k_scale=None,
        v_scale=None,
        out: torch.Tensor | None = None,
        lse: torch.Tensor | None = None,
        return_lse: bool = False,
        **_unused,
    ):
        """q: [batch, Hq, D] -> out [batch, Hq, D] (and lse [batch, Hq])."""
        if self._batch == 0:
            raise RuntimeError("plan() must be called before run()")
        _unit_scale(q_scale, "q_scale")
        _unit_scale(k_scale, "k_scale")
        _unit_scale(v_scale, "v_scale")
        if q.ndim != 3 or int(q.shape[0]) != self._batch:
            raise ValueError(f"q must be [{self._batch}, Hq, D] (one query per planned request), got {tuple(q.shape)}")
        return self._prefill.run(q, paged_kv_cache, out=out, lse=lse, return_lse=return_lse)

    def forward(
        self,
        q: torch.Tensor,
        paged_kv_cache,
        pos_encoding_mode: str = "NONE",
        q_scale=None,
        k_scale=None,
        v_scale=None,
        window_left: int = -1,
        logits_soft_cap: float | None = None,
        sm_scale: float | None = None,
        rope_scale: float | None = None,
        rope_theta: float | None = None,
    ) -> torch.Tensor:
        """The older entry point SGLang calls; sm_scale here overrides the plan's."""
        if pos_encoding_mode != "NONE":
            raise NotImplementedError("only pos_encoding_mode='NONE' is supported (RoPE is applied by the caller)")
        if window_left != -1 or logits_soft_cap not in (None, 0.0):
            raise NotImplementedError("sliding windows and logit soft-capping are not supported")
        plan = self._prefill.current_plan
        if plan is None:
            raise RuntimeError("plan() must be called before forward()")
        if sm_scale is not None:
            # a copy: a later plan() of the same shape may hand back the
            # cached plan object, which keeps the plan's own scale
            self._prefill._plan = dataclasses.replace(plan, sm_scale=float(sm_scale))
        return self.run(q, paged_kv_cache, q_scale=q_scale, k_scale=k_scale, v_scale=v_scale)

    def end_forward(self) -> None:
        """FlashInfer keeps this as a no-op."""


def make_decode_wrapper(*, args, flashinfer=None, kv_layout: str | None = None) -> BatchDecodeWithPagedKVCacheWrapper:
    """Workspace-backed decode wrapper (``flashinfer_full_verify.py:882-888``)
    for ``kv_layout`` pages (default: ``args.kv_layout`` when set, else NHD)."""
    workspace = torch.empty(int(args.workspace_mb) * 1024 * 1024, dtype=torch.uint8, device=args.device)
    layout = kv_layout or getattr(args, "kv_layout", None) or "NHD"
    return BatchDecodeWithPagedKVCacheWrapper(workspace, layout, backend=getattr(args, "flashinfer_backend", "auto"))


def plan_decode_wrapper(wrapper, *, seq_len: int, args, config, dtype: torch.dtype) -> None:
    """One request over pages 0 .. ceil(seq_len / page_size) - 1, with the
    reference's keyword retry ladder (``flashinfer_full_verify.py:891-927``)."""
    head_dim = getattr(config, "head_dim", int(config.hidden_size) // int(config.num_attention_heads))
    ps = int(args.page_size)
    pages = (int(seq_len) + ps - 1) // ps
    device = torch.device(args.device)
    indptr = torch.tensor([0, pages], dtype=torch.int32, device=device)
    indices = torch.arange(pages, dtype=torch.int32, device=device)
    last_len = torch.tensor([int(seq_len) - (pages - 1) * ps], dtype=torch.int32, device=device)
    attempts = [
        {"pos_encoding_mode": "NONE", "data_type": dtype},
        {"pos_encoding_mode": "NONE", "q_data_type": dtype},
        {"data_type": dtype},
        {},
    ]
    last_error: Exception | None = None
    for kwargs in attempts:
        try:
            wrapper.plan(indptr, indices, last_len, int(config.num_attention_heads), int(config.num_key_value_heads),
                         int(head_dim), ps, **kwargs)
            return
        except (AttributeError, TypeError) as exc:
            last_error = exc
    raise RuntimeError(f"BatchDecodeWithPagedKVCacheWrapper.plan failed: {last_error!r}")


__all__ = ["BatchDecodeWithPagedKVCacheWrapper", "make_decode_wrapper", "plan_decode_wrapper"]
