"""Calls of the frontier entry points (atlas_frontier_topk,
atlas_candidate_select) with the workspace they keep per device."""

from __future__ import annotations

import ctypes
import threading

import torch

from .. import _lib

_ws_lock = threading.Lock()
_workspaces: dict[torch.device, torch.Tensor] = {}


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A 256-byte aligned byte buffer of at least nbytes on device, kept per
    device (the launches clear what they need; calls on one device share it,
    so they must be stream-ordered)."""
    with _ws_lock:
        ws = _workspaces.get(device)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
            _workspaces[device] = ws
        return ws


def _as_rows(logits: torch.Tensor) -> torch.Tensor:
    if logits.ndim == 1:
        logits = logits.unsqueeze(0)
    if logits.ndim != 2:
        raise ValueError(f"expected 1D or 2D logits, got shape {tuple(logits.shape)}")
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    return logits


def frontier_topk(logits: torch.Tensor, k: int, *, proposal: torch.Tensor | None = None,
                  parent_info: torch.Tensor | None = None, select_mode: int = _lib.FRONTIER_NONE,
                  num_selected: int = 0, node_ids: torch.Tensor | None = None):
    """One launch pair over logits [rows, V].  Returns (token_logprobs [rows, k]
    in the logits dtype, token_ids [rows, k] int64, records or None,
    parent_rows or None, selected or None)."""
    rows_t = _as_rows(logits)
    device = _lib.require_device(rows_t, proposal, parent_info, node_ids, what="frontier top-k")
    dtype_code = _lib.dtype_code(rows_t.dtype)
    rows, vocab = int(rows_t.shape[0]), int(rows_t.shape[1])
    if k <= 0:
        raise ValueError("k must be positive")
    k = min(int(k), vocab)
    if k > _lib.MAX_FRONTIER_K:
        raise NotImplementedError(f"frontier top-k supports k <= {_lib.MAX_FRONTIER_K}, got {k}")
    if proposal is not None:
        if proposal.dtype != torch.float32 or tuple(proposal.shape) != (rows, vocab) or proposal.stride(-1) != 1:
            raise ValueError("proposal scores must be float32 [rows, vocab] with contiguous rows")
    lib = _lib.load()
    nbytes = int(lib.atlas_frontier_workspace_bytes(rows, vocab, k))
    if nbytes < 0:
        raise ValueError(f"frontier workspace: bad shape rows={rows} vocab={vocab} k={k}")
    ws = _workspace(device, nbytes)
    token_lp = torch.empty((rows, k), dtype=rows_t.dtype, device=device)
    token_ids = torch.empty((rows, k), dtype=torch.int64, device=device)
    records = parent_rows = selected = None
    n_nodes = 0
    if parent_info is not None:
        count = rows * k
        if count > _lib.MAX_FRONTIER_CANDIDATES:
            raise NotImplementedError(
                f"frontier selection supports up to {_lib.MAX_FRONTIER_CANDIDATES} candidates, got {count}")
        if node_ids is not None:
            node_ids = node_ids.to(device=device, dtype=torch.int64).reshape(-1).contiguous()
            n_nodes = int(node_ids.numel())
        records = torch.empty((count + n_nodes, 8), dtype=torch.int64, device=device)
        parent_rows = torch.empty(count, dtype=torch.int64, device=device)
        if select_mode in (_lib.FRONTIER_SELECT_GLOBAL, _lib.FRONTIER_SELECT_PER_ROOT):
            # per root: at most num_selected per root, so never more than count
            selected = torch.empty(min(count, int(num_selected) if select_mode == _lib.FRONTIER_SELECT_GLOBAL
                                       else count), dtype=torch.int64, device=device)
    rc = lib.atlas_frontier_topk(
        _lib.ptr(rows_t), rows, vocab, rows_t.stride(0), dtype_code, _lib.ptr(proposal),
        proposal.stride(0) if proposal is not None else 0, k, _lib.ptr(parent_info), select_mode,
        int(num_selected), _lib.ptr(node_ids), n_nodes, _lib.ptr(token_lp), _lib.ptr(token_ids), _lib.ptr(records),
        _lib.ptr(parent_rows), _lib.ptr(selected), _lib.ptr(ws), ws.numel(), _lib.stream_of(device))
    _lib.check(rc, "atlas_frontier_topk")
    return token_lp, token_ids, records, parent_rows, selected


def _column(t: torch.Tensor, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    t = t.reshape(-1)
    if t.dtype != dtype or t.device != device:
        t = t.to(device=device, dtype=dtype)
    return t


def candidate_select(batch, mode: int, *, num_selected: int = 0, selected_in: torch.Tensor | None = None,
                     node_ids: torch.Tensor | None = None, records: bool = False):
    """atlas_candidate_select over a PendingCandidateBatch.  Returns (order or
    None, selected or None, records or None)."""
    device = _lib.require_device(batch.pending_token_ids, what="frontier candidate order")
    cols = [
        _column(batch.parent_route_ids, torch.int64, device),
        _column(batch.stage1_root_ids, torch.int64, device),
        _column(batch.pending_token_ids, torch.int64, device),
        _column(batch.ranks_in_parent, torch.int64, device),
        _column(batch.cumulative_logprobs, torch.float64, device),
        _column(batch.parent_logprobs, torch.float64, device),
    ]
    count = int(cols[2].numel())
    if any(int(c.numel()) != count for c in cols):
        raise ValueError("candidate columns must have the same length")
    if count > _lib.MAX_FRONTIER_CANDIDATES:
        raise NotImplementedError(
            f"frontier selection supports up to {_lib.MAX_FRONTIER_CANDIDATES} candidates, got {count}")
    strides = (ctypes.c_int64 * 6)(*[int(c.stride(0)) for c in cols])
    order = selected = recs = None
    n_nodes = 0
    if node_ids is not None:
        node_ids = node_ids.to(device=device, dtype=torch.int64).reshape(-1).contiguous()
        n_nodes = int(node_ids.numel())
    if mode in (_lib.FRONTIER_ORDER, _lib.FRONTIER_ORDER_BY_ROOT):
        order = torch.empty(count, dtype=torch.int64, device=device)
    elif mode == _lib.FRONTIER_SELECT_GLOBAL:
        selected = torch.empty(min(count, int(num_selected)), dtype=torch.int64, device=device)
    elif mode == _lib.FRONTIER_SELECT_PER_ROOT:
        selected = torch.empty(count, dtype=torch.int64, device=device)
    n_sel_in = 0
    if selected_in is not None:
        selected_in = selected_in.to(device=device, dtype=torch.int64).reshape(-1).contiguous()
        n_sel_in = int(selected_in.numel())
    if records or mode == _lib.FRONTIER_PACK:
        recs = torch.empty((count + n_nodes, 8), dtype=torch.int64, device=device)
    rc = _lib.load().atlas_candidate_select(
        *[_lib.ptr(c) for c in cols], ctypes.cast(strides, ctypes.c_void_p), count, mode, int(num_selected),
        _lib.ptr(selected_in), n_sel_in, _lib.ptr(node_ids), n_nodes, _lib.ptr(order), _lib.ptr(selected),
        _lib.ptr(recs), _lib.stream_of(device))
    _lib.check(rc, "atlas_candidate_select")
    return order, selected, recs
