"""Frontier candidate helpers (reference ``flashinfer_paged/utils.py``).

The device-side order and selection run in one gfx950 launch
(atlas_candidate_select) instead of four stable argsorts with their gathers;
the Python-object helpers keep the reference's semantics on host objects.
"""

from __future__ import annotations

from collections import defaultdict
from typing import Iterable, Sequence

import torch

from .. import _lib
from ._frontier_native import candidate_select, frontier_topk
from .types import PendingCandidate, PendingCandidateBatch


def topk_logprobs(logits: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-k of log_softmax of one row (``utils.py:11-24``)."""
    if k <= 0:
        raise ValueError("k must be positive")
    if logits.ndim == 2:
        if logits.shape[0] != 1:
            raise ValueError("topk_logprobs expects a single row or a 1D tensor")
        logits = logits[0]
    if logits.ndim != 1:
        raise ValueError(f"expected 1D logits, got shape {tuple(logits.shape)}")
    lp, ids, _, _, _ = frontier_topk(logits.unsqueeze(0), min(k, int(logits.shape[-1])))
    return lp[0], ids[0]


def global_topk_candidates(candidates: Sequence[PendingCandidate], num_selected: int) -> list[PendingCandidate]:
    """Host-object order (``utils.py:27-43``): cumulative log-prob descending,
    then parent route, rank and token ascending."""
    if num_selected <= 0:
        raise ValueError("num_selected must be positive")
    ordered = sorted(candidates, key=lambda c: (c.cumulative_logprob, -c.parent_route_id, -c.rank_in_parent,
                                                -c.pending_token_id), reverse=True)
    return list(ordered[:num_selected])


def stable_candidate_order(candidates: PendingCandidateBatch, *, include_stage1_root: bool = False) -> torch.Tensor:
    """The full candidate order on the device (``utils.py:46-83``): score
    descending, then parent route, parent rank and token id ascending, exact
    ties in batch order; stage-1 root ascending first for forest selection."""
    mode = _lib.FRONTIER_ORDER_BY_ROOT if include_stage1_root else _lib.FRONTIER_ORDER
    order, _, _ = candidate_select(candidates, mode)
    return order


def global_topk_candidate_indices(candidates: PendingCandidateBatch, *, num_selected: int) -> torch.Tensor:
    """``utils.py:86-95``: the first num_selected of the order."""
    if num_selected <= 0:
        raise ValueError("num_selected must be positive")
    if candidates.candidate_count == 0:
        return torch.empty(0, dtype=torch.long, device=candidates.pending_token_ids.device)
    _, selected, _ = candidate_select(candidates, _lib.FRONTIER_SELECT_GLOBAL, num_selected=num_selected)
    return selected


def _per_root_total(num_selected: int, candidate_count: int,
                    root_candidate_counts: Sequence[tuple[int, int]]) -> int:
    ordered = sorted((int(r), int(n)) for r, n in root_candidate_counts)
    if sum(n for _, n in ordered) != candidate_count:
        raise ValueError("root candidate counts do not cover the candidate batch")
    return sum(min(int(num_selected), n) for _, n in ordered)


def per_root_topk_candidate_indices(candidates: PendingCandidateBatch, *, num_selected: int,
                                    root_candidate_counts: Sequence[tuple[int, int]]) -> torch.Tensor:
    """``utils.py:98-123``: the first num_selected of every stage-1 root, roots
    ascending (the roots' candidate counts must cover the batch)."""
    if num_selected <= 0:
        raise ValueError("num_selected must be positive")
    total = _per_root_total(num_selected, candidates.candidate_count, root_candidate_counts)
    if candidates.candidate_count == 0:
        return torch.empty(0, dtype=torch.long, device=candidates.pending_token_ids.device)
    _, selected, _ = candidate_select(candidates, _lib.FRONTIER_SELECT_PER_ROOT, num_selected=num_selected)
    return selected[:total]


def group_candidates_by_stage1_root(candidates: Iterable[PendingCandidate]) -> dict[int, list[PendingCandidate]]:
    grouped: dict[int, list[PendingCandidate]] = defaultdict(list)
    for c in candidates:
        grouped[c.stage1_root_id].append(c)
    return dict(grouped)


def topk_pairs_to_python(token_ids: torch.Tensor, token_logprobs: torch.Tensor) -> list[tuple[int, float]]:
    """A top-k result in one host batch (``utils.py:140-156``)."""
    if token_ids.shape != token_logprobs.shape:
        raise ValueError("token ids and logprobs must have matching shapes")
    packed = torch.stack((token_ids.to(dtype=torch.float64), token_logprobs.to(dtype=torch.float64)), dim=-1)
    rows = packed.detach().cpu().reshape(-1, 2).tolist()
    return [(int(t), float(lp)) for t, lp in rows]


def logprob_of_token(logits: torch.Tensor, token_id: int) -> float:
    logprobs = torch.log_softmax(logits, dim=-1)
    return float(logprobs[int(token_id)].detach().cpu())
