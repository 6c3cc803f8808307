"""Drafter frontier depth (reference ``flashinfer_paged/frontier.py``).

One depth on the device is the frontier launch pair: per-parent top-k of the
next-token log-probs, the candidate descriptors, their stable order and the
policy's selection, all written into the packed int64 records the host then
reads with one copy (the reference builds the same records from ~40 small
torch launches and three host-to-device tensor builds).
"""

from __future__ import annotations

from collections import Counter
from dataclasses import dataclass
from typing import Any, Protocol, Sequence

import numpy as np
import torch

from .. import _lib
from ._frontier_native import candidate_select, frontier_topk
from .kv import KVTreeStore
from .sampling import DrafterSamplingContext, gumbel_proposal
from .types import (
    DecodePhase,
    FrontierDecodeOutput,
    FrontierSelectionStats,
    FrontierStepOutput,
    PendingCandidate,
    PendingCandidateBatch,
    RouteState,
)
from .utils import (
    _per_root_total,
    global_topk_candidate_indices,
    global_topk_candidates,
    group_candidates_by_stage1_root,
    per_root_topk_candidate_indices,
)


class FrontierModelBackend(Protocol):
    def decode_frontier_one_token(self, active_routes: Sequence[RouteState],
                                  attention_backend: Any = None) -> FrontierDecodeOutput: ...


class SelectionPolicy(Protocol):
    phase: DecodePhase

    def select(self, candidates: Sequence[PendingCandidate], *, k: int,
               active_routes: Sequence[RouteState]) -> list[PendingCandidate]: ...

    def select_indices(self, candidates: PendingCandidateBatch, *, k: int,
                       active_routes: Sequence[RouteState]) -> torch.Tensor: ...


@dataclass(frozen=True)
class GlobalTopKSelection:
    """``frontier.py:58-78``: the k best candidates of the whole frontier."""

    phase: DecodePhase = DecodePhase.STAGE1

    def select(self, candidates, *, k, active_routes):
        return global_topk_candidates(candidates, num_selected=k)

    def select_indices(self, candidates, *, k, active_routes):
        return global_topk_candidate_indices(candidates, num_selected=k)

    def device_selection(self, *, k: int, active_routes: Sequence[RouteState]) -> tuple[int, int, int]:
        """(select mode, num_selected, number selected) for the fused launch."""
        return _lib.FRONTIER_SELECT_GLOBAL, int(k), -1


@dataclass(frozen=True)
class PerStage1RootTopKSelection:
    """``frontier.py:81-124``: the k best candidates of every stage-1 root."""

    phase: DecodePhase = DecodePhase.STAGE2

    def select(self, candidates, *, k, active_routes):
        active_roots = {route.stage1_root_id for route in active_routes}
        grouped = group_candidates_by_stage1_root(candidates)
        selected: list[PendingCandidate] = []
        for root_id in sorted(active_roots):
            root_candidates = grouped.get(root_id, [])
            if not root_candidates:
                raise ValueError(f"stage1 root {root_id} produced no candidates")
            selected.extend(global_topk_candidates(root_candidates, num_selected=k))
        return selected

    @staticmethod
    def _root_counts(candidates_per_parent: int, active_routes: Sequence[RouteState]) -> list[tuple[int, int]]:
        route_counts = Counter(int(route.stage1_root_id) for route in active_routes)
        counts = [(root, n * candidates_per_parent) for root, n in route_counts.items()]
        empty = [root for root, n in counts if n == 0]
        if empty:
            raise ValueError(f"stage1 root {min(empty)} produced no candidates")
        return counts

    def select_indices(self, candidates, *, k, active_routes):
        counts = self._root_counts(candidates.candidates_per_parent, active_routes)
        return per_root_topk_candidate_indices(candidates, num_selected=k, root_candidate_counts=counts)

    def device_selection(self, *, k: int, active_routes: Sequence[RouteState],
                         candidates_per_parent: int) -> tuple[int, int, int]:
        counts = self._root_counts(candidates_per_parent, active_routes)
        total = _per_root_total(k, candidates_per_parent * len(active_routes), counts)
        return _lib.FRONTIER_SELECT_PER_ROOT, int(k), total


def _parent_info(decoded_routes: Sequence[RouteState], device: torch.device) -> torch.Tensor:
    """[B, 3] int64 (route id, stage-1 root id, cumulative log-prob bits), one
    host-to-device copy."""
    host = torch.empty((len(decoded_routes), 3), dtype=torch.int64, pin_memory=True)
    rows = host.numpy()
    rows[:, 0] = [int(r.route_id) for r in decoded_routes]
    rows[:, 1] = [int(r.stage1_root_id) for r in decoded_routes]
    rows[:, 2] = np.asarray([float(r.cumulative_logprob) for r in decoded_routes], dtype=np.float64).view(np.int64)
    return host.to(device, non_blocking=True)


def _batch_from_records(records: torch.Tensor, parent_rows: torch.Tensor, count: int, k: int) -> PendingCandidateBatch:
    cand = records[:count]
    return PendingCandidateBatch(
        parent_route_ids=cand[:, 1],
        stage1_root_ids=cand[:, 2],
        parent_row_indices=parent_rows,
        pending_token_ids=cand[:, 3],
        cumulative_logprobs=cand[:, 5].view(torch.float64),
        parent_logprobs=cand[:, 6].view(torch.float64),
        ranks_in_parent=cand[:, 4],
        candidates_per_parent=k,
    )


def _proposal(next_token_logits, sampling, relative_parent_paths):
    if sampling is None or not sampling.config.do_sample:
        return None
    rows = next_token_logits if next_token_logits.ndim == 2 else next_token_logits.unsqueeze(0)
    return gumbel_proposal(rows, sampling, relative_parent_paths)


def _fused(decoded_routes, next_token_logits, *, k, sampling, relative_parent_paths, select_mode=_lib.FRONTIER_NONE,
           num_selected=0, node_ids=None):
    if len(decoded_routes) != int(next_token_logits.shape[0]):
        raise ValueError("decoded_routes and next_token_logits must have the same batch size")
    if k <= 0:
        raise ValueError("k must be positive")
    if relative_parent_paths is None:
        relative_parent_paths = tuple(() for _ in decoded_routes)
    device = _lib.require_device(next_token_logits, what="frontier candidates")
    if node_ids is not None:
        node_ids = node_ids.to(device=device, dtype=torch.int64)
    proposal = _proposal(next_token_logits, sampling, relative_parent_paths)
    token_lp, token_ids, records, parent_rows, selected = frontier_topk(
        next_token_logits, k, proposal=proposal, parent_info=_parent_info(decoded_routes, device),
        select_mode=select_mode, num_selected=num_selected, node_ids=node_ids)
    actual_k = int(token_ids.shape[-1])
    batch = _batch_from_records(records, parent_rows, len(decoded_routes) * actual_k, actual_k)
    return batch, records, selected


def build_pending_candidate_batch(decoded_routes: Sequence[RouteState], next_token_logits: torch.Tensor, *, k: int,
                                  sampling: DrafterSamplingContext | None = None,
                                  relative_parent_paths: Sequence[Sequence[int]] | None = None
                                  ) -> PendingCandidateBatch:
    """``frontier.py:127-185``: the parents' top-k children as device columns
    (strided views of the packed records; cumulative = parent + token
    log-prob in float64)."""
    batch, _, _ = _fused(decoded_routes, next_token_logits, k=k, sampling=sampling,
                         relative_parent_paths=relative_parent_paths)
    return batch


def _new_candidates(parent, root, token, cum, rank, plp) -> list[PendingCandidate]:
    """PendingCandidate objects from column lists with their field dicts set
    directly (the frozen dataclass's __init__ costs more than the rest of a
    frontier depth); equal to PendingCandidate(...) field for field."""
    new, setattr_ = object.__new__, object.__setattr__
    out = []
    for a, b, c, d, e, f in zip(parent, root, token, cum, rank, plp):
        o = new(PendingCandidate)
        setattr_(o, "__dict__", {"parent_route_id": a, "stage1_root_id": b, "pending_token_id": c,
                                 "cumulative_logprob": d, "rank_in_parent": e, "parent_logprob": f})
        out.append(o)
    return out


def _materialize_records(packed: torch.Tensor, candidate_count: int, selected_count: int,
                         new_node_ids_cpu, transferred_node_count: int, new_node_ids_source: str):
    host = packed.detach().cpu().numpy()
    cand = host[:candidate_count]
    materialized = _new_candidates(cand[:, 1].tolist(), cand[:, 2].tolist(), cand[:, 3].tolist(),
                                   cand[:, 5].view(np.float64).tolist(), cand[:, 4].tolist(),
                                   cand[:, 6].view(np.float64).tolist())
    by_order: list[PendingCandidate | None] = [None] * selected_count
    for i in np.flatnonzero((cand[:, 7] >= 0) & (cand[:, 7] < selected_count)).tolist():
        by_order[int(cand[i, 7])] = materialized[i]
    if any(c is None for c in by_order):
        raise RuntimeError("selected candidate order was not fully materialized")
    selected = [c for c in by_order if c is not None]
    if new_node_ids_cpu is not None:
        node_ids = [int(n) for n in new_node_ids_cpu]
    else:
        node_ids = host[candidate_count:, 1].tolist()
        if len(node_ids) != transferred_node_count:
            raise RuntimeError("new node id transfer produced the wrong number of ids")
    on_device = packed.device.type != "cpu"
    stats = FrontierSelectionStats(
        candidate_count=candidate_count, selected_count=selected_count, host_materialization_batches=1,
        host_materialization_elements=int(packed.numel()), host_transfer_batches=int(on_device),
        host_transfer_elements=int(packed.numel()) if on_device else 0, selection_device=str(packed.device),
        new_node_ids_source=new_node_ids_source)
    return materialized, selected, node_ids, stats


def materialize_pending_candidate_batch(candidates: PendingCandidateBatch, selected_indices: torch.Tensor, *,
                                        new_node_ids_cpu: Sequence[int] | None = None,
                                        new_node_ids_to_transfer: torch.Tensor | None = None,
                                        new_node_ids_source: str = "not_applicable"):
    """``frontier.py:188-265``: every candidate and the selection (in
    selection order), plus transferred node ids, through one packed host
    batch; the records are packed on the device in one launch."""
    count = candidates.candidate_count
    selected_count = int(selected_indices.numel())
    node_ids = None
    n_nodes = 0
    if new_node_ids_to_transfer is not None:
        node_ids = new_node_ids_to_transfer.reshape(-1)
        n_nodes = int(node_ids.numel())
    _, _, records = candidate_select(candidates, _lib.FRONTIER_PACK, selected_in=selected_indices,
                                     node_ids=node_ids, records=True)
    return _materialize_records(records, count, selected_count, new_node_ids_cpu, n_nodes, new_node_ids_source)


def collect_pending_candidates(decoded_routes: Sequence[RouteState], next_token_logits: torch.Tensor, *,
                               k: int) -> list[PendingCandidate]:
    _, records, _ = _fused(decoded_routes, next_token_logits, k=k, sampling=None, relative_parent_paths=None)
    count = len(decoded_routes) * min(int(k), int(next_token_logits.shape[-1]))
    candidates, _, _, _ = _materialize_records(records, count, 0, (), 0, "not_applicable")
    return candidates


def advance_frontier_one_token(active_routes: Sequence[RouteState], *, k: int, route_store: KVTreeStore,
                               model_backend: FrontierModelBackend, selection_policy: SelectionPolicy,
                               attention_backend: Any = None,
                               sampling: DrafterSamplingContext | None = None) -> FrontierStepOutput:
    """Decode one frontier depth and materialise its device selection once
    (``frontier.py:332-395``).  The two gfx950 policies select inside the
    frontier launch pair; another policy's select_indices runs on the
    candidate batch, then the records are packed."""
    if not active_routes:
        raise ValueError("active_routes cannot be empty")
    before = _node_counter_state(route_store)
    decode_output = model_backend.decode_frontier_one_token(active_routes, attention_backend=attention_backend)
    after = _node_counter_state(route_store)
    cpu_node_ids, node_ids_to_transfer, node_ids_source = _resolve_new_node_ids(
        decode_output, expected_count=len(active_routes), counter_before=before, counter_after=after)
    logits = decode_output.next_token_logits
    paths = [route_store.pending_token_path(route) for route in active_routes]
    actual_k = min(int(k), int(logits.shape[-1]))
    count = len(active_routes) * actual_k
    n_nodes = 0 if node_ids_to_transfer is None else int(node_ids_to_transfer.numel())
    if isinstance(selection_policy, (GlobalTopKSelection, PerStage1RootTopKSelection)):
        if isinstance(selection_policy, GlobalTopKSelection):
            mode, num, total = selection_policy.device_selection(k=k, active_routes=active_routes)
            total = min(count, num)
        else:
            mode, num, total = selection_policy.device_selection(k=k, active_routes=active_routes,
                                                                 candidates_per_parent=actual_k)
        _, records, _ = _fused(active_routes, logits, k=k, sampling=sampling, relative_parent_paths=paths,
                               select_mode=mode, num_selected=num, node_ids=node_ids_to_transfer)
        candidates, selected, new_node_ids, stats = _materialize_records(
            records, count, total, cpu_node_ids, n_nodes, node_ids_source)
    else:
        batch, _, _ = _fused(active_routes, logits, k=k, sampling=sampling, relative_parent_paths=paths)
        selected_indices = selection_policy.select_indices(batch, k=k, active_routes=active_routes)
        candidates, selected, new_node_ids, stats = materialize_pending_candidate_batch(
            batch, selected_indices, new_node_ids_cpu=cpu_node_ids, new_node_ids_to_transfer=node_ids_to_transfer,
            new_node_ids_source=node_ids_source)
    decoded = route_store.mark_routes_materialized(list(active_routes), new_node_ids, phase=selection_policy.phase)
    next_routes = route_store.materialize_route_descriptors(selected, parent_routes=decoded)
    route_store.release_routes_without_descendants(decoded, next_routes)
    return FrontierStepOutput(decoded_routes=decoded, next_routes=next_routes, candidates=candidates,
                              selected_candidates=selected, decode_output=decode_output, selection_stats=stats)


def _resolve_new_node_ids(decode_output: FrontierDecodeOutput, *, expected_count: int,
                          counter_before: tuple[int, int] | None, counter_after: tuple[int, int] | None):
    """``frontier.py:398-440``: node ids from the decode output, from the
    store's counter when the backend reserved exactly expected_count ids, or
    through the packed transfer."""
    if decode_output.new_node_ids_cpu is not None:
        ids = [int(n) for n in decode_output.new_node_ids_cpu]
        if len(ids) != expected_count:
            raise ValueError("new_node_ids_cpu must have one id per active route")
        return ids, None, "decode_output_cpu"
    if not isinstance(decode_output.new_node_ids, torch.Tensor):
        ids = [int(n) for n in decode_output.new_node_ids]
        if len(ids) != expected_count:
            raise ValueError("new_node_ids must have one id per active route")
        return ids, None, "decode_output_sequence"
    if int(decode_output.new_node_ids.numel()) != expected_count:
        raise ValueError("new_node_ids must have one id per active route")
    if (counter_before is not None and counter_after is not None and counter_before[1] == counter_after[1]
            and counter_after[0] == counter_before[0] + expected_count * counter_before[1]):
        return [counter_before[0] + i * counter_before[1] for i in range(expected_count)], None, "route_store_counter"
    return None, decode_output.new_node_ids, "packed_transfer"


def _node_counter_state(route_store: KVTreeStore) -> tuple[int, int] | None:
    """(next node id, step) of the store's id counter without consuming an
    id: this package's store reports it; a store counting with
    itertools.count (``kv.py:30``) is read through its pickling state
    (``frontier.py:443-456``)."""
    state = getattr(route_store, "node_counter_state", None)
    if callable(state):
        return state()
    reduce_method = getattr(getattr(route_store, "_node_ids", None), "__reduce__", None)
    if not callable(reduce_method):
        return None
    try:
        args = reduce_method()[1]
        return int(args[0]), (int(args[1]) if len(args) > 1 else 1)
    except (IndexError, TypeError, ValueError):
        return None
