"""Stand-in callers: the reference runtime's call sequences into the Target and
Drafter backends, written from its call sites without importing it.

* ``TargetRpcStandIn`` -- ``TargetServerApp`` / ``InProcessTargetClient``
  (``src/atlas_0709/rpc.py:66-160``): health reads ``runtime_metadata()``,
  prefill reads ``prefix.committed_length`` and ``prefix.metadata``, verify
  builds payloads with ``verify_payload_from_mapping`` and serialises the
  result field by field as ``target_verify_result_to_dict`` does
  (``rpc.py:15-63``).  Every response goes through ``json.dumps`` /
  ``json.loads``, as the HTTP transport sends it.
* ``edge_prepare_prefix`` / ``edge_fallback_handoff`` -- the edge controller's
  Drafter set-up and fallback EXTEND handoff
  (``src/atlas_0709/distributed_system.py:639-660``, ``:707-735``), with the
  prompt prefill of ``prefill_sglang_prefix``
  (``flashinfer_paged/sglang_runtime.py:1437-1500``) done in one chunk
  through the route pool and the executor's ``forward_extend``.
"""

from __future__ import annotations

import json
from types import SimpleNamespace
from typing import Any, Sequence

import torch

# keys distributed_system.py:680-705 forwards from a verify response to the
# evaluators (present when the policy produces them)
EDGE_DECISION_KEYS = (
    "selection_policy", "route_sampling_enabled", "route_sampling_scope", "route_sampling_seed",
    "route_sampling_round", "route_sampling_temperature", "route_sampling_uniform",
    "route_sampling_selected_probability", "route_sampling_selected_cdf_low", "route_sampling_selected_cdf_high",
    "route_sampling_boundary_margin", "route_sampling_ordered_candidates", "selected_draft_rank", "route0_route_id",
    "draft_top_route_id", "selected_route_changed_from_route0", "selected_first_token_changed_from_route0",
    "selected_minus_route0_draft_first_token_logprob", "selected_minus_route0_draft_logprob",
    "selected_minus_route0_target_selection_score", "route_intervention",
)

# the keys of the reference's runtime_metadata (target_runtime.py:322-359)
RUNTIME_METADATA_KEYS = (
    "backend", "model", "model_vocab_size", "tokenizer_vocab_size", "tokenizer_bos_token_id",
    "tokenizer_eos_token_id", "tokenizer_pad_token_id", "paged_kv", "custom_mask", "packed_custom_mask",
    "rope_applied", "logits_aligned", "runtime_alignment_checked", "semantic_correctness_required", "page_size",
    "dtype", "device", "flashinfer_version", "persistent_target_paged_kv", "deduplicated_tree_nodes",
    "selection_policy", "route_selection_policy", "route_sampling_scope", "route_sampling_temperature",
    "fallback_ar_sampling", "score_weights", "fallback_threshold", "first_token_threshold", "fallback_ar_tokens",
    "fallback_decode_wrapper_reused", "profile_fallback_ar", "committed_verify_rounds", "committed_prefix_length",
)

# the verify metadata keys of target_runtime.py:235-320 beyond the runtime
# metadata, per decision
VERIFY_COMMON_KEYS = (
    "route_count", "path_depth", "node_count", "unmerged_path_node_count", "kv_len", "prefix_len_before",
    "selection_policy", "selection_score_name", "fallback_threshold", "first_token_threshold",
    "fallback_ar_tokens", "route_sampling_enabled", "route_sampling_scope", "route_sampling_seed",
    "route_sampling_round", "route_sampling_temperature", "route_intervention", "selected_draft_rank",
    "route0_route_id", "draft_top_route_id", "selected_route_changed_from_route0",
    "selected_first_token_changed_from_route0", "selected_minus_route0_draft_first_token_logprob",
    "selected_minus_route0_draft_logprob", "selected_minus_route0_target_selection_score",
)
VERIFY_SELECT_KEYS = (
    "prefix_len_after", "target_kv_commit", "target_reprefill_after_verify", "fallback_triggered", "best_route_id",
    "best_selection_score", "best_first_token_logprob", "selected_route_id", "selected_selection_score",
    "selected_path_committed_tokens", "selected_path_was_truncated",
)
VERIFY_FALLBACK_KEYS = (
    "prefix_len_after", "target_kv_commit", "target_reprefill_after_verify", "fallback_triggered",
    "fallback_reason", "fallback_token_count", "best_route_id", "best_selection_score", "best_first_token_logprob",
    "fallback_ar_profile",
)


def _wire(obj: dict) -> dict:
    """What the HTTP transport delivers: the response as JSON."""
    return json.loads(json.dumps(obj))


def score_to_dict(score) -> dict:
    return {
        "route_id": int(score.route_id),
        "token_ids": [int(t) for t in score.token_ids],
        "target_logprob": float(score.target_logprob),
        "draft_logprob": float(score.draft_path_logprob),
        "draft_path_logprob": float(score.draft_path_logprob),
        "legacy_cumulative_draft_logprob": float(score.draft_logprob),
        "token_logprobs": [float(v) for v in score.token_logprobs],
        "first_token_logprob": None if score.first_token_logprob is None else float(score.first_token_logprob),
        "selection_score": None if score.selection_score is None else float(score.selection_score),
        "score_weights": [float(v) for v in score.score_weights],
        "draft_token_logprobs": [float(v) for v in score.draft_token_logprobs],
        "draft_first_token_logprob": score.draft_first_token_logprob,
    }


def verify_result_to_dict(result) -> dict:
    out = {"decision": str(result.decision), "scores": [score_to_dict(s) for s in result.scores],
           "metadata": dict(result.metadata)}
    if result.decision == "fallback_ar":
        out.update(selected_route_id=None, fallback_token_ids=[int(t) for t in result.fallback_token_ids],
                   fallback_reason=result.fallback_reason)
    else:
        out.update(selected_route_id=int(result.selected_route_id), selected_score=score_to_dict(result.selected_score))
    return out


class TargetRpcStandIn:
    """The Target server's request handling around a backend object."""

    def __init__(self, backend, verify_payload_from_mapping) -> None:
        self.backend = backend
        self.from_mapping = verify_payload_from_mapping

    def health(self) -> dict:
        return _wire({"ok": True, "service": "atlas_0709_target", "metadata": self.backend.runtime_metadata()})

    def prefill(self, request: dict) -> dict:
        ids = request.get("prompt_token_ids")
        if not isinstance(ids, list):
            raise ValueError("prefill requires prompt_token_ids: list[int]")
        prefix = self.backend.prefill([int(t) for t in ids])
        return _wire({"ok": True, "prompt_len": int(prefix.committed_length), "metadata": dict(prefix.metadata)})

    def verify(self, request: dict) -> dict:
        def opt(key):
            v = request.get(key)
            return None if v is None else int(v)

        payloads = [self.from_mapping(dict(item)) for item in request["routes"]]
        result = self.backend.verify_payloads(
            prefix_token_ids=[int(t) for t in request["prefix_token_ids"]], routes=payloads,
            fallback_max_tokens=opt("fallback_max_tokens"), selected_path_max_tokens=opt("selected_path_max_tokens"),
            eos_token_id=opt("eos_token_id"), route_sampling_seed=opt("route_sampling_seed"),
            route_sampling_round=opt("route_sampling_round"))
        return _wire({"ok": True, **verify_result_to_dict(result)})


def edge_decision_metadata(metadata: dict) -> dict:
    return {k: metadata[k] for k in EDGE_DECISION_KEYS if k in metadata}


def prefill_prefix(route_pool, executor, prompt: Sequence[int]):
    """One-chunk prompt prefill through the route pool: a request row, the
    prompt's slots continuing an empty prefix, the row write, one EXTEND
    forward, the row freed.  Returns (prefix slots, next-token logits)."""
    device = route_pool.device
    handle = SimpleNamespace(rid="atlas-prefix", req_pool_idx=None)
    rows = route_pool.req_to_token_pool.alloc([handle])
    row = int(torch.as_tensor(rows).reshape(-1)[0])
    handle.req_pool_idx = row
    n = len(prompt)
    try:
        slots = route_pool.allocate_extend_slots(prefix_lens=[0], seq_lens=[n],
                                                 last_locs=torch.full((1,), -1, dtype=torch.long, device=device))
        route_pool._write_req_token_row(row, slots)
        logits = executor.forward_extend(input_ids=torch.tensor(list(prompt), dtype=torch.long, device=device),
                                         out_cache_loc=slots, positions=torch.arange(n, device=device),
                                         req_pool_indices=torch.tensor([row], device=device),
                                         seq_lens_cpu=torch.tensor([n]))
    finally:
        route_pool.req_to_token_pool.free(handle)
    return slots, logits[-1]


def edge_prepare_prefix(mods: Any, *, runner: Any, page_size: int, prompt: Sequence[int], executor: Any = None,
                        device: str = "cpu") -> SimpleNamespace:
    """distributed_system.py:639-660."""
    store = mods.KVTreeStore()
    kw = {} if executor is None else {"executor": executor}
    backend = mods.SGLangFlashInferFrontierModelBackend.from_runner(
        route_store=store, model_runner=runner, page_size=page_size, device=device, **kw)
    backend.route_pool.clear_physical_state()
    slots, logits = prefill_prefix(backend.route_pool, backend.executor, prompt)
    prefix = backend.attach_prefilled_prefix(prompt_token_ids=list(prompt), prefix_slot_ids=slots,
                                             next_token_logits=logits)
    store.committed_token_ids = [int(t) for t in prompt]
    return SimpleNamespace(store=store, backend=backend, prefix=prefix)


def edge_fallback_handoff(ctx: SimpleNamespace, fallback_token_ids: Sequence[int]) -> dict:
    """distributed_system.py:707-735: drop every route row, prune, reset the
    speculative forest, then extend the persistent prefix."""
    suffix = [int(t) for t in fallback_token_ids]
    released_rows = ctx.backend.route_pool.retain_route_rows([])
    released_pages = ctx.backend.route_pool.release_unreferenced_node_slots([])
    ctx.store.committed_token_ids.extend(suffix)
    ctx.store.reset_speculative()
    logits = ctx.backend.append_known_tokens_as_prefix(suffix)
    return {"released_route_rows": released_rows, "released_kv_pages": released_pages, "logits": logits,
            "prefix_token_ids": tuple(int(t) for t in ctx.backend.prefix_token_ids),
            "prefix_view": ctx.store.prefix_view()}
