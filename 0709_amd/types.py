"""Types carried across the Target verify boundary (reference
``atlas_0709/types.py:15-20``, ``:105-148``)."""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Mapping

import torch


@dataclass(frozen=True)
class PrefixState:
    """What ``prefill`` returns: the committed prompt, the logits of the token
    after it, its length and the backend's runtime metadata."""

    token_ids: tuple[int, ...]
    next_token_logits: torch.Tensor
    committed_length: int
    metadata: Mapping[str, Any] = field(default_factory=dict)


@dataclass(frozen=True)
class TargetRouteScore:
    route_id: int
    token_ids: tuple[int, ...]
    target_logprob: float
    draft_logprob: float
    token_logprobs: tuple[float, ...] = ()
    first_token_logprob: float | None = None
    selection_score: float | None = None
    score_weights: tuple[float, ...] = ()
    draft_token_logprobs: tuple[float, ...] = ()

    @property
    def draft_first_token_logprob(self) -> float | None:
        return float(self.draft_token_logprobs[0]) if self.draft_token_logprobs else None

    @property
    def draft_path_logprob(self) -> float:
        """Score of the verified path itself (sum of its per-token draft
        log-probs when known, else the cumulative draft log-prob)."""
        if self.draft_token_logprobs:
            return float(sum(self.draft_token_logprobs))
        return float(self.draft_logprob)


@dataclass(frozen=True)
class TargetVerifyResult:
    selected_route_id: int | None
    scores: list[TargetRouteScore]
    metadata: Mapping[str, Any] = field(default_factory=dict)
    decision: str = "select"
    fallback_token_ids: tuple[int, ...] = ()
    fallback_reason: str | None = None

    @property
    def selected_score(self) -> TargetRouteScore:
        if self.selected_route_id is None:
            raise KeyError("fallback result does not have a selected route")
        for score in self.scores:
            if score.route_id == self.selected_route_id:
                return score
        raise KeyError(self.selected_route_id)
