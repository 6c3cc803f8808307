"""Drafter candidate sampling (reference ``flashinfer_paged/sampling.py``).

The per-parent top-k runs on the gfx950 frontier kernels: log_softmax and
top-k of every logits row in one launch pair.  The do_sample path draws its
Gumbel noise exactly as the reference does (one torch generator per parent,
seeded from the semantic prefix) and hands the proposal scores to the same
kernels, which take their top-k and gather the model log-probs.
"""

from __future__ import annotations

import hashlib
import math
import struct
from dataclasses import dataclass
from typing import Sequence

import torch

from ._frontier_native import frontier_topk

_SAMPLING_SEED_DOMAIN = b"atlas-0709-drafter-semantic-prefix-v1\0"
_TORCH_SEED_MASK = (1 << 63) - 1


@dataclass(frozen=True)
class DrafterSamplingConfig:
    """Request-level candidate sampling (``sampling.py:16-48``): Gumbel-top-k
    draws of k distinct children per parent when do_sample; the recorded
    scores stay the untempered model log-probs."""

    do_sample: bool = False
    seed: int = 0
    temperature: float = 1.0

    def validate(self) -> None:
        if not math.isfinite(float(self.temperature)) or float(self.temperature) <= 0.0:
            raise ValueError("drafter sampling temperature must be finite and positive")

    def to_dict(self) -> dict[str, object]:
        return {
            "do_sample": bool(self.do_sample),
            "seed": int(self.seed),
            "temperature": float(self.temperature),
            "candidate_sampling": ("semantic_prefix_gumbel_topk_without_replacement" if self.do_sample
                                   else "model_logprob_topk"),
            "rng_key": "request_seed_and_complete_semantic_parent_token_prefix" if self.do_sample else None,
        }


@dataclass(frozen=True)
class DrafterSamplingContext:
    """Sampling bound to the committed prefix (``sampling.py:51-86``): a
    child's RNG key hashes committed_token_ids + relative_parent_path."""

    config: DrafterSamplingConfig
    committed_token_ids: tuple[int, ...]

    def __post_init__(self) -> None:
        self.config.validate()
        object.__setattr__(self, "committed_token_ids", tuple(int(t) for t in self.committed_token_ids))

    def seed_for_parent(self, relative_parent_path: Sequence[int]) -> int:
        path = (*self.committed_token_ids, *(int(t) for t in relative_parent_path))
        digest = hashlib.blake2b(digest_size=8)
        digest.update(_SAMPLING_SEED_DOMAIN)
        digest.update(struct.pack("<Q", int(self.config.seed) & ((1 << 64) - 1)))
        digest.update(struct.pack("<Q", len(path)))
        for token_id in path:
            if token_id < 0 or token_id > _TORCH_SEED_MASK:
                raise ValueError(f"token id is outside the supported int63 range: {token_id}")
            digest.update(struct.pack("<Q", token_id))
        return int.from_bytes(digest.digest(), "little") & _TORCH_SEED_MASK


def _normalize_logits(logits: torch.Tensor) -> torch.Tensor:
    if logits.ndim == 1:
        return logits.unsqueeze(0)
    if logits.ndim != 2:
        raise ValueError(f"expected 1D or 2D logits, got shape {tuple(logits.shape)}")
    return logits


def gumbel_proposal(rows: torch.Tensor, sampling: DrafterSamplingContext,
                    relative_parent_paths: Sequence[Sequence[int]]) -> torch.Tensor:
    """Proposal scores x / temperature + Gumbel noise, one fresh generator per
    parent (``sampling.py:135-152``), as float32 [rows, V]."""
    vocab = int(rows.shape[1])
    temperature = float(sampling.config.temperature)
    out = torch.empty((int(rows.shape[0]), vocab), dtype=torch.float32, device=rows.device)
    for r, path in enumerate(relative_parent_paths):
        gen = torch.Generator(device=rows.device)
        gen.manual_seed(sampling.seed_for_parent(path))
        u = torch.rand((vocab,), device=rows.device, dtype=torch.float32, generator=gen)
        u = u.clamp_min(torch.finfo(torch.float32).tiny)
        out[r] = rows[r].to(torch.float32) / temperature + (-torch.log(-torch.log(u)))
    return out


def batch_parent_token_candidates(logits: torch.Tensor, *, k: int, sampling: DrafterSamplingContext | None,
                                  relative_parent_paths: Sequence[Sequence[int]]
                                  ) -> tuple[torch.Tensor, torch.Tensor]:
    """(token_logprobs [B, k] in the logits dtype, token_ids [B, k]) per parent
    row (``sampling.py:107-153``): the top-k of log_softmax(row), equal
    log-probs in ascending token order; with do_sample the top-k of the Gumbel
    proposal, log-probs gathered from the model distribution."""
    if k <= 0:
        raise ValueError("k must be positive")
    rows = _normalize_logits(logits)
    if len(relative_parent_paths) != int(rows.shape[0]):
        raise ValueError("relative_parent_paths must contain one semantic path per logits row")
    proposal = None
    if sampling is not None and sampling.config.do_sample:
        proposal = gumbel_proposal(rows, sampling, relative_parent_paths)
    token_lp, token_ids, _, _, _ = frontier_topk(rows, k, proposal=proposal)
    return token_lp, token_ids


def single_parent_token_candidates(logits: torch.Tensor, *, k: int, sampling: DrafterSamplingContext | None,
                                   relative_parent_path: Sequence[int] = ()) -> tuple[torch.Tensor, torch.Tensor]:
    rows = _normalize_logits(logits)
    if int(rows.shape[0]) != 1:
        raise ValueError("single-parent candidate selection expects exactly one logits row")
    lp, ids = batch_parent_token_candidates(rows, k=k, sampling=sampling,
                                            relative_parent_paths=(tuple(relative_parent_path),))
    return lp[0], ids[0]
