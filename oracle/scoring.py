"""Oracle: Target route scoring and selection (numpy + pure Python).

Test infrastructure only (see oracle/__init__.py).
"""

from __future__ import annotations

import hashlib
import math
from typing import Sequence

import numpy as np


def log_softmax(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    m = x.max(axis=-1, keepdims=True)
    return x - m - np.log(np.exp(x - m).sum(axis=-1, keepdims=True))


def route_token_logprobs(
    paths: Sequence[Sequence[int]],
    route_nodes: Sequence[Sequence[int]],
    prefix_logits: np.ndarray,
    verify_logits: np.ndarray,
) -> list[list[float]]:
    """_score_routes, target_runtime.py:732-742: the first token reads the
    prefix logits, token t > 0 reads the verify row of the route's node t - 1."""
    plp = log_softmax(prefix_logits)
    vlp = log_softmax(verify_logits)
    out = []
    for path, nodes in zip(paths, route_nodes):
        row = []
        for t, tok in enumerate(path):
            row.append(float(plp[int(tok)]) if t == 0 else float(vlp[int(nodes[t - 1]), int(tok)]))
        out.append(row)
    return out


def normalise_weights(weights: Sequence[float] | None) -> tuple[float, ...] | None:
    """_validate_score_weights, target_runtime.py:362-374."""
    if weights is None:
        return None
    values = tuple(float(v) for v in weights)
    if not values:
        return None
    if any(v < 0.0 for v in values):
        raise ValueError("score weights must be non-negative")
    total = sum(values)
    if total <= 0.0:
        raise ValueError("at least one score weight must be positive")
    return tuple(v / total for v in values)


def select_best(scores: Sequence[dict]) -> dict:
    """target_best, target_runtime.py:444-451: max over
    (selection score, draft path logprob, -route_id)."""
    return max(scores, key=lambda s: (s["selection_score"], s["draft_path_logprob"], -s["route_id"]))


def sample_route(scores: Sequence[dict], seed: int, round_index: int, temperature: float = 1.0) -> tuple[dict, float]:
    """target_sample, target_runtime.py:454-546: canonical ordering, softmax of
    scaled scores, SHA-256 seeded uniform draw, inverse-CDF pick."""
    ordered = sorted(scores, key=lambda s: (tuple(s["token_ids"]), s["draft_path_logprob"], s["selection_score"],
                                            s["route_id"]))
    logits = [s["selection_score"] / temperature for s in ordered]
    pos_inf = [math.isinf(v) and v > 0 for v in logits]
    if any(pos_inf):
        probs = [1.0 / sum(pos_inf) if f else 0.0 for f in pos_inf]
    else:
        finite = [v for v in logits if math.isfinite(v)]
        if not finite:
            probs = [1.0 / len(ordered)] * len(ordered)
        else:
            mx = max(finite)
            w = [0.0 if v == -math.inf else math.exp(v - mx) for v in logits]
            probs = [x / sum(w) for x in w]
    material = f"atlas0709-target-route-sample-v1:{int(seed)}:{int(round_index)}".encode("utf-8")
    draw = (int.from_bytes(hashlib.sha256(material).digest()[:8], "big") + 0.5) / float(1 << 64)
    cum = 0.0
    idx = len(ordered) - 1
    for i, p in enumerate(probs):
        if draw < cum + p or i == len(ordered) - 1:
            idx = i
            break
        cum += p
    return ordered[idx], draw


def truncate_path(token_ids: Sequence[int], node_ids: Sequence[int], max_tokens: int | None,
                  eos_token_id: int | None) -> tuple[tuple[int, ...], tuple[int, ...]]:
    """_truncate_selected_path, target_runtime.py:675-700."""
    if len(token_ids) != len(node_ids) or not token_ids:
        raise ValueError("selected path tokens and node ids must have equal non-zero length")
    limit = len(token_ids) if max_tokens is None else min(len(token_ids), int(max_tokens))
    if limit <= 0:
        raise ValueError("selected_path_max_tokens must be positive")
    toks = [int(t) for t in token_ids[:limit]]
    if eos_token_id is not None:
        for i, t in enumerate(toks):
            if t == int(eos_token_id):
                toks = toks[: i + 1]
                break
    return tuple(toks), tuple(int(n) for n in node_ids[: len(toks)])
