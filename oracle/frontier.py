"""Oracle: one Drafter frontier depth -- per-parent top-k, candidates, stable
order, selection and the packed records (numpy).

Test infrastructure only (see oracle/__init__.py).  Restates
flashinfer_paged/sampling.py:107-153 (log_softmax, topk; the Gumbel proposal
path), flashinfer_paged/frontier.py:127-185 (candidate batch), :188-265 (the
packed int64 records), flashinfer_paged/utils.py:46-123 (stable multi-key
order by successive stable argsorts, global and per-root top-n) and
utils.py:27-43 (the Python-object ordering the device order must equal).

log_softmax is rounded to the logits dtype the way torch's 16-bit kernel
returns it: (x - max) - log(sum exp(x - max)) in fp32, then one rounding.
torch.topk leaves the order of equal values unspecified; the oracle (like the
kernels) puts equal log-probs in ascending token order.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np

from .rope import round_to


def log_softmax_rounded(logits: np.ndarray, dtype: str) -> np.ndarray:
    """logits [rows, V] (values of the dtype as fp32) -> log-probs, fp32
    holding values of the dtype ("f32": no rounding)."""
    x = np.asarray(logits, dtype=np.float32)
    m = x.max(axis=-1, keepdims=True)
    s = np.exp((x - m).astype(np.float64)).sum(axis=-1, keepdims=True)
    lse = np.log(s).astype(np.float32)
    lp = ((x - m).astype(np.float32) - lse).astype(np.float32)
    return lp if dtype == "f32" else round_to(lp, dtype)


def topk_rows(values: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """Per row, the k largest values (descending, equal values by ascending
    index): (values [rows, k], indices [rows, k] int64)."""
    v = np.asarray(values)
    k = min(int(k), v.shape[-1])
    idx = np.argsort(-v, axis=-1, kind="stable")[:, :k]
    return np.take_along_axis(v, idx, axis=-1), idx.astype(np.int64)


def parent_token_candidates(logits: np.ndarray, k: int, dtype: str,
                            proposal: np.ndarray | None = None) -> tuple[np.ndarray, np.ndarray]:
    """batch_parent_token_candidates: top-k of the log-probs, or (with Gumbel
    proposal scores) the top-k of the proposal with the log-probs gathered."""
    lp = log_softmax_rounded(logits, dtype)
    if proposal is None:
        return topk_rows(lp, k)
    _, ids = topk_rows(np.asarray(proposal, dtype=np.float32), k)
    return np.take_along_axis(lp, ids, axis=-1), ids


def build_candidates(route_ids: Sequence[int], root_ids: Sequence[int], parent_logprobs: Sequence[float],
                     token_logprobs: np.ndarray, token_ids: np.ndarray) -> dict[str, np.ndarray]:
    """build_pending_candidate_batch's columns (row-major over parents)."""
    b, k = token_ids.shape
    parent_lp = np.repeat(np.asarray(parent_logprobs, dtype=np.float64), k)
    return {
        "parent_route_ids": np.repeat(np.asarray(route_ids, dtype=np.int64), k),
        "stage1_root_ids": np.repeat(np.asarray(root_ids, dtype=np.int64), k),
        "parent_row_indices": np.repeat(np.arange(b, dtype=np.int64), k),
        "pending_token_ids": token_ids.reshape(-1).astype(np.int64),
        "cumulative_logprobs": parent_lp + token_logprobs.reshape(-1).astype(np.float64),
        "parent_logprobs": parent_lp,
        "ranks_in_parent": np.tile(np.arange(k, dtype=np.int64), b),
    }


def _stable_argsort(values: np.ndarray, descending: bool) -> np.ndarray:
    v = np.asarray(values)
    if not descending:
        return np.argsort(v, kind="stable")
    if v.dtype.kind == "f":
        # torch puts NaN above every number; -0.0 equals 0.0
        key = np.where(np.isnan(v), -np.inf, -v)
        nan_first = np.isnan(v)
        order = np.argsort(key, kind="stable")
        return np.concatenate((order[nan_first[order]], order[~nan_first[order]]))
    return np.argsort(-v, kind="stable")


def stable_order(c: dict[str, np.ndarray], include_stage1_root: bool = False) -> np.ndarray:
    """Successive stable argsorts from the least to the most significant key:
    token, rank, parent route (ascending), cumulative log-prob (descending),
    then stage-1 root (ascending)."""
    order = np.arange(len(c["pending_token_ids"]), dtype=np.int64)
    keys = [(c["pending_token_ids"], False), (c["ranks_in_parent"], False), (c["parent_route_ids"], False),
            (c["cumulative_logprobs"], True)]
    if include_stage1_root:
        keys.append((c["stage1_root_ids"], False))
    for values, desc in keys:
        order = order[_stable_argsort(values[order], desc)]
    return order


def select_global(c: dict[str, np.ndarray], num_selected: int) -> np.ndarray:
    return stable_order(c)[: min(int(num_selected), len(c["pending_token_ids"]))]


def select_per_root(c: dict[str, np.ndarray], num_selected: int,
                    root_candidate_counts: Sequence[tuple[int, int]]) -> np.ndarray:
    counts = sorted((int(r), int(n)) for r, n in root_candidate_counts)
    if sum(n for _, n in counts) != len(c["pending_token_ids"]):
        raise ValueError("root candidate counts do not cover the candidate batch")
    order = stable_order(c, include_stage1_root=True)
    parts, off = [], 0
    for _, n in counts:
        parts.append(order[off: off + min(int(num_selected), n)])
        off += n
    return np.concatenate(parts) if parts else order[:0]


def pack_records(c: dict[str, np.ndarray], selected: np.ndarray,
                 node_ids: Sequence[int] | None = None) -> np.ndarray:
    """The [count + nodes, 8] int64 records of materialize_pending_candidate_batch."""
    n = len(c["pending_token_ids"])
    order_col = np.full(n, -1, dtype=np.int64)
    order_col[np.asarray(selected, dtype=np.int64)] = np.arange(len(selected), dtype=np.int64)
    rec = np.stack((np.zeros(n, np.int64), c["parent_route_ids"], c["stage1_root_ids"], c["pending_token_ids"],
                    c["ranks_in_parent"], c["cumulative_logprobs"].astype(np.float64).view(np.int64),
                    c["parent_logprobs"].astype(np.float64).view(np.int64), order_col), axis=1)
    if node_ids:
        nodes = np.zeros((len(node_ids), 8), dtype=np.int64)
        nodes[:, 0] = 1
        nodes[:, 1] = np.asarray(node_ids, dtype=np.int64)
        rec = np.concatenate((rec, nodes), axis=0)
    return rec


def python_order(c: dict[str, np.ndarray]) -> list[int]:
    """global_topk_candidates' order (utils.py:27-43): sorted by (cumulative,
    -parent, -rank, -token), reverse=True, on Python objects."""
    rows = list(range(len(c["pending_token_ids"])))
    return sorted(rows, key=lambda i: (float(c["cumulative_logprobs"][i]), -int(c["parent_route_ids"][i]),
                                       -int(c["ranks_in_parent"][i]), -int(c["pending_token_ids"][i])),
                  reverse=True)
