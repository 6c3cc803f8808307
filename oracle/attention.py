"""Oracle: ancestor-masked paged attention in closed form (numpy).

Test infrastructure only (see oracle/__init__.py).  Restates what the
reference's FlashInfer call computes (flashinfer_full_verify.py:953-985 plan
with causal=False and custom_mask, :1223 run): for each request, the keys are
the first kv_len rows of its pages (kv_indices[kv_indptr[b]:kv_indptr[b+1]],
page-major, page_size rows per page), and for query row q and head h

    s = (Q[q, h] . K[:, h // group]) * sm_scale,  s[~mask[q]] = -inf
    O[q, h] = softmax(s) . V[:, h // group],  lse[q, h] = log(sum(exp(s)))

with sm_scale = 1/sqrt(D) (FlashInfer's default when none is given) and a
natural-log LSE.  A fully masked row gives O = 0 and lse = -inf.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np


def gather_request_kv(kv_cache: np.ndarray, pages: Sequence[int], kv_len: int) -> tuple[np.ndarray, np.ndarray]:
    """[pages, 2, ps, H, D] -> K, V of shape [kv_len, H, D]."""
    sel = kv_cache[np.asarray(pages, dtype=np.int64)]
    ps = kv_cache.shape[2]
    h, d = kv_cache.shape[3], kv_cache.shape[4]
    k = sel[:, 0].reshape(len(pages) * ps, h, d)[:kv_len]
    v = sel[:, 1].reshape(len(pages) * ps, h, d)[:kv_len]
    return k, v


def masked_attention(
    q: np.ndarray,
    kv_cache: np.ndarray,
    qo_indptr: Sequence[int],
    kv_indptr: Sequence[int],
    kv_indices: Sequence[int],
    kv_last_page_len: Sequence[int],
    *,
    masks: Sequence[np.ndarray | None] | None = None,
    causal: bool = False,
    sm_scale: float | None = None,
    dtype=np.float64,
) -> tuple[np.ndarray, np.ndarray]:
    """Returns (O [nnz, Hq, D], lse [nnz, Hq]) in ``dtype``.

    ``masks[b]`` is the request's dense bool mask [qo_len, kv_len] (None =
    all visible).  ``causal`` makes key p visible to row i iff
    p <= kv_len - qo_len + i.
    """
    nnz, hq, d = q.shape
    hkv = kv_cache.shape[3]
    group = hq // hkv
    scale = (1.0 / np.sqrt(d)) if sm_scale is None else float(sm_scale)
    ps = kv_cache.shape[2]
    out = np.zeros((nnz, hq, d), dtype=dtype)
    lse = np.full((nnz, hq), -np.inf, dtype=dtype)
    batch = len(qo_indptr) - 1
    for b in range(batch):
        q0, q1 = int(qo_indptr[b]), int(qo_indptr[b + 1])
        pages = list(kv_indices[int(kv_indptr[b]) : int(kv_indptr[b + 1])])
        if q1 == q0 or not pages:
            continue
        kv_len = (len(pages) - 1) * ps + int(kv_last_page_len[b])
        k, v = gather_request_kv(kv_cache, pages, kv_len)
        k = k.astype(dtype)
        v = v.astype(dtype)
        qo = q1 - q0
        if masks is not None and masks[b] is not None:
            mask = np.asarray(masks[b], dtype=bool).reshape(qo, kv_len)
        elif causal:
            mask = np.arange(kv_len)[None, :] <= (kv_len - qo + np.arange(qo))[:, None]
        else:
            mask = np.ones((qo, kv_len), dtype=bool)
        qb = q[q0:q1].astype(dtype)
        for h in range(hkv):
            qg = qb[:, h * group : (h + 1) * group, :].reshape(qo * group, d)
            s = (qg @ k[:, h, :].T) * scale
            mg = np.repeat(mask, group, axis=0)
            s = np.where(mg, s, -np.inf)
            m = s.max(axis=1, keepdims=True)
            dead = ~np.isfinite(m[:, 0])
            m = np.where(np.isfinite(m), m, 0.0)
            p = np.exp(s - m)
            l = p.sum(axis=1, keepdims=True)
            o = (p @ v[:, h, :]) / np.where(l > 0, l, 1.0)
            o[dead] = 0.0
            ls = (m + np.log(np.where(l > 0, l, 1.0)))[:, 0]
            ls[dead] = -np.inf
            out[q0:q1, h * group : (h + 1) * group, :] = o.reshape(qo, group, d)
            lse[q0:q1, h * group : (h + 1) * group] = ls.reshape(qo, group)
    return out, lse
