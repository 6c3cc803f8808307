"""Seeded synthetic inputs of the paged-KV tree path's benchmark configurations.

Every generator draws from ``torch.Generator`` seeds so the HIP path and the
CPU checker see identical inputs.  Geometry names:

* ``LLAMA_8B``  -- 32 layers, 32 query heads, 8 KV heads, head_dim 128;
* ``LLAMA_1B``  -- 16 layers, 32 query heads, 8 KV heads, head_dim 64.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Sequence

import torch

VOCAB = 128256


@dataclass(frozen=True)
class Geometry:
    layers: int
    q_heads: int
    kv_heads: int
    head_dim: int

    @property
    def group(self) -> int:
        return self.q_heads // self.kv_heads

    def token_bytes(self, elem: int = 2) -> int:
        """K + V bytes of one token in one layer."""
        return 2 * self.kv_heads * self.head_dim * elem


LLAMA_8B = Geometry(32, 32, 8, 128)
LLAMA_1B = Geometry(16, 32, 8, 64)


def tree_routes(seed: int, k: int = 3, depth: int = 4) -> list[tuple[int, ...]]:
    """k independent routes of ``depth`` random token ids (no shared prefix)."""
    gen = torch.Generator().manual_seed(seed)
    return [tuple(int(x) for x in torch.randint(0, VOCAB, (depth,), generator=gen)) for _ in range(k)]


def forest_routes(seed: int, k: int = 3, depth: int = 4) -> list[tuple[int, ...]]:
    """k * k routes by seeded branching: k stage-1 roots, each forking into k
    routes that share a random-length prefix (0 .. depth-1 tokens) with their
    root.  Deduplication leaves at most k * k * depth nodes."""
    gen = torch.Generator().manual_seed(seed)
    roots = [[int(x) for x in torch.randint(0, VOCAB, (depth,), generator=gen)] for _ in range(k)]
    routes = []
    for i in range(k):
        for _ in range(k):
            shared = int(torch.randint(0, depth, (1,), generator=gen))
            tail = [int(x) for x in torch.randint(0, VOCAB, (depth - shared,), generator=gen)]
            routes.append(tuple(roots[i][:shared] + tail))
    return routes


@dataclass
class PagedTargetKV:
    """One request's Target KV in a paged pool, all layers in one allocation.

    ``pool[l]`` is layer l's page view: ``[pool_pages, 2, page_size, Hkv, D]``
    ("NHD") or ``[pool_pages, 2, Hkv, page_size, D]`` ("HND", each KV head's
    keys of a page contiguous); the request's pages are ``kv_indices`` (a
    random permutation of pool pages).
    """

    pool: torch.Tensor  # [L, pool_pages, 2, ps, Hkv, D] or [L, pool_pages, 2, Hkv, ps, D]
    kv_indices: torch.Tensor  # int32 [pages]
    page_size: int
    kv_layout: str = "NHD"

    @property
    def layers(self) -> list[torch.Tensor]:
        return list(self.pool.unbind(0))

    def nhd_layer(self, l: int) -> torch.Tensor:
        """Layer l as an ``[pool_pages, 2, page_size, Hkv, D]`` view."""
        return self.pool[l] if self.kv_layout == "NHD" else self.pool[l].permute(0, 1, 3, 2, 4)


def make_paged_target_kv(
    geom: Geometry,
    *,
    kv_len: int,
    page_size: int,
    dtype: torch.dtype,
    device: torch.device,
    seed: int = 0,
    spare_pages: int = 0,
    scale: float = 0.1,
    kv_layout: str = "NHD",
) -> PagedTargetKV:
    """The values depend on the seed only: an "HND" pool holds the same keys
    and values as the "NHD" pool of the same seed."""
    if kv_layout not in ("NHD", "HND"):
        raise ValueError(f"kv_layout must be 'NHD' or 'HND', got {kv_layout!r}")
    pages = math.ceil(kv_len / page_size)
    pool_pages = pages + spare_pages
    gen = torch.Generator(device=device).manual_seed(seed)
    nhd = (pool_pages, 2, page_size, geom.kv_heads, geom.head_dim)
    page = nhd if kv_layout == "NHD" else (pool_pages, 2, geom.kv_heads, page_size, geom.head_dim)
    kv = PagedTargetKV(pool=torch.empty((geom.layers,) + page, dtype=dtype, device=device), kv_indices=None,
                       page_size=page_size, kv_layout=kv_layout)
    for l in range(geom.layers):
        kv.nhd_layer(l).copy_(torch.randn(nhd, generator=gen, device=device, dtype=torch.float32) * scale)
    perm_gen = torch.Generator().manual_seed(seed + 1)
    kv.kv_indices = torch.randperm(pool_pages, generator=perm_gen)[:pages].to(torch.int32).to(device)
    return kv


def random_queries(geom: Geometry, n: int, *, dtype: torch.dtype, device: torch.device, seed: int,
                   scale: float = 0.1) -> list[torch.Tensor]:
    gen = torch.Generator(device=device).manual_seed(seed)
    return [
        (torch.randn((n, geom.q_heads, geom.head_dim), generator=gen, device=device) * scale).to(dtype)
        for _ in range(geom.layers)
    ]


def verify_attention_bytes(geom: Geometry, *, kv_len: int, nodes: int, page_size: int, elem: int = 2) -> int:
    """Algorithmic HBM bytes of one layer's verify attention: K and V of every
    key once, Q read and O written once, fp32 LSE, page indices, one 64-bit
    ancestor mask word per node."""
    kv = kv_len * geom.kv_heads * geom.head_dim * elem * 2
    qo = 2 * nodes * geom.q_heads * geom.head_dim * elem
    return kv + qo + nodes * geom.q_heads * 4 + 4 * math.ceil(kv_len / page_size) + 8 * nodes


def verify_attention_flops(geom: Geometry, visible_keys: Sequence[int]) -> int:
    """4 * Hq * D flops per visible (query, key) pair (QK^T and PV)."""
    return 4 * geom.q_heads * geom.head_dim * int(sum(visible_keys))


@dataclass
class BatchedVerifyCase:
    """Host description of the batched Target verify (32 requests, 8B
    geometry, page 16): per request a committed prefix, a k=3 d=4 tree of
    independent routes, its pages scattered over a pool, and the route its
    commit selects.  ``page_ids`` lists every request's pages in request
    order (request b's pages are ``page_ids[kv_indptr[b]:kv_indptr[b + 1]]``)."""

    page_size: int
    pool_pages: int
    prefixes: list[int]
    routes: list[list[tuple[int, ...]]]
    nodes: list[int]
    kv_lens: list[int]
    req_pages: list[int]
    kv_indptr: list[int]
    qo_indptr: list[int]
    page_ids: torch.Tensor  # int64 [sum(req_pages)], distinct pool pages
    selected: list[int]  # route index committed per request

    @property
    def need_pages(self) -> int:
        return self.kv_indptr[-1]


def batched_verify_need_pages(*, requests: int = 32, page_size: int = 16, seed: int = 4, min_prefix: int = 1024,
                              max_prefix: int = 16384) -> int:
    """Pages the batched verify's requests occupy (to size its pool)."""
    gen = torch.Generator().manual_seed(seed)
    prefixes = [int(x) for x in torch.randint(min_prefix, max_prefix + 1, (requests,), generator=gen)]
    nodes = [len({tuple(r[: i + 1]) for r in tree_routes(100 + b) for i in range(len(r))}) for b in range(requests)]
    return sum(math.ceil((p + n) / page_size) for p, n in zip(prefixes, nodes))


def batched_verify_case(*, pool_pages: int, requests: int = 32, page_size: int = 16, seed: int = 4,
                        min_prefix: int = 1024, max_prefix: int = 16384) -> BatchedVerifyCase:
    """Seeded batched verify: prefixes uniform in [min_prefix, max_prefix],
    routes ``tree_routes(100 + b)`` (12 nodes after dedup), pages drawn
    without replacement from ``pool_pages`` by a random permutation, and a
    uniformly drawn route to commit per request."""
    gen = torch.Generator().manual_seed(seed)
    prefixes = [int(x) for x in torch.randint(min_prefix, max_prefix + 1, (requests,), generator=gen)]
    routes = [tree_routes(100 + b) for b in range(requests)]
    nodes = [len({tuple(r[: i + 1]) for r in rs for i in range(len(r))}) for rs in routes]
    kv_lens = [p + n for p, n in zip(prefixes, nodes)]
    req_pages = [math.ceil(k / page_size) for k in kv_lens]
    kv_indptr = [0]
    for n in req_pages:
        kv_indptr.append(kv_indptr[-1] + n)
    qo_indptr = [0]
    for n in nodes:
        qo_indptr.append(qo_indptr[-1] + n)
    if kv_indptr[-1] > pool_pages:
        raise ValueError(f"pool of {pool_pages} pages is smaller than the {kv_indptr[-1]} pages requested")
    page_ids = torch.randperm(pool_pages, generator=gen)[: kv_indptr[-1]]
    selected = [int(torch.randint(0, len(r), (1,), generator=gen)) for r in routes]
    return BatchedVerifyCase(page_size=page_size, pool_pages=pool_pages, prefixes=prefixes, routes=routes,
                             nodes=nodes, kv_lens=kv_lens, req_pages=req_pages, kv_indptr=kv_indptr,
                             qo_indptr=qo_indptr, page_ids=page_ids, selected=selected)
