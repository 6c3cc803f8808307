"""The Drafter decode cascade plan, on the host.

For random forked page tables (families of routes that share leading full
pages, each route with its own tail pages, singles in between) every route
must attend to exactly its own keys, through its own page ids, once each,
whether a key is streamed by its group's shared-prefix items or by its own
tail item; every (group, KV head) merge item must combine exactly the partial
rows its items write, and no two merge items may share partial rows.  The
plan's install step is captured instead of uploading, so no GPU is needed."""

import math
import random
from collections import Counter, defaultdict

import torch
from hypothesis import HealthCheck, assume, given, settings
from hypothesis import strategies as st

from helpers import pkg

da = pkg("decode_attention")


def _plan(page_lists, last_lens, hq, hkv, d, ps, ws_bytes=1 << 26, split_target=None):
    """The cascade planner on host tensors, its install step captured; None
    when it declines (no two neighbouring routes share enough pages: the plan
    is then an ordinary one-request-per-route prefill plan)."""
    w = da.BatchDecodeWithPagedKVCacheWrapper(torch.empty(ws_bytes, dtype=torch.uint8))
    w._prefill.split_target_items = split_target
    captured = {}

    def install(**kw):
        captured.update(kw)

    w._prefill._install = install
    indptr = [0]
    for p in page_lists:
        indptr.append(indptr[-1] + len(p))
    indices = torch.tensor([x for p in page_lists for x in p], dtype=torch.int32)
    if not w._plan_cascade(torch.tensor(indptr, dtype=torch.int32), indices,
                           torch.tensor(last_lens, dtype=torch.int32), hq, hkv, d, ps, torch.float16, torch.float16,
                           None, True):
        return None
    return w, captured


def _check(w, cap, page_lists, last_lens, hq, hkv, ps):
    group = hq // hkv
    dec = cap["dec"]
    idx = cap["indices_src"].tolist()
    kv_lens = [(len(p) - 1) * ps + last if p else 0 for p, last in zip(page_lists, last_lens)]
    qo = dec["qo"]  # first route of each planned request (a group or a single route)
    seen = defaultdict(Counter)  # (route, kv head) -> Counter of (page id, offset)
    writes = defaultdict(Counter)  # (planned request, kv head) -> Counter of partial rows
    solo = set()
    for it in dec["work"]:
        gi, h, r0, nr, k0, k1, base = it[:7]
        first, n, keys, col, page_off = it[7:12]
        assert tuple(it[12:]) == (0, 0, 0, 0) and col == 0
        assert first == qo[gi] and 0 <= k0 <= k1 <= keys and nr > 0 and r0 % group == 0 and nr % group == 0
        assert 0 <= page_off and page_off + math.ceil(keys / ps) <= len(idx)
        routes = range(first + r0 // group, first + (r0 + nr) // group)
        assert routes.stop <= first + n
        for r in routes:
            for key in range(k0, k1):
                seen[(r, h)][(idx[page_off + key // ps], key % ps)] += 1
        if base < 0:
            solo.add((gi, h))
        else:
            for row in range(nr):
                writes[(gi, h)][base + row] += 1
    for r, (pages, kv) in enumerate(zip(page_lists, kv_lens)):
        own = Counter((pages[key // ps], key % ps) for key in range(kv))
        for h in range(hkv):
            assert seen[(r, h)] == own, f"route {r}, KV head {h}: keys not covered exactly once"
    # merge items: the partial rows of their items, exactly, disjoint
    regions = []
    merged = set()
    for m in range(dec["num_merge"]):
        gi, h, r0, rows, base, nsplit, z0, z1 = dec["meta"][dec["merge_off"] + 8 * m: dec["merge_off"] + 8 * m + 8]
        assert (r0, z0, z1) == (0, 0, 0) and (gi, h) not in solo and (gi, h) not in merged
        merged.add((gi, h))
        assert writes[(gi, h)] == Counter(range(base, base + nsplit * rows))
        regions.append((base, base + nsplit * rows))
    assert merged | solo == {(gi, h) for gi in range(len(qo) - 1) for h in range(hkv)}
    assert not (merged & solo)
    regions.sort()
    assert all(a1 <= b0 for (_, a1), (b0, _) in zip(regions, regions[1:]))
    assert dec["partial_rows"] == sum(e - s for s, e in regions)


@st.composite
def forked_tables(draw):
    """Families of routes sharing a random number of leading pages (each route
    keeps a prefix of the family's pages, then pages of its own), with single
    routes in between; page ids unique unless shared."""
    hq, hkv = draw(st.sampled_from([(32, 8), (8, 8), (16, 2), (32, 4)]))
    d = draw(st.sampled_from([64, 128]))
    ps = draw(st.sampled_from([1, 16, 64]))
    rng = random.Random(draw(st.integers(0, 1 << 30)))
    next_page = [1]

    def fresh(n):
        out = list(range(next_page[0], next_page[0] + n))
        next_page[0] += n
        return out

    page_lists, last_lens = [], []
    for _ in range(draw(st.integers(1, 5))):
        if rng.random() < 0.3:
            n_routes = 1
        else:
            n_routes = rng.randint(2, 12)
        family = fresh(rng.randint(0, 40))
        for _ in range(n_routes):
            keep = family[: rng.randint(max(0, len(family) - 3), len(family))]
            page_lists.append(keep + fresh(rng.randint(1, 3)))
            last_lens.append(rng.randint(1, ps))
    if len(page_lists) < 2:
        page_lists.append(fresh(2))
        last_lens.append(1)
    return page_lists, last_lens, hq, hkv, d, ps


@settings(max_examples=200, deadline=None, derandomize=True, suppress_health_check=[HealthCheck.too_slow])
@given(forked_tables(), st.sampled_from([None, 8, 64, 400]))
def test_cascade_plans_cover_each_route_exactly_once(table, split_target):
    page_lists, last_lens, hq, hkv, d, ps = table
    planned = _plan(page_lists, last_lens, hq, hkv, d, ps, split_target=split_target)
    assume(planned is not None)
    _check(*planned, page_lists, last_lens, hq, hkv, ps)


def test_forked_routes_form_one_cascade_group():
    """Nine routes over a 20-page shared prefix, each with its own tail page:
    one cascade group, the prefix streamed once per KV head (in splits), one
    tail item per route and KV head."""
    shared = list(range(100, 120))
    pages = [shared + [200 + r] for r in range(9)]
    w, cap = _plan(pages, [5] * 9, 32, 8, 128, 16)
    assert w.cascade_groups == 1
    _check(w, cap, pages, [5] * 9, 32, 8, 16)
    tails = [it for it in cap["dec"]["work"] if it[3] == 4]  # one route's GQA rows
    assert len(tails) == 9 * 8


def test_cascade_declines_routes_without_shared_pages():
    """Routes with distinct pages, or sharing fewer leading full pages than
    the cascade minimum, are left to the one-request-per-route plan."""
    pages = [[10 + 3 * r, 11 + 3 * r, 12 + 3 * r] for r in range(4)]
    assert _plan(pages, [7, 1, 16, 3], 32, 8, 128, 16) is None
    one_shared = [[5, 10 + r, 20 + r] for r in range(4)]
    assert _plan(one_shared, [3] * 4, 32, 8, 128, 16) is None
    two_shared = [[5, 6, 20 + r] for r in range(4)]
    assert _plan(two_shared, [3] * 4, 32, 8, 128, 16) is not None
