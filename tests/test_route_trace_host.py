"""Drafter fork / COW / promote / prune / EXTEND traces through the route-pool
bridge on host pools, checked against what the operations fix:

* every live route's slot path holds the value ids of its committed prefix
  followed by its own nodes (no COW contamination, no lost copy);
* the committed prefix holds the prefix's value ids;
* owned pages and the allocator's free pages partition the pool (no leak, no
  double free);
* every route passes ``validate_route_physical_state`` (page layout,
  ownership, request row == slot path);
* COW copies happen exactly where two writers share a partial tail page.
"""

import pytest
import torch

from helpers import pkg
from oracle.route_pool import OracleAllocator, OracleReqPool


def _run(plans, page_size, num_pages, check):
    dw = pkg("drafter_workload")
    alloc = OracleAllocator(num_pages=num_pages, page_size=page_size)
    rows = OracleReqPool(size=128, max_context_len=4096)
    wl = dw.DrafterForkWorkload(plans=plans, req_pool=rows, allocator=alloc, page_size=page_size, device="cpu",
                                writer=lambda s, v: alloc.kv.write(s.cpu().numpy(), v.numpy()),
                                use_page_attention_metadata=False)
    wl.run(lambda phase: check(wl, alloc, rows, phase))
    return wl, alloc


def _invariants(wl, alloc, rows, phase):
    ps = wl.page_size
    owned_all = set()
    for req in wl.requests:
        b = req.bridge
        pre = b.prefix_slot_ids.tolist()
        assert alloc.kv.values[pre].tolist() == req.prefix_value_ids[: len(pre)], phase
        for r in req.active:
            if int(r.route_id) not in b.route_slot_paths:
                continue  # not yet decoded since its fork
            path = b.route_slot_paths[int(r.route_id)].tolist()
            assert alloc.kv.values[path].tolist() == wl.expected_path_values(req, r), (phase, r.route_id)
            b.validate_route_physical_state(r)
        b._materialize_pending_owned_pages()
        owned = set(b.owned_page_ids)
        assert not (owned & owned_all), f"{phase}: page owned by two requests"
        owned_all |= owned
    free = alloc.free_pages
    assert len(free) == len(set(free)), f"{phase}: duplicate free page"
    assert not (owned_all & set(free)), f"{phase}: page both owned and free"
    assert owned_all | set(free) == set(range(1, alloc.policy.num_pages + 1)), f"{phase}: leaked pages"


def test_config1_trace_invariants_and_cow_counts():
    dw = pkg("drafter_workload")
    wl, alloc = _run(dw.config1_plans(0), 16, 4096, _invariants)
    b = wl.requests[0].bridge
    # 3 routes fork at the 1000-token prefix, whose tail page holds 8 tokens:
    # 2 copies x 8 slots at the first frontier; nothing else is shared.
    first = alloc.kv.moves[0]
    assert len(first[0]) == 16 and first[1] == list(range(first[1][0], first[1][0] + 8)) * 2
    assert b.cow_pages_copied >= 2
    stats = wl.requests[0].stats
    assert stats[0]["committed_kv_tokens"] == 4 and stats[0]["retained_routes"] == 1


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_config5_trace_invariants(seed):
    dw = pkg("drafter_workload")
    plans = dw.config5_plans(8, 64, seed)
    wl, alloc = _run(plans, 64, 640, _invariants)
    for req in wl.requests:
        assert req.bridge.cow_pages_copied > 0
        commit = req.stats[0]
        assert commit["retained_routes"] == 3 and commit["released_kv_pages"] >= 0
        assert req.bridge.prefix_slot_count == req.plan.prefix_len + req.plan.commit_depth + len(req.plan.extend_tokens)


def test_planted_contamination_is_caught():
    """A move that writes a COW copy's source instead of its destination
    (dst and src swapped) must break the content invariant."""
    dw = pkg("drafter_workload")
    alloc = OracleAllocator(num_pages=4096, page_size=16)
    rows = OracleReqPool(size=16, max_context_len=2048)
    kv = alloc.kv
    real_move = kv.move_kv_cache

    def swapped(dst, src):
        real_move(src, dst)

    kv.move_kv_cache = swapped
    wl = dw.DrafterForkWorkload(plans=dw.config1_plans(0), req_pool=rows, allocator=alloc, page_size=16, device="cpu",
                                writer=lambda s, v: kv.write(s.cpu().numpy(), v.numpy()),
                                use_page_attention_metadata=False)
    with pytest.raises(AssertionError):
        wl.run(lambda phase: _invariants(wl, alloc, rows, phase))


def test_kv_pattern_is_device_independent_and_distinct():
    dw = pkg("drafter_workload")
    ids = torch.arange(1, 200)
    a = dw.kv_pattern(ids, 3, 1, 8, 64)
    assert a.dtype == torch.int16 and a.shape == (199, 8, 64)
    assert torch.equal(a, dw.kv_pattern(ids.flip(0), 3, 1, 8, 64).flip(0))
    assert not torch.equal(a, dw.kv_pattern(ids, 3, 0, 8, 64))
    rows = a.reshape(199, -1)
    assert len({tuple(r.tolist()) for r in rows}) == 199
