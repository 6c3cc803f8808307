"""Route-pool bridge on the native HIP pools vs the same trace on host pools:
slot paths, leases, request rows, owned pages, the allocator's free list and
every live slot's K/V bytes (all layers) must be identical at every phase.
Both runs must also hold, at every phase, the invariants the allocator's
arithmetic fixes (free, owned and padding pages partition the pool, no
duplicate free page, live slots on their own request's pages), and
configuration 1 must commit the route the Target's target_best order picks."""

import dataclasses

import pytest
import torch

from helpers import check_allocator_invariants, pkg
from oracle.route_pool import OracleAllocator, OracleReqPool
from oracle.scoring import select_best

pytestmark = pytest.mark.gpu


def _device_run(plans, *, page_size, num_pages, layers, heads, head_dim, dev, host_phases, batched=False):
    """Runs the trace on the native pools; after each phase compares the
    bookkeeping and the live slots' K/V bytes with the host run's phase.
    ``batched``: every decode step of all requests is one fused frontier step
    (one launch for the requests' slot paths, rows and page tables)."""
    dw = pkg("drafter_workload")
    npool = pkg("flashinfer_paged.native_pool")
    req, kv, alloc = npool.create_native_pools(num_pages=num_pages, page_size=page_size, dtype=torch.bfloat16,
                                               head_num=heads, head_dim=head_dim, layer_num=layers,
                                               max_running_requests=128, max_context_len=4096, device=dev)

    def writer(slots, vids):
        v = vids.to(dev)
        k_rows = [dw.kv_pattern(v, l, 0, heads, head_dim).view(torch.bfloat16) for l in range(layers)]
        v_rows = [dw.kv_pattern(v, l, 1, heads, head_dim).view(torch.bfloat16) for l in range(layers)]
        kv.set_kv_buffer_all_layers(slots, k_rows, v_rows)

    wl = dw.DrafterForkWorkload(plans=plans, req_pool=req, allocator=alloc, page_size=page_size, device=dev,
                                writer=writer, batched=batched)
    seen = []

    def compare(phase):
        torch.cuda.synchronize()
        i = len(seen)
        seen.append(phase)
        hphase, hs, values = host_phases[i]
        assert hphase == phase
        ds = _state(wl, alloc.free_pages.tolist(), req.req_to_token)
        _check_invariants(ds, num_pages, page_size, f"device run after {phase}")
        assert ds == hs, f"bookkeeping differs after {phase}"
        _check_kv(kv, values, _live_slots(hs), layers, heads, head_dim, dev, phase)

    wl.run(compare)
    assert seen == [p for p, _, _ in host_phases]
    return wl


def _host_run(plans, *, page_size, num_pages, phases):
    dw = pkg("drafter_workload")
    alloc = OracleAllocator(num_pages=num_pages, page_size=page_size)
    rows = OracleReqPool(size=128, max_context_len=4096)
    wl = dw.DrafterForkWorkload(plans=plans, req_pool=rows, allocator=alloc, page_size=page_size, device="cpu",
                                writer=lambda s, v: alloc.kv.write(s.numpy(), v.numpy()),
                                use_page_attention_metadata=False)
    candidates = []

    def record(phase):
        state = _state(wl, alloc.free_pages, rows.req_to_token)
        _check_invariants(state, num_pages, page_size, f"host run after {phase}")
        phases.append((phase, state, alloc.kv.values.copy()))
        if phase.startswith("decode"):
            # the routes the commit chooses among are the last stage-1 step's
            candidates[:] = [[(int(r.route_id), tuple(int(n) for n in r.kv_view.node_ids),
                               float(r.cumulative_logprob)) for r in q.active] for q in wl.requests]

    wl.run(record)
    wl.commit_candidates = candidates
    return wl


def _state(wl, free_pages, req_to_token):
    out = {"free": list(free_pages)}
    for i, r in enumerate(wl.requests):
        b = r.bridge
        b.check_pending_device_checks()
        rows = {}
        for rid, row in sorted(b.route_rows.items()):
            n = int(row.written_length)
            rows[rid] = (row.req_pool_index, n, row.pending_dirty_start,
                         req_to_token[row.req_pool_index, :n].cpu().tolist())
        b._materialize_pending_owned_pages()
        out[i] = {
            "prefix": b.prefix_slot_ids.cpu().tolist(),
            "paths": {rid: p.cpu().tolist() for rid, p in sorted(b.route_slot_paths.items())},
            "keys": dict(sorted(b.route_tail_page_keys.items())),
            "prefix_keys": (b.prefix_tail_page_key, dict(b.prefix_partial_tail_keys)),
            "rows": rows,
            "owned": sorted(set(b.owned_page_ids)),
            # page-index counts differ by design: the host run builds no page metadata
            "counters": {k: v for k, v in b.hot_path_counters().items() if k != "attention_metadata_page_indices"},
            "stats": list(r.stats),
        }
    return out


def _check_invariants(state, num_pages, page_size, where):
    reqs = [v for k, v in state.items() if k != "free"]
    live = [list(v["prefix"]) + [x for p in v["paths"].values() for x in p] for v in reqs]
    check_allocator_invariants(num_pages, state["free"], [v["owned"] for v in reqs], live, page_size, where)


def _live_slots(state):
    slots = set()
    for k, v in state.items():
        if k == "free":
            continue
        slots.update(v["prefix"])
        for p in v["paths"].values():
            slots.update(p)
    return sorted(slots)


def _check_kv(kv, values, slots, layers, heads, head_dim, dev, phase):
    dw = pkg("drafter_workload")
    s = torch.tensor(slots, dtype=torch.long, device=dev)
    ids = torch.tensor(values[slots], dtype=torch.long, device=dev)
    for l in range(layers):
        for which, buf in ((0, kv.k_buffer[l]), (1, kv.v_buffer[l])):
            got = buf[s].view(torch.int16)
            exp = dw.kv_pattern(ids, l, which, heads, head_dim)
            bad = (got != exp).reshape(len(slots), -1).any(-1)
            assert not bool(bad.any()), f"{phase}: layer {l} kv {which} differs at slots " \
                                        f"{s[bad][:8].tolist()}"


@pytest.mark.parametrize("case", ["config1", "config5_seed0", "config5_seed1", "config1_batched",
                                  "config5_seed0_batched", "config5_seed1_batched", "config5_seed2_batched",
                                  "config5_seed3_batched", "config5_ps16_seed4", "config5_ps16_seed5_batched"])
def test_route_pool_trace_matches_host_pools(dev, case):
    """The ``_batched`` cases run each decode step of all requests as one
    fused frontier step (and the commit, prune and EXTEND as one call each)
    against the same per-request host trace; the ``_ps16`` cases use pages of
    16 tokens."""
    dw = pkg("drafter_workload")
    batched = case.endswith("_batched")
    name = case.removesuffix("_batched")
    if name == "config1":
        plans, ps, pages = dw.config1_plans(0), 16, 4096
    else:
        # config5[_ps16]_seed<k>: the fork stress with pages of 64 (or 16) tokens
        ps = 16 if "_ps16_" in name else 64
        plans, pages = dw.config5_plans(8, ps, int(name.rsplit("seed", 1)[1])), 640 if ps == 64 else 2560
    layers, heads, head_dim = 16, 8, 64
    print(f"route-pool trace {case}: page_size {ps}, {pages} pages", flush=True)
    host = []
    hw = _host_run(plans, page_size=ps, num_pages=pages, phases=host)
    dw_run = _device_run(plans, page_size=ps, num_pages=pages, layers=layers, heads=heads, head_dim=head_dim,
                         dev=dev, host_phases=host, batched=batched)
    if batched:
        assert all(r.bridge.attention_metadata_builds > 0 for r in dw_run.requests)
    assert [r.selected_route_id for r in dw_run.requests] == [r.selected_route_id for r in hw.requests]
    if case == "config1":
        # the committed route is the best by (sum of node log-probs, draft
        # log-prob, -route id), recomputed from the candidates and node log-probs
        req = hw.requests[0]
        scores = [{"selection_score": sum(req.node_logprobs[n] for n in nodes), "draft_path_logprob": cum,
                   "route_id": rid} for rid, nodes, cum in hw.commit_candidates[0]]
        assert len(scores) == 3
        assert req.selected_route_id == select_best(scores)["route_id"]


@pytest.mark.parametrize("batched", [False, True])
def test_route_pool_trace_with_sweep_fallback_matches_host_pools(dev, monkeypatch, batched):
    """With the prune by paths out of reach (its path limit patched to 0),
    every prune takes the mark-and-sweep launches and its read-back a
    separate gather launch; the trace still matches the host pools phase by
    phase."""
    dw = pkg("drafter_workload")
    lib_mod = pkg("_lib")
    monkeypatch.setattr(lib_mod, "PRUNE_MAX_PATHS", 0)
    plans, ps, pages = dw.config5_plans(8, 64, 1), 64, 640
    print(f"route-pool trace with the sweep fallback, batched={batched}", flush=True)
    host = []
    hw = _host_run(plans, page_size=ps, num_pages=pages, phases=host)
    dw_run = _device_run(plans, page_size=ps, num_pages=pages, layers=4, heads=8, head_dim=64, dev=dev,
                         host_phases=host, batched=batched)
    assert [r.selected_route_id for r in dw_run.requests] == [r.selected_route_id for r in hw.requests]


def test_device_ownership_set_operations(dev):
    sr = pkg("flashinfer_paged.sglang_runtime")
    own = sr.DeviceOwnedPages(100, 16, dev)
    own.mark_slots(torch.tensor([0, 17, 33, 1599], device=dev))
    assert own == {0, 1, 2, 99}
    own.update({40, 41})
    own.difference_update([1])
    own.remove(99)
    assert sorted(own) == [0, 2, 40, 41] and 40 in own and 1 not in own and len(own) == 4
    freed = own.sweep(torch.tensor([32, 41 * 16 + 3], device=dev))
    assert freed.tolist() == [0, 40] and own == {2, 41}
    with pytest.raises(KeyError):
        own.remove(7)
    own.clear()
    assert own == set()


def test_frontier_page_metadata_matches_oracle(dev, monkeypatch):
    """The per-route host path of prepare_frontier (what a bridge over other
    pools runs; over the native pools a request's step goes through the
    multi-request launch, checked in test_fused_frontier_metadata_matches_oracle)."""
    from oracle import paged_kv as ref
    sr = pkg("flashinfer_paged.sglang_runtime")
    monkeypatch.setattr(sr, "fused_frontier_supported", lambda bridges: False)
    dw = pkg("drafter_workload")
    npool = pkg("flashinfer_paged.native_pool")
    req, kv, alloc = npool.create_native_pools(num_pages=640, page_size=64, dtype=torch.bfloat16, head_num=8,
                                               head_dim=64, layer_num=2, max_running_requests=128,
                                               max_context_len=4096, device=dev)
    specs = []

    def writer(slots, vids):
        rows = [torch.zeros((int(slots.numel()), 8, 64), dtype=torch.bfloat16, device=dev)] * 2
        kv.set_kv_buffer_all_layers(slots, rows, rows)

    wl = dw.DrafterForkWorkload(plans=dw.config5_plans(2, 64, 3), req_pool=req, allocator=alloc, page_size=64,
                                device=dev, writer=writer)
    orig = wl.requests[0].bridge.prepare_frontier

    def spy(routes, **kw):
        ids, md = orig(routes, **kw)
        paths = [wl.requests[0].bridge.route_slot_paths[int(r.route_id)].tolist() for r in routes]
        specs.append((md, paths))
        return ids, md

    wl.requests[0].bridge.prepare_frontier = spy
    wl.run()
    assert specs
    for md, paths in specs:
        exp = ref.paged_metadata(paths, 64)
        spec = md.paged_decode_spec
        assert spec.kv_indptr.tolist() == exp.kv_indptr
        assert spec.kv_indices.tolist() == exp.kv_page_indices
        assert spec.kv_last_page_len.tolist() == exp.kv_last_page_len
        assert md.seq_lens_cpu.tolist() == exp.seq_lens


def test_fused_frontier_metadata_matches_oracle(dev):
    """The union batch of a fused frontier step (4 requests): page tables
    equal the oracle's paged metadata of all routes' new slot paths in request
    order; input ids, sequence lengths, positions, request rows and decode
    slots match each route's state."""
    from oracle import paged_kv as ref
    dw = pkg("drafter_workload")
    npool = pkg("flashinfer_paged.native_pool")
    req, kv, alloc = npool.create_native_pools(num_pages=640, page_size=64, dtype=torch.bfloat16, head_num=8,
                                               head_dim=64, layer_num=2, max_running_requests=128,
                                               max_context_len=4096, device=dev)

    def writer(slots, vids):
        rows = [torch.zeros((int(slots.numel()), 8, 64), dtype=torch.bfloat16, device=dev)] * 2
        kv.set_kv_buffer_all_layers(slots, rows, rows)

    wl = dw.DrafterForkWorkload(plans=dw.config5_plans(4, 64, 5), req_pool=req, allocator=alloc, page_size=64,
                                device=dev, writer=writer, batched=True)
    ex = wl.requests[0].backend.executor
    orig = ex.forward_frontier
    steps = []

    def spy(*, input_ids, route_kv_metadata):
        md = route_kv_metadata
        routes = [(q, r) for q in wl.requests for r in q.active]
        assert int(md.out_cache_loc.numel()) == len(routes), "every request takes part in each step"
        paths = [q.bridge.route_slot_paths[int(r.route_id)].tolist() for q, r in routes]
        rows = [q.bridge.route_rows[int(r.route_id)].req_pool_index for q, r in routes]
        tokens = [int(r.pending_token_id) for _, r in routes]
        steps.append((md, input_ids.tolist(), paths, rows, tokens))
        return orig(input_ids=input_ids, route_kv_metadata=route_kv_metadata)

    ex.forward_frontier = spy
    wl.run()
    assert len(steps) == 10  # 8 stage-1 steps, one after the commit, one after the EXTEND
    for md, ids, paths, rows, tokens in steps:
        exp = ref.paged_metadata(paths, 64)
        spec = md.paged_decode_spec
        assert spec.kv_indptr.tolist() == exp.kv_indptr
        assert spec.kv_indices.tolist() == exp.kv_page_indices
        assert spec.kv_last_page_len.tolist() == exp.kv_last_page_len
        assert md.seq_lens_cpu.tolist() == exp.seq_lens == md.seq_lens.tolist()
        assert md.positions.tolist() == [n - 1 for n in exp.seq_lens]
        assert md.out_cache_loc.tolist() == [p[-1] for p in paths]
        assert md.req_pool_indices.tolist() == rows and ids == tokens
        assert md.seq_lens_sum == sum(exp.seq_lens) and md.page_index_count == len(exp.kv_page_indices)


@pytest.mark.parametrize("descriptors", ["device", "launch_arguments"])
def test_fused_frontier_rejects_out_of_range_descriptors(dev, descriptors):
    """A route descriptor whose request row lies outside the row table is
    skipped by the kernel's own range checks and reported in its check word;
    the in-range route of the same launch is written and its word is 0.  The
    same through both entry points: descriptors in device memory, and
    descriptors passed in the launch's arguments (which also writes the
    model inputs)."""
    import ctypes
    import numpy as np
    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    ps = 16
    path = torch.arange(32, 37, dtype=torch.int64, device=dev)  # 5 slots on page 2
    table = torch.zeros((4, 64), dtype=torch.int64, device=dev)
    free = torch.tensor([7, 8], dtype=torch.int64, device=dev)
    bitmap = torch.zeros(1, dtype=torch.int32, device=dev)
    desc = []
    for row in (1, 9):  # 9 is outside the 4-row table
        desc += [path.data_ptr(), 5, 0, -1, 0, -1, 0 if row == 1 else 6, 0 if row == 1 else 1, row, 0,
                 bitmap.data_ptr(), 0, 2]
    words = torch.full((2,), -5, dtype=torch.int64, device=dev)
    flat = torch.full((12,), -5, dtype=torch.int64, device=dev)
    out = torch.full((2,), -5, dtype=torch.int64, device=dev)
    i32 = torch.full((3 * 2 + 1 + 2,), -5, dtype=torch.int32, device=dev)
    batch = torch.full((10,), -5, dtype=torch.int64, device=dev)
    tail = (lib_mod.ptr(free), 2, ps, 32, lib_mod.ptr(table), 4, 64, lib_mod.ptr(flat), 12, lib_mod.ptr(out), None,
            None, 0, lib_mod.ptr(i32[:3]), lib_mod.ptr(i32[3:5]), lib_mod.ptr(i32[5:7]), lib_mod.ptr(i32[7:]), 2,
            lib_mod.ptr(words))
    print(f"fused frontier: out-of-range descriptor, {descriptors}", flush=True)
    if descriptors == "device":
        d = torch.tensor(desc, dtype=torch.int64, device=dev)
        rc = lib.atlas_pool_prepare_frontier(lib_mod.ptr(d), 2, *tail, lib_mod.stream_of(dev))
    else:
        host = np.asarray(desc + [11, 12] + [40, 41], dtype=np.int64)
        base = host.ctypes.data
        rc = lib.atlas_pool_prepare_frontier_host(base, base + 8 * 26, base + 8 * 28, 2, *tail, lib_mod.ptr(batch),
                                                  lib_mod.stream_of(dev))
    lib_mod.check(rc, "atlas_pool_prepare_frontier")
    torch.cuda.synchronize()
    assert words.tolist() == [0, lib_mod.FRONTIER_BAD_DESCRIPTOR]
    assert flat[:6].tolist() == [32, 33, 34, 35, 36, 37] and flat[6:].tolist() == [-5] * 6
    assert out.tolist() == [37, -5]
    assert table[1, :6].tolist() == [32, 33, 34, 35, 36, 37] and int(table[2:].abs().sum()) == 0
    assert i32[:2].tolist() == [0, 1] and i32[3].item() == 6 and i32[5].item() == 6 and i32[7].item() == 2
    assert bitmap.item() == 1 << 2
    if descriptors == "launch_arguments":
        # tokens, sequence lengths, positions, request rows, route ids
        assert batch.tolist() == [11, 12, 6, 6, 5, 5, 1, 9, 40, 41]
    else:
        assert batch.tolist() == [-5] * 10


def test_batched_extend_equals_per_request_calls_and_refusals(dev):
    """append_known_tokens_as_prefix_many over shared native pools against
    one append_known_tokens_as_prefix per request, from the same state (after
    stage 1, the commit and every request's prune): the same logits rows,
    prefix slots, prefix pages, owned pages, free list and counters.  Empty
    suffixes and mismatched list lengths are refused before any state
    changes."""
    dw = pkg("drafter_workload")
    npool = pkg("flashinfer_paged.native_pool")
    sr = pkg("flashinfer_paged.sglang_runtime")

    def setup():
        req, kv, alloc = npool.create_native_pools(num_pages=640, page_size=64, dtype=torch.bfloat16, head_num=8,
                                                   head_dim=64, layer_num=2, max_running_requests=128,
                                                   max_context_len=4096, device=dev)

        def writer(slots, vids):
            rows = [torch.zeros((int(slots.numel()), 8, 64), dtype=torch.bfloat16, device=dev)] * 2
            kv.set_kv_buffer_all_layers(slots, rows, rows)

        wl = dw.DrafterForkWorkload(plans=dw.config5_plans(4, 64, 7), req_pool=req, allocator=alloc, page_size=64,
                                    device=dev, writer=writer, batched=True)
        wl.prefill()
        wl.stage1()
        wl.commit()
        for r in wl.requests:
            r.bridge.retain_route_rows([])
            r.bridge.release_unreferenced_node_slots([])
        return wl, alloc

    def state(wl, alloc):
        torch.cuda.synchronize()
        return ([r.bridge.prefix_slot_ids.tolist() for r in wl.requests],
                [sorted(r.bridge.prefix_page_ids) for r in wl.requests],
                [sorted(r.bridge.owned_page_ids) for r in wl.requests],
                alloc.free_pages.tolist(), [r.bridge.hot_path_counters() for r in wl.requests],
                [r.backend.prefix_token_ids for r in wl.requests])

    suffixes = [(5, 6, 7, 8), (9,), (10, 11), (12, 13, 14, 15, 16)]
    wl, alloc = setup()
    backends = [r.backend for r in wl.requests]
    before = state(wl, alloc)
    with pytest.raises(ValueError):
        sr.SGLangFlashInferFrontierModelBackend.append_known_tokens_as_prefix_many(backends, suffixes[:3])
    with pytest.raises(ValueError):
        sr.SGLangFlashInferFrontierModelBackend.append_known_tokens_as_prefix_many(backends, [(1,), (), (2,), (3,)])
    assert state(wl, alloc) == before
    got = sr.SGLangFlashInferFrontierModelBackend.append_known_tokens_as_prefix_many(backends, suffixes)
    batched = state(wl, alloc)

    wl2, alloc2 = setup()
    ref = [r.backend.append_known_tokens_as_prefix(sfx) for r, sfx in zip(wl2.requests, suffixes)]
    assert state(wl2, alloc2) == batched
    assert len(got) == len(ref) and all(torch.equal(a, b) for a, b in zip(got, ref))
    for r, sfx in zip(wl.requests, suffixes):
        assert int(r.bridge.prefix_slot_ids.numel()) == len(r.backend.prefix_token_ids)
        assert r.backend.prefix_token_ids[-len(sfx):] == sfx


def test_batched_commit_equals_per_request_calls_and_refusals(dev):
    """commit_stage1_and_promote_many over shared native pools against one
    commit_stage1_and_promote per request, from the same state (after stage
    1): the same promoted routes and stats, prefix slots and pages, owned
    pages, node slots, request rows, free list and counters, and the same
    state again after the EXTEND phase's batched prunes.  Mismatched list
    lengths and a committed route with no materialized node are refused
    before any state changes."""
    dw = pkg("drafter_workload")
    npool = pkg("flashinfer_paged.native_pool")
    sr = pkg("flashinfer_paged.sglang_runtime")

    def setup(batched_commit):
        req, kv, alloc = npool.create_native_pools(num_pages=640, page_size=64, dtype=torch.bfloat16, head_num=8,
                                                   head_dim=64, layer_num=2, max_running_requests=128,
                                                   max_context_len=4096, device=dev)

        def writer(slots, vids):
            rows = [torch.zeros((int(slots.numel()), 8, 64), dtype=torch.bfloat16, device=dev)] * 2
            kv.set_kv_buffer_all_layers(slots, rows, rows)

        wl = dw.DrafterForkWorkload(plans=dw.config5_plans(5, 64, 11), req_pool=req, allocator=alloc, page_size=64,
                                    device=dev, writer=writer, batched=True)
        wl.prefill()
        wl.stage1()
        wl.batched = batched_commit
        return wl, alloc, req

    def state(wl, alloc, req):
        torch.cuda.synchronize()
        b = [r.bridge for r in wl.requests]
        return ([x.prefix_slot_ids.tolist() for x in b], [sorted(x.prefix_page_ids) for x in b],
                [x.prefix_slot_count for x in b], [sorted(x.owned_page_ids) for x in b],
                [sorted(x.node_slot_ids) for x in b], [sorted(x.route_rows) for x in b],
                [sorted(x.route_slot_paths) for x in b], [x.prefix_tail_page_key for x in b],
                alloc.free_pages.tolist(), list(req._free_rows), [x.hot_path_counters() for x in b],
                [r.backend.prefix_token_ids for r in wl.requests])

    wl, alloc, req = setup(True)
    backends = [r.backend for r in wl.requests]
    before = state(wl, alloc, req)
    picks = wl.select_commits()
    many = sr.SGLangFlashInferFrontierModelBackend.commit_stage1_and_promote_many
    with pytest.raises(ValueError):
        many(backends, [c for c, _ in picks][:4], [k for _, k in picks])
    c2 = picks[2][0]
    root = dataclasses.replace(c2, kv_view=dataclasses.replace(c2.kv_view, node_ids=()))  # no materialized node
    with pytest.raises(ValueError):
        many(backends, [c for c, _ in picks[:2]] + [root] + [c for c, _ in picks[3:]], [k for _, k in picks])
    assert state(wl, alloc, req) == before
    got = many(backends, [c for c, _ in picks], [k for _, k in picks])
    batched = state(wl, alloc, req)

    wl2, alloc2, req2 = setup(False)
    picks2 = wl2.select_commits()
    ref = [r.backend.commit_stage1_and_promote(committed_route=c, retained_routes=k)
           for r, (c, k) in zip(wl2.requests, picks2)]
    assert state(wl2, alloc2, req2) == batched
    assert [[int(x.route_id) for x in p] for p, _ in got] == [[int(x.route_id) for x in p] for p, _ in ref]
    assert [s for _, s in got] == [s for _, s in ref]
    assert sum(s["released_kv_pages"] for _, s in got) > 0

    # the EXTEND phase's prunes: one count read-back for all against one call each
    for w, results, batched_prune in ((wl, got, True), (wl2, ref, False)):
        for r, (promoted, _) in zip(w.requests, results):
            r.active = promoted
        w.batched = batched_prune
        w.fallback_extend()
    assert state(wl, alloc, req) == state(wl2, alloc2, req2)
    assert [r.stats for r in wl.requests] == [r.stats for r in wl2.requests]


def test_fused_frontier_refused_for_pages_leaves_no_trace(dev):
    """A multi-request frontier step refused because the pool has too few
    pages changes no copy-on-write lease, copy counter, dirty start, written
    request row or free page (children only take their rows and inherit
    their parents' paths and leases, as a per-request call does before its
    own allocation fails).  Retried
    after the pages come back, it leaves exactly the state of the same step
    that never failed: in particular the forked routes still get their tail
    copies, so no two routes share a decode slot."""
    dw = pkg("drafter_workload")
    npool = pkg("flashinfer_paged.native_pool")
    sr = pkg("flashinfer_paged.sglang_runtime")
    plans = [dw.ForkPlan(prefix_len=p, steps=2, forks={0: 3}, commit_depth=1, post_steps=0, extend_tokens=(1,),
                         seed=40 + i) for i, p in enumerate((100, 77, 130))]

    def setup():
        req, kv, alloc = npool.create_native_pools(num_pages=64, page_size=16, dtype=torch.bfloat16, head_num=2,
                                                   head_dim=64, layer_num=2, max_running_requests=32,
                                                   max_context_len=1024, device=dev)
        def writer(slots, vids):
            r = [torch.zeros((int(slots.numel()), 2, 64), dtype=torch.bfloat16, device=dev)] * 2
            kv.set_kv_buffer_all_layers(slots, r, r)

        wl = dw.DrafterForkWorkload(plans=plans, req_pool=req, allocator=alloc, page_size=16, device=dev,
                                    writer=writer, batched=True)
        wl.prefill()
        for r in wl.requests:
            wl._fork(r, 3)
        held = alloc.alloc(int(alloc.available_size()))
        return wl, alloc, held

    def snapshot(wl):
        torch.cuda.synchronize()
        out = []
        for r in wl.requests:
            b = r.bridge
            out.append((dict(b.route_tail_page_keys), b.next_tail_page_key, b.hot_path_counters(),
                        {rid: (row.written_length, row.pending_dirty_start) for rid, row in b.route_rows.items()},
                        {rid: p.tolist() for rid, p in b.route_slot_paths.items()}))
        return out

    def step(wl):
        return sr.SGLangFlashInferFrontierModelBackend.decode_frontiers([r.backend for r in wl.requests],
                                                                       [r.active for r in wl.requests])

    wl, alloc, held = setup()
    before = snapshot(wl)
    free_before = alloc.free_pages[alloc._head:].tolist()
    with pytest.raises(RuntimeError, match="cannot allocate"):
        step(wl)
    after = snapshot(wl)
    assert alloc.free_pages[alloc._head:].tolist() == free_before
    for r, (k0, n0, c0, rows0, _), (k1, n1, c1, rows1, paths1) in zip(wl.requests, before, after):
        assert c1 == c0
        # rows existing before are untouched; the children hold rows with
        # nothing written (the reference's prepare_frontier also takes the
        # routes' rows first, sglang_runtime.py:808)
        assert {k: v for k, v in rows1.items() if k in rows0} == rows0
        assert all(v == (0, None) for k, v in rows1.items() if k not in rows0)
        # the three children still share the prefix tail's one lease: none got
        # the fresh lease of a copy that did not happen
        assert len({k1[int(route.route_id)] for route in r.active}) == 1
        assert all(k1[k] == v for k, v in k0.items())
    alloc.free(held)
    outs = step(wl)
    got = snapshot(wl)

    wl2, alloc2, held2 = setup()
    alloc2.free(held2)
    step(wl2)
    want = snapshot(wl2)
    # node ids differ (the refused call reserved some), so compare slot state only
    assert [(k, n, c, rows, paths) for k, n, c, rows, paths in got] == \
           [(k, n, c, rows, paths) for k, n, c, rows, paths in want]
    assert alloc.free_pages[alloc._head:].tolist() == alloc2.free_pages[alloc2._head:].tolist()
    for out in outs:
        assert out.metadata["cow_pages_copied_total"] == 2
    slots = torch.cat([torch.tensor([int(p[-1]) for p in s[4].values() if p]) for s in got])
    assert int(slots.unique().numel()) == int(slots.numel())
