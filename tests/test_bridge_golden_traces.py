"""Multi-step route-pool bridge traces against the reference's bridge classes.

``tests/golden/bridge_traces.json`` holds the traces of
``tests/golden/bridge_trace.py`` run over the reference's ``KVTreeStore``,
``SGLangRoutePoolBridge`` and ``SGLangFlashInferFrontierModelBackend``
(``flashinfer_paged/kv.py``, ``flashinfer_paged/sglang_runtime.py``), written by
``tests/golden/make_bridge_traces.py``.  The same driver runs here over this
package's classes on the same host pools; every pool call (allocations, KV
moves, request-row writes, frees), every frontier's slots and counters, and
the bridge's state after every phase (slot paths, leases, rows, owned pages,
reference counts, counters) must be equal.

What the fixture does not come from: the pools under both bridges are the
oracle's host pools (``oracle/route_pool.py``), whose free-list policy is a
restatement of SGLang's paged allocator (SGLang is absent), and the fallback
EXTEND is the reference's sequence of bridge calls made by the generator,
because its model forward needs SGLang.  So the bridge logic is pinned
against the reference; the allocator's free-list order is pinned only by the
invariants its arithmetic fixes, checked here on every phase of both traces."""

import json
import os
import sys
from types import SimpleNamespace

import pytest

from helpers import check_allocator_invariants, pkg

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
sys.path.insert(0, GOLDEN)

import bridge_trace  # noqa: E402
from oracle import route_pool  # noqa: E402


@pytest.fixture(scope="module")
def golden():
    with open(os.path.join(GOLDEN, "bridge_traces.json")) as f:
        return json.load(f)


def _mods():
    kv = pkg("flashinfer_paged.kv")
    sr = pkg("flashinfer_paged.sglang_runtime")
    ty = pkg("flashinfer_paged.types")
    return SimpleNamespace(KVTreeStore=kv.KVTreeStore, SGLangRoutePoolBridge=sr.SGLangRoutePoolBridge,
                           SGLangFlashInferFrontierModelBackend=sr.SGLangFlashInferFrontierModelBackend,
                           DecodePhase=ty.DecodePhase, RouteState=ty.RouteState)


def _extend(backend, tokens):
    backend.append_known_tokens_as_prefix(tokens)


def _first_difference(a, b, path=""):
    if type(a) is not type(b):
        return path, a, b
    if isinstance(a, dict):
        for k in sorted(set(a) | set(b)):
            if k not in a or k not in b:
                return f"{path}.{k}", a.get(k, "<missing>"), b.get(k, "<missing>")
            d = _first_difference(a[k], b[k], f"{path}.{k}")
            if d:
                return d
        return None
    if isinstance(a, list):
        for i, (x, y) in enumerate(zip(a, b)):
            d = _first_difference(x, y, f"{path}[{i}]")
            if d:
                return d
        if len(a) != len(b):
            return f"{path} (length)", len(a), len(b)
        return None
    return None if a == b else (path, a, b)


@pytest.mark.parametrize("scenario", bridge_trace.SCENARIOS)
def test_bridge_trace_equals_reference(golden, scenario):
    ours = json.loads(json.dumps(bridge_trace.run(_mods(), scenario, _extend, oracle_pools=route_pool)))
    ref = golden[scenario]
    assert [p["phase"] for p in ours["phases"]] == [p["phase"] for p in ref["phases"]]
    for mine, theirs in zip(ours["phases"], ref["phases"]):
        d = _first_difference(mine, theirs, mine["phase"])
        assert d is None, f"{scenario}: first difference at {d[0]}: ours {d[1]!r}, reference {d[2]!r}"


def _unrle(runs):
    return [first + i for first, n in runs for i in range(n)]


def _check_trace_invariants(trace, label):
    ps, num_pages = trace["page_size"], trace["num_pages"]
    for ph in trace["phases"]:
        owned = [_unrle(r["owned_pages"]) for r in ph["requests"]]
        live = []
        for r in ph["requests"]:
            slots = _unrle(r["prefix"]) if r["prefix"] is not None else []
            for path in r["paths"].values():
                slots.extend(_unrle(path))
            live.append(slots)
        check_allocator_invariants(num_pages, _unrle(ph["free_pages"]), owned, live, ps,
                                   where=f"{label} after {ph['phase']}")


@pytest.mark.parametrize("scenario", bridge_trace.SCENARIOS)
def test_trace_allocator_invariants(golden, scenario):
    _check_trace_invariants(golden[scenario], f"{scenario} (fixture)")
    ours = json.loads(json.dumps(bridge_trace.run(_mods(), scenario, _extend, oracle_pools=route_pool)))
    _check_trace_invariants(ours, scenario)


def test_golden_traces_exercise_the_rules(golden):
    """The fixture covers what it is meant to: tail copies, request-row
    full inits and appends, promotion, prune frees and the EXTEND.  (A
    request-row COW patch never arises in a fork sequence: the child that
    takes over its parent's row is also the first writer of the shared tail,
    ``sglang_runtime.py:343-351``; the patch rule is pinned by the reference's
    unit literal in test_route_pool_host.py.)"""
    events = [ev[0] for sc in golden.values() for ph in sc["phases"] for ev in ph["events"]]
    for kind in ("move", "alloc", "alloc_decode", "alloc_extend", "free", "row_alloc", "row_free", "row_write"):
        assert kind in events, kind
    fr = [f for sc in golden.values() for ph in sc["phases"] for f in ph.get("frontiers", [])]
    deltas = [f["counter_delta"] for f in fr]
    assert any(f["cow_total"][0] for f in fr)
    assert any(d.get("req_row_full_init_calls", 0) for d in deltas)
    assert any(d.get("req_row_append_calls", 0) for d in deltas)
    stats = [s for sc in golden.values() for ph in sc["phases"] for s in ph.get("stats", [])]
    assert all(s["released_kv_pages"] >= 0 for s in stats) and any(s["released_kv_pages"] for s in stats)


def test_allocator_invariant_check_catches_planted_mistakes(golden):
    """The invariant check fails on a free page that is also owned, on a
    duplicate free page, on a leaked page and on a live slot off its owner's
    pages."""
    import copy

    trace = golden["fork_mid_page_page4"]
    _check_trace_invariants(trace, "unchanged")
    ph = -1
    owned0 = _unrle(trace["phases"][ph]["requests"][0]["owned_pages"])
    plants = []
    t = copy.deepcopy(trace)  # owned page also on the free list
    t["phases"][ph]["free_pages"].append([owned0[0], 1])
    plants.append(t)
    t = copy.deepcopy(trace)  # duplicate free page
    t["phases"][ph]["free_pages"].append(list(t["phases"][ph]["free_pages"][0][:1]) + [1])
    plants.append(t)
    t = copy.deepcopy(trace)  # a page leaked: neither free nor owned
    t["phases"][ph]["requests"][0]["owned_pages"] = [[p, 1] for p in owned0[1:]]
    plants.append(t)
    t = copy.deepcopy(trace)  # a live slot on a page the request does not own
    stray = next(p for p in range(1, trace["num_pages"] + 1) if p not in owned0)
    t["phases"][ph]["requests"][0]["prefix"].append([stray * trace["page_size"], 1])
    plants.append(t)
    for t in plants:
        with pytest.raises(AssertionError):
            _check_trace_invariants(t, "planted")
