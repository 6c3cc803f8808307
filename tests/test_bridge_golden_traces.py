"""Multi-step route-pool bridge traces against the reference's own bridge.

``tests/golden/bridge_traces.json`` holds the traces of
``tests/golden/bridge_trace.py`` run over the reference's ``KVTreeStore``,
``SGLangRoutePoolBridge`` and ``SGLangFlashInferFrontierModelBackend``
(``flashinfer_paged/kv.py``, ``flashinfer_paged/sglang_runtime.py``), written by
``tests/golden/make_bridge_traces.py``.  The same driver runs here over this
package's classes on the same host pools; every pool call (allocations, KV
moves, request-row writes, frees), every frontier's slots and counters, and
the bridge's state after every phase (slot paths, leases, rows, owned pages,
reference counts, counters) must be equal."""

import json
import os
import sys
from types import SimpleNamespace

import pytest

from helpers import pkg

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
