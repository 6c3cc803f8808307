"""Multi-step route-pool bridge trace (test infrastructure).

One seeded sequence per scenario:

1. prefill each request's prefix (one ``alloc_extend`` from an empty prefix);
2. frontier decode steps; before some steps every active route forks into
   three children, at whatever fill level the shared tail page has, so the
   children's first frontier copies the tail;
3. commit the fork point of a random final route, keep its descendants,
   promote and prune (``commit_stage1_and_promote``);
4. one decode step of the kept routes;
5. fallback EXTEND: release every route row, prune, append four known tokens
   to the prefix, then decode one step from a fresh root.

The pools are the oracle's host pools (paged free list, KV content as value
ids, request rows) behind logging wrappers.  The record holds every pool call
in order, every frontier's inputs and metadata, and the bridge's and the
store's state after every phase.

``run(mods, scenario, extend)`` drives the classes it is given.
``make_bridge_traces.py`` runs it on the reference's
(``flashinfer_paged/kv.py``, ``flashinfer_paged/sglang_runtime.py``) and writes
``bridge_traces.json``; ``tests/test_bridge_golden_traces.py`` runs it on this
package's and compares.

Two normalisations make the records comparable:

* consecutive ``move_kv_cache`` calls are merged into one: the reference
  moves one copied page per call (``sglang_runtime.py:780-785``); a frontier's
  copies may also go in one call;
* slot and value lists are stored as runs ``[first, length]`` of consecutive
  integers, which keeps the file small.
"""

from __future__ import annotations

import random
from types import SimpleNamespace
from typing import Any, Callable

import numpy as np
import torch

VOCAB = 128256


def rle(x) -> list[list[int]]:
    """Runs of consecutive integers as [first, length]."""
    if isinstance(x, torch.Tensor):
        x = x.detach().cpu().reshape(-1).tolist()
    elif isinstance(x, np.ndarray):
        x = x.reshape(-1).tolist()
    runs: list[list[int]] = []
    for v in x:
        v = int(v)
        if runs and runs[-1][0] + runs[-1][1] == v:
            runs[-1][1] += 1
        else:
            runs.append([v, 1])
    return runs


def _ints(x) -> list[int]:
    if isinstance(x, torch.Tensor):
        return [int(v) for v in x.detach().cpu().reshape(-1).tolist()]
    return [int(v) for v in x]


# ----------------------------------------------------------------- pools
class LoggedKV:
    def __init__(self, inner, log: list) -> None:
        self.inner = inner
        self.log = log

    @property
    def values(self) -> np.ndarray:
        return self.inner.values

    def move_kv_cache(self, dst, src) -> None:
        self.log.append(["move", rle(dst), rle(src)])
        self.inner.move_kv_cache(dst, src)

    def write(self, slots, value_ids) -> None:
        self.inner.write(slots, value_ids)


class LoggedAllocator:
    def __init__(self, inner, log: list) -> None:
        self.inner = inner
        self.log = log
        self.kv = LoggedKV(inner.get_kvcache(), log)
        self.page_size = inner.page_size

    @property
    def free_pages(self) -> list[int]:
        return self.inner.free_pages

    def get_kvcache(self) -> LoggedKV:
        return self.kv

    def alloc(self, need_size):
        out = self.inner.alloc(need_size)
        self.log.append(["alloc", int(need_size), None if out is None else rle(out)])
        return out

    def alloc_decode(self, seq_lens, seq_lens_cpu, last_loc):
        out = self.inner.alloc_decode(seq_lens, seq_lens_cpu, last_loc)
        self.log.append(["alloc_decode", _ints(seq_lens_cpu), _ints(last_loc), None if out is None else rle(out)])
        return out

    def alloc_extend(self, prefix_lens, prefix_lens_cpu, seq_lens, seq_lens_cpu, last_loc, extend_num_tokens):
        out = self.inner.alloc_extend(prefix_lens, prefix_lens_cpu, seq_lens, seq_lens_cpu, last_loc,
                                      extend_num_tokens)
        self.log.append(["alloc_extend", _ints(prefix_lens_cpu), _ints(seq_lens_cpu), _ints(last_loc),
                         int(extend_num_tokens), None if out is None else rle(out)])
        return out

    def free(self, slots) -> None:
        self.log.append(["free", rle(torch.as_tensor(slots))])
        self.inner.free(slots)

    def clear(self) -> None:
        self.inner.clear()


class LoggedReqPool:
    def __init__(self, inner, log: list) -> None:
        self.inner = inner
        self.log = log
        self.req_to_token = inner.req_to_token

    def alloc(self, reqs):
        rows = self.inner.alloc(reqs)
        self.log.append(["row_alloc", len(reqs), None if rows is None else _ints(rows)])
        return rows

    def free(self, req) -> None:
        row = getattr(req, "req_pool_idx", req)
        self.log.append(["row_free", None if row is None else int(row)])
        self.inner.free(req)

    def write(self, indices, values) -> None:
        row, pos = indices
        if isinstance(pos, slice):
            self.log.append(["row_write", int(row), pos.start, pos.stop, rle(values)])
        else:
            self.log.append(["row_write_index", rle(torch.as_tensor(row)), rle(torch.as_tensor(pos)), rle(values)])
        self.inner.write(indices, values)

    def clear(self) -> None:
        self.inner.clear()


def normalise(log: list) -> list:
    """Merge runs of consecutive move events into one move."""
    out: list = []
    for ev in log:
        if ev[0] == "move" and out and out[-1][0] == "move":
            out[-1] = ["move", _join(out[-1][1], ev[1]), _join(out[-1][2], ev[2])]
        else:
            out.append(ev)
    return out


def _join(a: list, b: list) -> list:
    a = [list(r) for r in a]
    for first, n in b:
        if a and a[-1][0] + a[-1][1] == first:
            a[-1][1] += n
        else:
            a.append([first, n])
    return a


# ----------------------------------------------------------------- model
class PatternModel:
    """Stands in for the Drafter model: every new token's KV slot gets the
    next value id; logits are zeros."""

    def __init__(self, kv: LoggedKV, counter: list[int]) -> None:
        self.kv = kv
        self.counter = counter
        # the frontier backend asks the runner for its eager runner
        self.model_runner = SimpleNamespace(eager_runner=object())
        self.last: tuple[list[int], list[int]] | None = None

    def runtime_metadata(self, **_kw) -> dict:
        return {}

    def _write(self, slots: torch.Tensor) -> torch.Tensor:
        n = int(slots.numel())
        vids = list(range(self.counter[0], self.counter[0] + n))
        self.counter[0] += n
        self.kv.write(slots.detach().cpu().numpy(), np.asarray(vids, dtype=np.int64))
        self.last = (_ints(slots), vids)
        return torch.zeros((n, 8), dtype=torch.float32)

    def forward_frontier(self, *, input_ids, route_kv_metadata):
        return self._write(route_kv_metadata.out_cache_loc)

    def forward_extend(self, *, input_ids, out_cache_loc, positions, req_pool_indices, seq_lens_cpu):
        return self._write(out_cache_loc)


# ----------------------------------------------------------------- scenarios
def scenario_plans(name: str) -> tuple[int, int, list[dict]]:
    """(page_size, num_pages, plans) of a named scenario."""
    if name == "fork_1000_page16":
        # one request, 1000-token prefix (tail page holds 8), three routes of
        # depth 4 forking at the prefix, commit a whole route
        rng = random.Random(0)
        return 16, 4096, [dict(prefix_len=1000, steps=4, forks={0: 3}, commit_depth=4,
                               extend=[rng.randrange(VOCAB) for _ in range(4)], seed=0)]
    if name == "fork_stress_8req_page64":
        # eight requests, two 3-way forks at random depths, 8 decode steps,
        # commit the second fork point and keep its three children
        rng = random.Random(5)
        plans = []
        for r in range(8):
            prefix = rng.randrange(2 * 64, 16 * 64)
            if prefix % 64 == 0:
                prefix += 1 + rng.randrange(63)
            a = rng.randrange(1, 4)
            b = rng.randrange(1, 4)
            plans.append(dict(prefix_len=prefix, steps=8, forks={a: 3, a + b: 3}, commit_depth=a + b,
                              extend=[rng.randrange(VOCAB) for _ in range(4)], seed=5000 + r))
        return 64, 1024, plans
    if name == "fork_mid_page_page4":
        # small pages: forks at every fill level of a 4-slot page, three
        # requests sharing the pools, prefixes ending mid-page and on a boundary
        rng = random.Random(7)
        plans = []
        for r, prefix in enumerate((9, 12, 14)):
            plans.append(dict(prefix_len=prefix, steps=7, forks={0: 2, 2: 3, 5: 2}, commit_depth=3,
                              extend=[rng.randrange(VOCAB) for _ in range(5)], seed=7000 + r))
        return 4, 512, plans
    raise KeyError(name)


SCENARIOS = ("fork_1000_page16", "fork_stress_8req_page64", "fork_mid_page_page4")


def run(mods: Any, scenario: str, extend: Callable[[Any, list[int]], None], *, oracle_pools: Any) -> dict:
    """Drive one scenario through ``mods`` (``KVTreeStore``,
    ``SGLangRoutePoolBridge``, ``SGLangFlashInferFrontierModelBackend``,
    ``DecodePhase``, ``RouteState``); ``extend(backend, tokens)`` runs the fallback EXTEND.
    ``oracle_pools`` provides ``OracleAllocator`` and ``OracleReqPool``."""
    page_size, num_pages, plans = scenario_plans(scenario)
    log: list = []
    alloc = LoggedAllocator(oracle_pools.OracleAllocator(num_pages=num_pages, page_size=page_size), log)
    rows = LoggedReqPool(oracle_pools.OracleReqPool(size=96, max_context_len=2048), log)
    counter = [1]
    model = PatternModel(alloc.kv, counter)
    reqs = []
    for plan in plans:
        store = mods.KVTreeStore()
        bridge = mods.SGLangRoutePoolBridge(req_to_token_pool=rows, token_to_kv_pool_allocator=alloc,
                                            page_size=page_size, device="cpu", use_page_attention_metadata=False)
        backend = mods.SGLangFlashInferFrontierModelBackend(route_store=store, executor=model, route_pool=bridge)
        reqs.append(SimpleNamespace(plan=plan, store=store, bridge=bridge, backend=backend,
                                    rng=random.Random(plan["seed"]), active=[]))
    phases: list = []

    def snap(name: str) -> None:
        phases.append({"phase": name, "events": normalise(log[:]), "requests": [_state(r, alloc) for r in reqs],
                       "free_pages": rle(alloc.free_pages)})
        log.clear()

    # 1. prefill
    for req in reqs:
        n = req.plan["prefix_len"]
        zero = torch.zeros(1, dtype=torch.long)
        slots = alloc.alloc_extend(zero, zero, torch.tensor([n]), torch.tensor([n]),
                                   torch.full((1,), -1, dtype=torch.long), n)
        model._write(slots)
        tokens = [req.rng.randrange(VOCAB) for _ in range(n)]
        req.backend.attach_prefilled_prefix(prompt_token_ids=tokens, prefix_slot_ids=slots,
                                            next_token_logits=torch.zeros(8))
        req.active = [_root(mods, req.store, req.rng.randrange(VOCAB), n)]
    snap("prefill")

    def decode(req, step=None):
        if step is not None and step in req.plan["forks"]:
            children = []
            for parent in req.active:
                for _ in range(req.plan["forks"][step]):
                    lp = -round(req.rng.random() * 4.0, 6)
                    children.append(req.store.clone_route_with_new_pending(parent, req.rng.randrange(VOCAB),
                                                                           parent.cumulative_logprob + lp))
            req.store.release_routes_without_descendants(req.active, children)
            req.active = children
        out = req.backend.decode_frontier_one_token(req.active)
        md = out.metadata
        frontier = {
            "routes": [int(r.route_id) for r in req.active],
            "new_node_ids": [int(x) for x in out.new_node_ids],
            "written": model.last[0],
            "cow_total": [md["cow_pages_copied_total"], md["cow_tokens_copied_total"]],
            "counter_delta": dict(sorted(md["hot_path_counter_delta"].items())),
        }
        req.store.mark_routes_materialized(req.active, out.new_node_ids, mods.DecodePhase.STAGE1)
        for r in req.active:
            r.pending_token_id = req.rng.randrange(VOCAB)
        return frontier

    # 2. stage-1 decode steps
    steps = max(r.plan["steps"] for r in reqs)
    for t in range(steps):
        fr = []
        for req in reqs:
            if t < req.plan["steps"]:
                fr.append(decode(req, t))
        snap(f"decode{t}")
        phases[-1]["frontiers"] = fr

    # 3. commit + promote + prune
    stats = []
    for req in reqs:
        final = req.rng.choice(req.active)
        committed = final
        while committed.total_materialized_depth() > req.plan["commit_depth"]:
            committed = req.store.get_route(int(committed.parent_route_id))
        nodes = committed.kv_view.node_ids
        keep = [r for r in req.active if r.kv_view.node_ids[: len(nodes)] == nodes]
        promoted, st = req.backend.commit_stage1_and_promote(committed_route=committed, retained_routes=keep)
        req.active = list(promoted)
        stats.append({k: int(v) for k, v in sorted(st.items())})
    snap("commit")
    phases[-1]["stats"] = stats

    # 4. decode of the kept routes
    phases_fr = [decode(req) for req in reqs]
    snap("post_decode")
    phases[-1]["frontiers"] = phases_fr

    # 5. fallback EXTEND, then a fresh root
    released = []
    for req in reqs:
        b = req.bridge
        released.append([int(b.retain_route_rows([])), int(b.release_unreferenced_node_slots([]))])
        extend(req.backend, list(req.plan["extend"]))
        req.active = [_root(mods, req.store, req.rng.randrange(VOCAB), len(req.backend.prefix_token_ids))]
    snap("extend")
    phases[-1]["released"] = released
    phases_fr = [decode(req) for req in reqs]
    snap("extend_decode")
    phases[-1]["frontiers"] = phases_fr
    return {"scenario": scenario, "page_size": page_size, "num_pages": num_pages, "phases": phases}


def _root(mods: Any, store: Any, token: int, committed: int):
    """A stage-1 root route on the committed prefix, registered as the
    reference's builders register theirs (``builders.py:45-59``)."""
    rid = store.allocate_route_id()
    return store.register_route(mods.RouteState(
        route_id=rid, stage1_root_id=rid, parent_route_id=None, materialized_leaf_node_id=None,
        pending_token_id=int(token), cumulative_logprob=0.0, stage1_depth=0, stage2_depth=0,
        kv_view=store.prefix_view(committed).fork()))


def _state(req, alloc: LoggedAllocator) -> dict:
    b = req.bridge
    b._materialize_pending_owned_pages()
    values = alloc.kv.values

    def path_values(p):
        return rle(values[np.asarray(_ints(p), dtype=np.int64)])

    node_slots = {}
    for nid, s in sorted(b.node_slot_ids.items()):
        node_slots[str(int(nid))] = _ints(torch.as_tensor(s))[0]
    return {
        "prefix": rle(b.prefix_slot_ids) if b.prefix_slot_ids is not None else None,
        "prefix_values": path_values(b.prefix_slot_ids) if b.prefix_slot_ids is not None else None,
        "prefix_pages": sorted(int(p) for p in b.prefix_page_ids),
        "prefix_tail_key": b.prefix_tail_page_key,
        "prefix_partial_tail_keys": {str(k): int(v) for k, v in sorted(b.prefix_partial_tail_keys.items())},
        "next_tail_key": int(b.next_tail_page_key),
        "rows": {str(rid): [int(r.req_pool_index), int(r.written_length),
                            None if r.pending_dirty_start is None else int(r.pending_dirty_start)]
                 for rid, r in sorted(b.route_rows.items())},
        "paths": {str(rid): rle(p) for rid, p in sorted(b.route_slot_paths.items())},
        "path_values": {str(rid): path_values(p) for rid, p in sorted(b.route_slot_paths.items())},
        "tail_keys": {str(rid): int(k) for rid, k in sorted(b.route_tail_page_keys.items())},
        "owned_pages": rle(sorted(int(p) for p in b.owned_page_ids)),
        "node_slots": node_slots,
        "ref_counts": {str(k): int(v) for k, v in sorted(b.page_reference_counts().items())},
        "counters": dict(sorted(b.hot_path_counters().items())),
        "cow": [int(b.cow_pages_copied), int(b.cow_tokens_copied)],
        "active": [[int(r.route_id), None if r.parent_route_id is None else int(r.parent_route_id),
                    int(r.stage1_root_id), [int(n) for n in r.kv_view.node_ids],
                    int(r.kv_view.prefix.committed_length), int(r.stage1_depth), int(r.stage2_depth)]
                   for r in req.active],
        "prefix_tokens": len(req.backend.prefix_token_ids),
    }
