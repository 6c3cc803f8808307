"""Drafter route-pool fork workload: seeded fork / decode / promote / prune /
fallback-EXTEND sequences driven through the route-pool bridge.

One request = one ``KVTreeStore`` + one ``SGLangRoutePoolBridge`` + one
frontier backend; all requests share one allocator, KV pool and request-row
pool, as the Drafter's requests share SGLang's pools.  The model is replaced
by an executor that writes, for every new token, a K/V row pattern derived
from a value id (``kv_pattern``), so the KV content of every slot is known
exactly: slot s holds the pattern of the value id last written or moved to it.

The sequence per request (``run``):

1. prefill ``prefix_len`` tokens (``alloc_extend`` from an empty prefix);
2. ``steps`` frontier decode steps; before step t every active route forks
   into ``forks[t]`` children (forks happen at arbitrary fill levels of the
   shared tail page, so the children's first frontier copies the tail);
3. commit a route (an ancestor at depth ``commit_depth`` of a random final
   route, or, with ``select="best"``, of the final route with the highest
   sum of its nodes' log-probs, each node drawn as -(u * 5), u uniform in
   [0, 1)), keep its descendants, promote, prune;
4. ``post_steps`` decode steps of the kept routes;
5. fallback EXTEND: drop every route, prune, append ``extend_tokens``
   known tokens to the prefix with one EXTEND, then decode ``post_steps``
   steps from a fresh root.
"""

from __future__ import annotations

import random
from dataclasses import dataclass, field
from typing import Any, Callable, Sequence

import torch

from .flashinfer_paged.kv import KVTreeStore
from .flashinfer_paged.sglang_runtime import (SGLangFlashInferFrontierModelBackend, SGLangRoutePoolBridge,
                                              fused_frontier_supported, release_unreferenced_node_slots_many)
from .flashinfer_paged.types import DecodePhase, RouteState

VOCAB = 128256


def kv_pattern(value_ids: torch.Tensor, layer: int, kv: int, heads: int, head_dim: int) -> torch.Tensor:
    """int16 row pattern [n, heads, head_dim] of each value id (a 64-bit
    multiply-xorshift hash; identical on every device)."""
    v = value_ids.to(torch.int64).reshape(-1, 1, 1)
    h = torch.arange(heads, dtype=torch.int64, device=v.device).reshape(1, -1, 1)
    d = torch.arange(head_dim, dtype=torch.int64, device=v.device).reshape(1, 1, -1)
    x = v * 0x9E3779B1 + (layer * 2 + kv) * 0x85EBCA77 + h * 0xC2B2AE3D + d * 0x27D4EB2F
    x = x ^ (x >> 15)
    x = x * 0x2C1B3C6D
    x = x ^ (x >> 12)
    x = x & 0xFFFF
    return (x - ((x >> 15) << 16)).to(torch.int16)


@dataclass(frozen=True)
class ForkPlan:
    prefix_len: int
    steps: int
    forks: dict[int, int]
    commit_depth: int
    post_steps: int
    extend_tokens: tuple[int, ...]
    seed: int
    select: str = "random"  # "random" or "best" (highest sum of node log-probs)


def config1_plans(seed: int = 0) -> list[ForkPlan]:
    """1000-token prefix (tail page holds 8 at page 16), k=3 routes of depth 4
    forking at the prefix; commit the whole route with the highest sum of
    random node log-probs, keep it."""
    rng = random.Random(seed)
    return [ForkPlan(prefix_len=1000, steps=4, forks={0: 3}, commit_depth=4, post_steps=1,
                     extend_tokens=tuple(rng.randrange(VOCAB) for _ in range(4)), seed=seed, select="best")]


def config5_plans(n_requests: int = 8, page_size: int = 64, seed: int = 0) -> list[ForkPlan]:
    """8 requests, 9 routes each from two 3-way forks at random depths, 8
    decode steps; commit the second-level fork point, keep its 3 children."""
    rng = random.Random(seed)
    plans = []
    for r in range(n_requests):
        prefix = rng.randrange(2 * page_size, 16 * page_size)
        if prefix % page_size == 0:
            prefix += 1 + rng.randrange(page_size - 1)
        a = rng.randrange(1, 4)
        b = rng.randrange(1, 4)
        plans.append(ForkPlan(prefix_len=prefix, steps=8, forks={a: 3, a + b: 3}, commit_depth=a + b, post_steps=1,
                              extend_tokens=tuple(rng.randrange(VOCAB) for _ in range(4)), seed=seed * 1000 + r))
    return plans


class PatternExecutor:
    """Stands in for the Drafter model: writes each new token's K/V pattern
    and returns zero logits.  ``writer(slots, value_ids)`` stores the rows."""

    def __init__(self, writer: Callable[[torch.Tensor, torch.Tensor], None], ids: "ValueIds", vocab: int = 8) -> None:
        self.writer = writer
        self.ids = ids
        self.vocab = vocab

    def _write(self, slots: torch.Tensor) -> torch.Tensor:
        vids = self.ids.take(int(slots.numel()))
        self.writer(slots, vids)
        return torch.zeros((int(slots.numel()), self.vocab), dtype=torch.float32, device=slots.device)

    def forward_frontier(self, *, input_ids, route_kv_metadata):
        return self._write(route_kv_metadata.out_cache_loc)

    def forward_extend(self, *, input_ids, out_cache_loc, positions, req_pool_indices, seq_lens_cpu):
        return self._write(out_cache_loc)


class ValueIds:
    def __init__(self) -> None:
        self.next = 1
        self.log: list[tuple[int, int]] = []

    def take(self, n: int) -> torch.Tensor:
        out = torch.arange(self.next, self.next + n, dtype=torch.int64)
        self.log.append((self.next, n))
        self.next += n
        return out


@dataclass
class RequestState:
    plan: ForkPlan
    store: KVTreeStore
    bridge: SGLangRoutePoolBridge
    backend: SGLangFlashInferFrontierModelBackend
    rng: random.Random
    active: list[RouteState] = field(default_factory=list)
    prefix_value_ids: list[int] = field(default_factory=list)
    node_value_ids: dict[int, int] = field(default_factory=dict)
    stats: list[dict[str, int]] = field(default_factory=list)
    # select="best": each materialized node's log-prob, from its own generator
    # (the request's main generator, which draws tokens, is left as it is)
    node_logprobs: dict[int, float] = field(default_factory=dict)
    logprob_rng: random.Random | None = None
    selected_route_id: int | None = None


class DrafterForkWorkload:
    """Runs ``ForkPlan``s through bridges over shared pools.

    ``writer(slots, value_ids)`` writes KV rows; ``on_phase(name)`` is
    called after every phase (for state comparison or timing)."""

    def __init__(self, *, plans: Sequence[ForkPlan], req_pool: Any, allocator: Any, page_size: int,
                 device, writer: Callable[[torch.Tensor, torch.Tensor], None],
                 use_page_attention_metadata: bool = True, batched: bool = False) -> None:
        self.page_size = int(page_size)
        # batched: each decode step runs every request's frontier as one
        # step (SGLangFlashInferFrontierModelBackend.decode_frontiers), whose
        # writer call covers all requests' new slots in request order -- the
        # value ids the per-request calls take one after another
        self.batched = bool(batched)
        self.device = torch.device(device)
        self.allocator = allocator
        self.req_pool = req_pool
        self.ids = ValueIds()
        self.writer = writer
        self.requests: list[RequestState] = []
        for plan in plans:
            store = KVTreeStore()
            bridge = SGLangRoutePoolBridge(req_to_token_pool=req_pool, token_to_kv_pool_allocator=allocator,
                                           page_size=page_size, device=self.device,
                                           use_page_attention_metadata=use_page_attention_metadata)
            executor = PatternExecutor(self._record_writer, self.ids)
            backend = SGLangFlashInferFrontierModelBackend(route_store=store, executor=executor, route_pool=bridge)
            self.requests.append(RequestState(plan, store, bridge, backend, random.Random(plan.seed),
                                              logprob_rng=random.Random(plan.seed + 0x5EED)))
        self._last_write: tuple[torch.Tensor, torch.Tensor] | None = None

    def _record_writer(self, slots: torch.Tensor, vids: torch.Tensor) -> None:
        self._last_write = (slots, vids)
        self.writer(slots, vids)

    # ------------------------------------------------------------ phases
    def prefill(self) -> None:
        for req in self.requests:
            n = req.plan.prefix_len
            dev = self.device
            zero = torch.zeros(1, dtype=torch.int64)
            slots = self.allocator.alloc_extend(zero.to(dev), zero, torch.tensor([n], device=dev),
                                                torch.tensor([n]), torch.full((1,), -1, dtype=torch.int64, device=dev),
                                                n)
            if slots is None:
                raise RuntimeError("pool too small for the prefill")
            vids = self.ids.take(n)
            self.writer(slots, vids)
            req.prefix_value_ids = vids.tolist()
            tokens = [req.rng.randrange(VOCAB) for _ in range(n)]
            req.backend.attach_prefilled_prefix(prompt_token_ids=tokens, prefix_slot_ids=slots,
                                                next_token_logits=torch.zeros(8, device=dev))
            req.active = [req.store.new_root_route(req.rng.randrange(VOCAB), req.store.prefix_view(n))]

    def _fork(self, req: RequestState, fanout: int) -> None:
        children = []
        for parent in req.active:
            for _ in range(fanout):
                children.append(req.store.clone_route_with_new_pending(parent, req.rng.randrange(VOCAB)))
        req.store.release_routes_without_descendants(req.active, children)
        req.active = children

    def decode_step(self, req: RequestState, step: int | None = None) -> None:
        if step is not None and step in req.plan.forks:
            self._fork(req, req.plan.forks[step])
        out = req.backend.decode_frontier_one_token(req.active)
        _, vids = self._last_write
        self._after_decode(req, out, vids.tolist())

    def decode_steps(self, reqs: Sequence[RequestState], step: int | None = None) -> None:
        """One decode step of several requests: one batched frontier step in
        batched mode, else one call per request in order."""
        if not self.batched or not fused_frontier_supported([r.bridge for r in reqs]):
            for req in reqs:
                self.decode_step(req, step)
            return
        for req in reqs:
            if step is not None and step in req.plan.forks:
                self._fork(req, req.plan.forks[step])
        outs = SGLangFlashInferFrontierModelBackend.decode_frontiers([r.backend for r in reqs],
                                                                     [r.active for r in reqs])
        _, vids = self._last_write
        values = vids.tolist()
        off = 0
        for req, out in zip(reqs, outs):
            n = len(out.new_node_ids)
            self._after_decode(req, out, values[off : off + n])
            off += n

    def _after_decode(self, req: RequestState, out, values: list[int]) -> None:
        for nid, v in zip(out.new_node_ids, values):
            req.node_value_ids[int(nid)] = int(v)
            if req.plan.select == "best":
                req.node_logprobs[int(nid)] = -(req.logprob_rng.random() * 5.0)
        req.store.mark_routes_materialized(req.active, out.new_node_ids, DecodePhase.STAGE1)
        for r in req.active:
            r.pending_token_id = req.rng.randrange(VOCAB)

    def _post_steps(self) -> None:
        if not self.batched:
            for req in self.requests:
                for _ in range(req.plan.post_steps):
                    self.decode_step(req)
            return
        for k in range(max(r.plan.post_steps for r in self.requests)):
            self.decode_steps([r for r in self.requests if k < r.plan.post_steps])

    def stage1(self, on_step: Callable[[str], None] | None = None) -> None:
        steps = max(r.plan.steps for r in self.requests)
        for t in range(steps):
            self.decode_steps([r for r in self.requests if t < r.plan.steps], t)
            if on_step is not None:
                on_step(f"decode{t}")

    def commit(self) -> None:
        """Every request commits its selected route's path up to its commit
        depth, keeps the routes that extend it, promotes and prunes: one
        batched call over the shared pools (``batched``), else one call per
        request.  Both leave the same state."""
        picks = self.select_commits()
        if self.batched:
            results = SGLangFlashInferFrontierModelBackend.commit_stage1_and_promote_many(
                [r.backend for r in self.requests], [c for c, _ in picks], [k for _, k in picks])
        else:
            results = [req.backend.commit_stage1_and_promote(committed_route=c, retained_routes=k)
                       for req, (c, k) in zip(self.requests, picks)]
        for req, (promoted, stats) in zip(self.requests, results):
            req.active = promoted
            req.stats.append(stats)

    def select_commits(self) -> list[tuple[RouteState, list[RouteState]]]:
        """Each request's committed route (the selected final route's ancestor
        at the commit depth) and the active routes that extend it; records the
        selection and the committed value ids."""
        picks = []
        for req in self.requests:
            if req.plan.select == "best":
                # the Target's target_best order (src/atlas_0709/target_runtime.py:444-451):
                # score, then the draft path log-prob, then the lower route id
                final = max(req.active, key=lambda r: (self.route_score(req, r), float(r.cumulative_logprob),
                                                       -int(r.route_id)))
            else:
                final = req.rng.choice(req.active)
            req.selected_route_id = int(final.route_id)
            committed = final
            while committed.total_materialized_depth() > req.plan.commit_depth:
                committed = req.store.routes[int(committed.parent_route_id)]
            nodes = committed.kv_view.node_ids
            keep = [r for r in req.active if r.kv_view.node_ids[: len(nodes)] == nodes]
            req.prefix_value_ids = req.prefix_value_ids + [req.node_value_ids[int(n)] for n in nodes]
            picks.append((committed, keep))
        return picks

    def post_decode(self) -> None:
        self._post_steps()

    def fallback_extend(self) -> None:
        """Every request drops its routes and prunes, then the EXTENDs run in
        request order: one batched call over the shared pools (``batched``),
        else one call per request.  Both take the same pages in the same
        order."""
        for req in self.requests:
            req.bridge.retain_route_rows([])
        bridges = [r.bridge for r in self.requests]
        if self.batched:
            released = release_unreferenced_node_slots_many(bridges, [[] for _ in bridges])
        else:
            released = [b.release_unreferenced_node_slots([]) for b in bridges]
        for req, n in zip(self.requests, released):
            req.stats.append({"released_kv_pages": n})
        before = self.ids.next
        if self.batched:
            SGLangFlashInferFrontierModelBackend.append_known_tokens_as_prefix_many(
                [r.backend for r in self.requests], [r.plan.extend_tokens for r in self.requests])
        else:
            for req in self.requests:
                req.backend.append_known_tokens_as_prefix(req.plan.extend_tokens)
        for req in self.requests:
            n = len(req.plan.extend_tokens)
            req.prefix_value_ids = req.prefix_value_ids + list(range(before, before + n))
            before += n
            req.active = [req.store.new_root_route(req.rng.randrange(VOCAB),
                                                   req.store.prefix_view(len(req.backend.prefix_token_ids)))]
        # The logical store's committed tokens lag the EXTEND suffix; the
        # root's prefix view carries the true committed length.
        self._post_steps()

    def run(self, on_phase: Callable[[str], None] | None = None) -> None:
        cb = on_phase or (lambda _name: None)
        self.prefill()
        cb("prefill")
        self.stage1(cb)
        self.commit()
        cb("commit")
        self.post_decode()
        cb("post_decode")
        self.fallback_extend()
        cb("extend")

    @staticmethod
    def route_score(req: RequestState, route: RouteState) -> float:
        """Sum of the log-probs of a route's materialized nodes, in node order."""
        total = 0.0
        for n in route.kv_view.node_ids:
            total += req.node_logprobs[int(n)]
        return total

    # ------------------------------------------------------------ expected content
    def expected_path_values(self, req: RequestState, route: RouteState) -> list[int]:
        """Value ids a route's slot path must hold: the committed prefix's,
        then one per materialized node."""
        n = int(route.kv_view.prefix.committed_length)
        return req.prefix_value_ids[:n] + [req.node_value_ids[int(x)] for x in route.kv_view.node_ids]
