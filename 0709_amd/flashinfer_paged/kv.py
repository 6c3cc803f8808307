"""Logical route / node store driving the route pool and the frontier (the
parts of reference ``flashinfer_paged/kv.py:21-258`` those paths use).

Nodes and routes are ids only; the physical KV of a node lives wherever the
route pool placed it.  Ids start at 1 and increase (``kv.py:30-31``).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Sequence

from .types import DecodePhase, PendingCandidate, PrefixKVView, RouteKVView, RouteState


@dataclass
class KVTreeNode:
    node_id: int
    token_id: int
    parent_node_id: int | None
    stage1_root_id: int
    depth: int
    owner_route_id: int | None = None
    committed: bool = False


class KVTreeStore:
    def __init__(self) -> None:
        self._next_route = 1
        self._next_node = 1
        self.nodes: dict[int, KVTreeNode] = {}
        self.routes: dict[int, RouteState] = {}
        self.committed_token_ids: list[int] = []
        self._release_hooks: list[Callable[[Sequence[RouteState], Sequence[RouteState]], None]] = []

    def reset_speculative(self) -> None:
        """Forget every node and route; the committed tokens and the id
        counters stay (``kv.py:37-39``: the fallback EXTEND handoff drops the
        speculative forest this way before rebuilding stage 1)."""
        self.nodes.clear()
        self.routes.clear()

    def add_route_release_hook(self, hook) -> None:
        self._release_hooks.append(hook)

    def allocate_route_id(self) -> int:
        rid, self._next_route = self._next_route, self._next_route + 1
        return rid

    def allocate_node_id(self) -> int:
        nid, self._next_node = self._next_node, self._next_node + 1
        return nid

    def reserve_node_ids(self, num_nodes: int) -> list[int]:
        return [self.allocate_node_id() for _ in range(int(num_nodes))]

    def prefix_view(self, committed_length: int | None = None) -> PrefixKVView:
        n = len(self.committed_token_ids) if committed_length is None else int(committed_length)
        return PrefixKVView(committed_length=n)

    def register_route(self, route: RouteState) -> RouteState:
        self.routes[int(route.route_id)] = route
        return route

    def get_route(self, route_id: int) -> RouteState:
        return self.routes[int(route_id)]

    def get_routes(self, route_ids) -> list[RouteState]:
        return [self.get_route(r) for r in route_ids]

    def node_counter_state(self) -> tuple[int, int]:
        """(next node id, step) without consuming an id."""
        return self._next_node, 1

    def new_root_route(self, pending_token_id: int, prefix: PrefixKVView) -> RouteState:
        rid = self.allocate_route_id()
        return self.register_route(RouteState(route_id=rid, stage1_root_id=rid, parent_route_id=None,
                                              materialized_leaf_node_id=None, pending_token_id=int(pending_token_id),
                                              cumulative_logprob=0.0, stage1_depth=0, stage2_depth=0,
                                              kv_view=prefix.fork()))

    def mark_routes_materialized(self, routes: Sequence[RouteState], new_node_ids: Sequence[int],
                                 phase: DecodePhase = DecodePhase.STAGE1) -> list[RouteState]:
        """Each route's pending token becomes node ``new_node_ids[i]`` at the
        end of its path (``kv.py:57-100``)."""
        if len(routes) != len(new_node_ids):
            raise ValueError("routes and new_node_ids must have the same length")
        for route, raw in zip(routes, new_node_ids):
            nid = int(raw)
            parent = route.kv_view.node_ids[-1] if route.kv_view.node_ids else None
            self.nodes[nid] = KVTreeNode(nid, int(route.pending_token_id), parent, route.stage1_root_id,
                                         route.total_materialized_depth() + 1, owner_route_id=route.route_id)
            route.materialized_leaf_node_id = nid
            route.kv_view = route.kv_view.append_node(nid)
            if phase == DecodePhase.STAGE1:
                route.stage1_depth += 1
            elif phase == DecodePhase.STAGE2:
                route.stage2_depth += 1
            else:
                raise ValueError(f"unsupported decode phase: {phase}")
            self.register_route(route)
        return list(routes)

    def clone_route_with_new_pending(self, route: RouteState, pending_token_id: int,
                                     cumulative_logprob: float = 0.0) -> RouteState:
        """A child sharing the parent's path with its own pending token
        (``kv.py:231-258``)."""
        rid = self.allocate_route_id()
        return self.register_route(RouteState(
            route_id=rid, stage1_root_id=route.stage1_root_id, parent_route_id=route.route_id,
            materialized_leaf_node_id=route.materialized_leaf_node_id, pending_token_id=int(pending_token_id),
            cumulative_logprob=float(cumulative_logprob), stage1_depth=route.stage1_depth,
            stage2_depth=route.stage2_depth, kv_view=route.kv_view.fork()))

    def materialize_route_descriptors(self, selected: Sequence[PendingCandidate],
                                      parent_routes: Sequence[RouteState]) -> list[RouteState]:
        """One new route per selected candidate, forked from its parent route,
        with the candidate's token pending (``kv.py:113-152``)."""
        parents = {route.route_id: route for route in parent_routes}
        out: list[RouteState] = []
        for cand in selected:
            parent = parents.get(cand.parent_route_id)
            if parent is None:
                parent = self.get_route(cand.parent_route_id)
            rid = self.allocate_route_id()
            if parent.token_logprobs and len(parent.token_logprobs) != parent.total_materialized_depth():
                raise ValueError(
                    "decoded parent token_logprobs must match its materialized path: "
                    f"route_id={parent.route_id}, logprobs={len(parent.token_logprobs)}, "
                    f"materialized_depth={parent.total_materialized_depth()}")
            local = float(cand.cumulative_logprob - cand.parent_logprob)
            route = RouteState(route_id=rid, stage1_root_id=cand.stage1_root_id, parent_route_id=parent.route_id,
                               materialized_leaf_node_id=parent.materialized_leaf_node_id,
                               pending_token_id=int(cand.pending_token_id),
                               cumulative_logprob=float(cand.cumulative_logprob), stage1_depth=parent.stage1_depth,
                               stage2_depth=parent.stage2_depth, kv_view=parent.kv_view.fork(),
                               token_logprobs=(*parent.token_logprobs, local) if parent.token_logprobs else ())
            out.append(self.register_route(route))
        return out

    def release_routes_without_descendants(self, previous: Sequence[RouteState], nxt: Sequence[RouteState]) -> None:
        for hook in self._release_hooks:
            hook(previous, nxt)

    def tokens_for_node_ids(self, node_ids: Sequence[int]) -> tuple[int, ...]:
        return tuple(self.nodes[int(n)].token_id for n in node_ids)

    def tokens_for_view(self, kv_view: RouteKVView) -> tuple[int, ...]:
        return self.tokens_for_node_ids(kv_view.node_ids)

    def materialized_token_path(self, route: RouteState) -> tuple[int, ...]:
        return self.tokens_for_view(route.kv_view)

    def pending_token_path(self, route: RouteState) -> tuple[int, ...]:
        return (*self.materialized_token_path(route), int(route.pending_token_id))

    def node_path_for_route(self, route: RouteState) -> tuple[int, ...]:
        return tuple(route.kv_view.node_ids)

    def commit_route(self, route: RouteState, max_tokens: int | None = None) -> tuple[int, ...]:
        nodes = self.node_path_for_route(route)
        if max_tokens is not None:
            nodes = nodes[:max_tokens]
        for n in nodes:
            self.nodes[n].committed = True
        tokens = self.tokens_for_node_ids(nodes)
        self.committed_token_ids.extend(tokens)
        return tokens

    def promote_routes_after_commit(self, committed_route: RouteState, routes: Sequence[RouteState],
                                    new_prefix: PrefixKVView) -> list[RouteState]:
        """Rebase retained routes onto the new prefix: drop the committed node
        path, stage-2 depth becomes stage-1, each route is its own root
        (``kv.py:193-229``)."""
        committed = self.node_path_for_route(committed_route)
        out = []
        for route in routes:
            if route.kv_view.node_ids[: len(committed)] != committed:
                raise ValueError("cannot promote a route outside the committed branch")
            suffix = route.kv_view.node_ids[len(committed):]
            if route.token_logprobs:
                depth = route.total_materialized_depth()
                if len(route.token_logprobs) not in (depth, depth + 1):
                    raise ValueError(
                        "promoted route token_logprobs do not match its token path: "
                        f"route_id={route.route_id}, logprobs={len(route.token_logprobs)}, "
                        f"valid_lengths={[depth, depth + 1]}")
                route.token_logprobs = tuple(route.token_logprobs[len(committed):])
            route.kv_view = RouteKVView(prefix=new_prefix, node_ids=tuple(suffix))
            route.materialized_leaf_node_id = suffix[-1] if suffix else None
            route.stage1_depth = route.stage2_depth
            route.stage2_depth = 0
            route.stage1_root_id = route.route_id
            route.parent_route_id = None
            self.register_route(route)
            out.append(route)
        return out
