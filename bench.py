"""Benchmark of the paged-KV tree path on one MI355X.

Headline step (Llama-3.1-8B KV geometry, fp16, page 16, 32 layers, committed
prefix 16384, forest of k^2 = 9 routes of depth 4 deduplicated to <= 36
nodes, prefix pages in a random permutation of the pool):

    dedup + mask + attention plan (host)
    32 x [ write the tree nodes' K/V (append kernel) ; masked verify attention ]
    route scoring on device (log-sum-exp + gather) -> best route (host)
    commit the selected route into the prefix (one all-layer launch)
    prune: free the pages that only held tree nodes (mark/sweep kernels)

``value`` is the verify attention time per layer: HIP events around
back-to-back replays of a graph holding the 32 layers' attention launches
(the same launches the timed steps replay inside the forward graph).  Two more legs measure the KV
bandwidth kernels at their bandwidth-sized configurations: the batched
32-request commit (bf16, pages scattered over a large pool) and the Drafter
tail-page copy-on-write of 8 requests x 9 forked routes (Llama-3.2-1B KV
geometry, bf16, page 64).  The CPU baseline is the oracle's float32
attention on a bounded sample of the same layers, on the host cores.
"""

from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
METRIC = "tree-verify attn µs/layer + KV commit/COW GB/s, 8B geom, 16k prefix, 1 GPU"


def _measured_traffic(path: Path) -> int | None:
    """HBM bytes per attention launch pair from the committed counter summary
    (``hbm_bytes_per_launch: N`` in its text block), or None."""
    try:
        for line in path.read_text().splitlines():
            if line.startswith("hbm_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        return None
    return None


def _pkg(name):
    return importlib.import_module(f"0709_amd.{name}")


def _ev():
    return torch.cuda.Event(enable_timing=True)


# Planner settings given on the command line, applied to every verify
# attention wrapper the bench builds (headline and attention legs).
PLAN_TUNING: dict = {}

# Page layout of the Target KV pools the bench builds: "HND" pages
# [pages, 2, Hkv, page_size, D] (each KV head's keys of a page contiguous,
# the layout the verify attention reads fastest) or the reference's "NHD"
# [pages, 2, page_size, Hkv, D].
KV_LAYOUT = "HND"


class HeadlineStep:
    def __init__(self, dev, *, prefix_len=16384, page_size=16, seed=0, split_target=None, max_rows=None,
                 routes=None):
        wl = _pkg("workloads")
        ffv = _pkg("flashinfer_full_verify")
        self.ffv = ffv
        self.kv_ops = _pkg("kv_ops")
        self.tr = _pkg("target_runtime")
        self.lib = _pkg("_lib")
        self.dev = dev
        self.geom = wl.LLAMA_8B
        self.prefix_len = prefix_len
        self.ps = page_size
        self.routes = wl.forest_routes(seed) if routes is None else list(routes)
        spec, _ = ffv.build_deduplicated_tree_spec_from_paths(paths=self.routes, prefix_len=prefix_len,
                                                              page_size=page_size, device=dev)
        self.n = spec.node_count
        self.kv_len = prefix_len + self.n
        self.pages = math.ceil(self.kv_len / page_size)
        self.kv_layout = KV_LAYOUT
        self.kv = wl.make_paged_target_kv(self.geom, kv_len=self.kv_len, page_size=page_size, dtype=torch.float16,
                                          device=dev, seed=seed, spare_pages=64, kv_layout=self.kv_layout)
        self.layers = self.kv.layers
        self.q = wl.random_queries(self.geom, self.n, dtype=torch.float16, device=dev, seed=seed + 7)
        g = torch.Generator(device=dev).manual_seed(seed + 11)
        shp = (self.n, self.geom.kv_heads, self.geom.head_dim)
        self.k_new = [(torch.randn(shp, generator=g, device=dev) * 0.1).half() for _ in range(self.geom.layers)]
        self.v_new = [(torch.randn(shp, generator=g, device=dev) * 0.1).half() for _ in range(self.geom.layers)]
        # rotary tables of the tree positions (prefix_len + depth), fp32 angles
        # rounded to the dtype, Llama-3.1 theta
        inv = 1.0 / (500000.0 ** (torch.arange(0, self.geom.head_dim, 2, dtype=torch.float32) / self.geom.head_dim))
        emb = torch.outer((prefix_len + spec.depths.cpu()).float(), inv)
        emb = torch.cat((emb, emb), dim=-1)
        self.rope_cos, self.rope_sin = emb.cos().half().to(dev), emb.sin().half().to(dev)
        self.verify_logits = (torch.randn((self.n, 128256), generator=g, device=dev) * 2.0).half()
        self.prefix_logits = (torch.randn((128256,), generator=g, device=dev) * 2.0).half()
        ws = torch.empty(256 * 1024 * 1024, dtype=torch.uint8, device=dev)
        self.wrapper = ffv.BatchPrefillWithPagedKVCacheWrapper(ws, self.kv_layout)
        for key, value in PLAN_TUNING.items():
            setattr(self.wrapper, key, value)
        if split_target is not None:
            self.wrapper.split_target_items = split_target
        if max_rows is not None:
            self.wrapper.max_rows_per_item = max_rows
        self.kv_indices_host = self.kv.kv_indices.cpu().tolist()
        # physical slots of the tree node positions (page table lookup on host, once)
        pos = torch.arange(prefix_len, self.kv_len)
        idx = torch.tensor(self.kv_indices_host, dtype=torch.int64)
        self.tree_slots = (idx[pos // page_size] * page_size + pos % page_size).to(dev)
        # the plan reads these back on the host: their values travel with them
        # (as with the tree builder's own index tensors), so no device read
        last = self.kv_len - (self.pages - 1) * page_size
        self.kv_indptr = ffv.with_host_values(torch.tensor([0, self.pages], dtype=torch.int32, device=dev),
                                              [0, self.pages])
        self.last = ffv.with_host_values(torch.tensor([last], dtype=torch.int32, device=dev), [last])
        # page ownership of the pool for the prune
        pool_pages = int(self.kv.pool.shape[1])
        self.pool_pages = pool_pages
        words = (pool_pages + 31) // 32
        self.owned = torch.zeros(words, dtype=torch.int32, device=dev)
        self.live = torch.zeros(words, dtype=torch.int32, device=dev)
        self.free_pages = torch.zeros(pool_pages, dtype=torch.int64, device=dev)
        self.free_count = torch.zeros(1, dtype=torch.int64, device=dev)
        all_pos = torch.arange(self.kv_len)
        self.all_slots = (idx[all_pos // page_size] * page_size + all_pos % page_size).to(dev)
        self.live_path = (self.lib.SlotPath * 1)()
        # the Target runtime's scoring and selection (target_best, logits-dtype
        # rounding, no thresholds), without a model
        self.backend = object.__new__(self.tr.DirectFlashInferMaskedTreeVerifyBackend)
        self.backend.score_weights = None
        self.backend.route_selection_policy = "target_best"
        self.backend.match_logits_dtype_rounding = True
        self.backend.fallback_threshold = None
        self.backend.first_token_threshold = None
        self.live_path[0].slots = self.all_slots.data_ptr()
        self.fwd_events = []
        self.commit_events = []
        self.prune_events = []
        self.record = False

    def _timed(self, bucket, fn):
        if not self.record:
            return fn()
        a, b = _ev(), _ev()
        a.record()
        r = fn()
        b.record()
        bucket.append((a, b))
        return r

    def plan(self):
        spec, route_nodes = self.ffv.build_deduplicated_tree_spec_from_paths(
            paths=self.routes, prefix_len=self.prefix_len, page_size=self.ps, device=self.dev)
        self.wrapper.plan(spec.qo_indptr, self.kv_indptr, self.kv.kv_indices, self.last, self.geom.q_heads,
                          self.geom.kv_heads, self.geom.head_dim, self.ps, custom_mask=spec.bool_mask,
                          causal=False, q_data_type=torch.float16)
        return route_nodes

    def _rotate(self, x):
        h = x.shape[-1] // 2
        cos, sin = self.rope_cos[:, None, :], self.rope_sin[:, None, :]
        return (x * cos) + (torch.cat((-x[..., h:], x[..., :h]), dim=-1) * sin)

    def forward(self, with_append=True, fused=True, rope=None, with_lse=False):
        """The per-layer device work of the verify forward: write the tree
        nodes' K/V, then masked attention.  ``fused``: both in one launch per
        layer (the rows are written inside the attention kernel); otherwise
        an append launch, then the attention.  ``rope``: the queries and keys
        arrive before the rotary embedding, which runs inside the launch
        ("fused") or as the reference's torch ops ahead of it ("torch")."""
        for l in range(self.geom.layers):
            layer = self.layers[l]
            if rope == "fused":
                self.wrapper.run(self.q[l], layer, out=self.outs[l], append_key_states=self.k_new[l],
                                 append_value_states=self.v_new[l], rope_cos_sin=(self.rope_cos, self.rope_sin))
                continue
            if rope == "torch":
                self.wrapper.run(self._rotate(self.q[l]), layer, out=self.outs[l],
                                 append_key_states=self._rotate(self.k_new[l]), append_value_states=self.v_new[l])
                continue
            if with_append and fused:
                self.wrapper.run(self.q[l], layer, out=self.outs[l], append_key_states=self.k_new[l],
                                 append_value_states=self.v_new[l])
                continue
            if with_append:
                self.kv_ops.append_paged([layer], [self.k_new[l]], [self.v_new[l]], dst_slots=self.tree_slots,
                                         kv_layout=self.kv_layout)
            self.wrapper.run(self.q[l], layer, out=self.outs[l], lse=self.lses[l] if with_lse else None)

    def capture(self):
        """HIP graphs of the 32-layer forward (append + attention) and of the
        attention launches alone.  plan() writes into the wrapper's persistent
        buffers, so replays use the plan of the current step."""
        self.outs = [torch.empty_like(q) for q in self.q]
        self.lses = [torch.empty(q.shape[:2], dtype=torch.float32, device=q.device) for q in self.q]
        self.plan()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.forward()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph_fwd_separate = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph_fwd_separate):
            self.forward(fused=False)
        self.graph_fwd_rope = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph_fwd_rope):
            self.forward(rope="fused")
        self.graph_fwd_torch_rope = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph_fwd_torch_rope):
            self.forward(rope="torch")
        self.graph_fwd = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph_fwd):
            self.forward()
        self.graph_attn = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph_attn):
            self.forward(with_append=False)
        torch.cuda.synchronize()

    def step(self):
        lib = self.lib
        stream = lib.stream_of(self.dev)
        route_nodes = self.plan()
        self._timed(self.fwd_events, self.graph_fwd.replay)
        # scoring, the route selection and the commit of the selected route
        # queued on the device behind the forward, then the prune; the host
        # waits only for the scores (and the device's choice, checked against
        # the runtime's host selection)
        backend = self.backend
        payloads = [self.tr.VerifyRoutePayload(route_id=i, token_ids=r, draft_logprob=0.0)
                    for i, r in enumerate(self.routes)]
        inputs = backend._device_selection_inputs(payloads, self.routes, route_nodes)
        depth = len(self.routes[0])
        # the live set: the committed path's page starts and its last slot,
        # sampled inside the prune launch
        self.live_path[0].len = self.prefix_len + depth

        def prune():
            # pages of the whole request (prefix + tree) are owned at verify
            # time; marked here, behind the selection and the commit, since
            # only the prune reads them
            rc = lib.load().atlas_mark_pages(lib.ptr(self.owned), self.pool_pages, lib.ptr(self.all_slots),
                                             self.kv_len, self.ps, stream)
            lib.check(rc, "atlas_mark_pages")
            rc = lib.load().atlas_prune_pages_paths(lib.ptr(self.owned), lib.ptr(self.live), self.pool_pages,
                                                    self.live_path, 1, 1, self.ps, lib.ptr(self.free_pages),
                                                    lib.ptr(self.free_count), stream)
            lib.check(rc, "atlas_prune_pages_paths")

        commit_mark = [None]

        def before_commit():
            if self.record:
                commit_mark[0] = _ev()
                commit_mark[0].record()

        def then():
            if self.record:
                end = _ev()
                end.record()
                self.commit_events.append((commit_mark[0], end))
            self._timed(self.prune_events, prune)

        scores, chosen, count = backend._score_select_commit(
            routes=payloads, paths=self.routes, prefix_logits=self.prefix_logits, verify_logits=self.verify_logits,
            route_to_node_paths=route_nodes, inputs=inputs, commit_lens=[depth] * len(self.routes),
            prefix_len=self.prefix_len, layers=self.layers, kv_indptr=self.kv_indptr, kv_indices=self.kv.kv_indices,
            kv_layout=self.kv_layout, before_commit=before_commit, then=then)
        best = backend._select_route(scores)
        if int(best.route_id) != chosen or count != depth:
            raise RuntimeError(f"device selection {chosen} ({count} tokens) differs from the host's {best.route_id}")
        # the pruned-page count stays on the device: nothing in the step waits
        # for it (the caller reads it once, after the timed steps)
        return int(best.route_id), count, self.free_count

    def attention_only(self, replays, graph=None):
        """ms per layer of back-to-back replays of the attention graph (or of
        ``graph``, another 32-layer graph)."""
        graph = graph if graph is not None else self.graph_attn
        torch.cuda.synchronize()
        a, b = _ev(), _ev()
        a.record()
        for _ in range(replays):
            graph.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / (replays * self.geom.layers)


def attention_leg(dev, *, prefix_len, routes, with_lse, replays=10):
    """Verify attention alone, 32 layers of Llama-3.1-8B KV geometry, fp16,
    page 16, from a HIP graph of the 32 layers' launches (each layer its own
    KV pages, so the working set exceeds the caches): µs per layer and the
    fraction of the HBM roofline."""
    wl = _pkg("workloads")
    step = HeadlineStep(dev, prefix_len=prefix_len, routes=routes)
    step.outs = [torch.empty_like(q) for q in step.q]
    step.lses = [torch.empty(q.shape[:2], dtype=torch.float32, device=q.device) for q in step.q]
    step.plan()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step.forward(with_append=False, with_lse=with_lse)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step.forward(with_append=False, with_lse=with_lse)
    graph.replay()
    us = step.attention_only(replays, graph) * 1000.0
    nbytes = wl.verify_attention_bytes(step.geom, kv_len=step.kv_len, nodes=step.n, page_size=step.ps)
    plan = step.wrapper.current_plan
    out = {"prefix_len": prefix_len, "nodes": step.n, "kv_len": step.kv_len, "lse": with_lse,
           "work_items": plan.num_work, "merge_items": plan.num_merge, "us_per_layer": round(us, 3),
           "bytes_per_layer": nbytes, "roofline_us": round(nbytes / (HBM_PEAK_GBPS * 1e3), 3),
           "GBps": round(nbytes / (us * 1e-6) / 1e9, 1), "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
           "tree_tokens_per_s": round(step.n / (us * 1e-6 * step.geom.layers), 1)}
    del step, graph
    torch.cuda.empty_cache()
    return out


def _mean_ms(pairs):
    return statistics.fmean(a.elapsed_time(b) for a, b in pairs) if pairs else float("nan")


def batched_leg(dev, *, pool_gb=200.0, requests=32, layers_timed=32, iters=5, profile_launches=0):
    """Batched Target verify: 32 requests, Llama-3.1-8B KV geometry, bf16,
    page 16, prefixes uniform in [1024, 16384], pages scattered over a pool of
    about ``pool_gb`` GB (32 layers x pages x 64 KiB).  Each request has a
    k=3 d=4 tree (12 queries, ancestor mask).  Times the 32-layer masked
    attention, then the per-request 4-token commit (dedup node ids: a one-pass
    in-place copy) and the prune of the tree pages."""
    kv_ops = _pkg("kv_ops")
    wl = _pkg("workloads")
    ffv = _pkg("flashinfer_full_verify")
    lib = _pkg("_lib")

    geom = wl.LLAMA_8B
    ps = 16
    page_bytes = 2 * ps * geom.kv_heads * geom.head_dim * 2
    need_pages = wl.batched_verify_need_pages(requests=requests, page_size=ps)
    pool = None
    while pool is None:
        pool_pages = max(need_pages + 64, int(pool_gb * 1e9 / (geom.layers * page_bytes)))
        try:
            page = (2, ps, geom.kv_heads, geom.head_dim) if KV_LAYOUT == "NHD" else (2, geom.kv_heads, ps,
                                                                                          geom.head_dim)
            pool = torch.empty((geom.layers, pool_pages) + page, dtype=torch.bfloat16, device=dev)
        except torch.cuda.OutOfMemoryError:
            pool_gb /= 2
            if pool_gb < 1:
                raise
    case = wl.batched_verify_case(pool_pages=pool_pages, requests=requests, page_size=ps)
    prefixes, routes, nodes, kv_lens, req_pages = case.prefixes, case.routes, case.nodes, case.kv_lens, case.req_pages
    specs = [ffv.build_deduplicated_tree_spec_from_paths(paths=r, prefix_len=p, page_size=ps, device=dev)
             for r, p in zip(routes, prefixes)]
    assert [sp.node_count for sp, _ in specs] == nodes
    perm = case.page_ids
    gen = torch.Generator().manual_seed(41)  # instances of the cold commit leg
    used = perm.to(dev)
    g = torch.Generator(device=dev).manual_seed(5)
    for l in range(geom.layers):
        pool[l, used] = (torch.randn((need_pages,) + page, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    layers = list(pool.unbind(0))
    kv_indptr_h = case.kv_indptr
    qo_h = case.qo_indptr
    flat_mask = torch.cat([sp.bool_mask for sp, _ in specs])
    kv_indptr = torch.tensor(kv_indptr_h, dtype=torch.int32, device=dev)
    kv_indices = perm.to(torch.int32).to(dev)
    last = torch.tensor([k - (n - 1) * ps for k, n in zip(kv_lens, req_pages)], dtype=torch.int32, device=dev)
    qo = torch.tensor(qo_h, dtype=torch.int32, device=dev)
    nnz = qo_h[-1]
    q = [(torch.randn((nnz, geom.q_heads, geom.head_dim), generator=g, device=dev) * 0.1).to(torch.bfloat16)
         for _ in range(layers_timed)]
    outs = [torch.empty_like(x) for x in q]
    ws = torch.empty(512 * 1024 * 1024, dtype=torch.uint8, device=dev)
    w = ffv.BatchPrefillWithPagedKVCacheWrapper(ws, KV_LAYOUT)
    w.plan(qo, kv_indptr, kv_indices, last, geom.q_heads, geom.kv_heads, geom.head_dim, ps, custom_mask=flat_mask,
           causal=False, q_data_type=torch.bfloat16)

    def fwd():
        for l in range(layers_timed):
            w.run(q[l], layers[l], out=outs[l])

    side = torch.cuda.Stream()
    a, b = _ev(), _ev()
    if not profile_launches:
        fwd()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fwd()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fwd()
        graph.replay()
        torch.cuda.synchronize()
        print("batched leg: pool and plans ready", file=sys.stderr, flush=True)
        a.record()
        for _ in range(iters):
            graph.replay()
        b.record()
        torch.cuda.synchronize()
        attn_us = a.elapsed_time(b) * 1000.0 / (iters * layers_timed)
    attn_bytes = sum(wl.verify_attention_bytes(geom, kv_len=k, nodes=n, page_size=ps) for k, n in zip(kv_lens, nodes))

    # commit: the selected route of every request (dedup node ids)
    sel = case.selected
    item_req, src, dst = [], [], []
    for bi, ((_, rnodes), p) in enumerate(zip(specs, prefixes)):
        for i, nd in enumerate(rnodes[sel[bi]]):
            item_req.append(bi)
            src.append(p + nd)
            dst.append(p + i)
    staging = kv_ops.commit_positions_need_staging(src, dst, item_req)
    args = dict(kv_indptr=kv_indptr, kv_indices=kv_indices,
                item_req=torch.tensor(item_req, dtype=torch.int32, device=dev))
    src_t = torch.tensor(src, device=dev)
    dst_t = torch.tensor(dst, device=dev)
    if profile_launches:
        # eager commit launches for counter runs, each on its own page table
        # (the same positions on other physical pages), so every copy is cold
        for k in range(profile_launches):
            kv_idx = torch.randperm(pool_pages, generator=gen)[:need_pages].to(torch.int32).to(dev)
            kv_ops.commit_paged(layers, src_t, dst_t, needs_staging=staging, kv_layout=KV_LAYOUT, **dict(args, kv_indices=kv_idx))
            torch.cuda.synchronize()
            print(f"batched leg: commit launch {k} done", file=sys.stderr, flush=True)
        return {"profile_launches": profile_launches, "items": len(src), "moved_bytes":
                len(src) * geom.layers * geom.token_bytes()}
    for _ in range(5):
        kv_ops.commit_paged(layers, src_t, dst_t, needs_staging=staging, kv_layout=KV_LAYOUT, **args)
    torch.cuda.synchronize()
    print("batched leg: attention timed", file=sys.stderr, flush=True)
    a.record()
    for _ in range(50):
        kv_ops.commit_paged(layers, src_t, dst_t, needs_staging=staging, kv_layout=KV_LAYOUT, **args)
    b.record()
    torch.cuda.synchronize()
    commit_call_us = a.elapsed_time(b) * 1000.0 / 50
    # Device time of the commit launch, from HIP graphs (no per-call host
    # work between launches).  Cold: 40 commit instances in rotation, each
    # with its own page table (the same positions on other physical pages),
    # 1.3 GB of rows in all, more than L2 plus the 256 MB Infinity Cache, so
    # every copy streams from and to HBM.  Hot: one instance repeated (its
    # 16 MiB of rows stay in the caches).
    n_inst = 40
    inst_args = [args] + [dict(args, kv_indices=torch.randperm(pool_pages, generator=gen)[:need_pages]
                               .to(torch.int32).to(dev)) for _ in range(n_inst - 1)]
    with torch.cuda.stream(side):
        kv_ops.commit_paged(layers, src_t, dst_t, needs_staging=staging, kv_layout=KV_LAYOUT, **args)
    torch.cuda.current_stream().wait_stream(side)
    cgraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(cgraph):
        for k in range(n_inst):
            kv_ops.commit_paged(layers, src_t, dst_t, needs_staging=staging, kv_layout=KV_LAYOUT, **inst_args[k])
    hgraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(hgraph):
        for _ in range(20):
            kv_ops.commit_paged(layers, src_t, dst_t, needs_staging=staging, kv_layout=KV_LAYOUT, **args)
    cgraph.replay()
    hgraph.replay()
    torch.cuda.synchronize()
    print("batched leg: commit instances ready", file=sys.stderr, flush=True)
    a.record()
    for _ in range(5):
        cgraph.replay()
    b.record()
    torch.cuda.synchronize()
    commit_us = a.elapsed_time(b) * 1000.0 / (5 * n_inst)
    a.record()
    for _ in range(5):
        hgraph.replay()
    b.record()
    torch.cuda.synchronize()
    print("batched leg: commit timed", file=sys.stderr, flush=True)
    hot_commit_us = a.elapsed_time(b) * 1000.0 / 100
    moved = len(src) * geom.layers * geom.token_bytes()
    floors = commit_floors(dev, layers, inst_args, item_req, src, dst, moved, ps, side, lib)

    # prune: pages of every request owned; live = prefix + committed tokens
    words = (pool_pages + 31) // 32
    owned = torch.zeros(words, dtype=torch.int32, device=dev)
    live_bm = torch.zeros_like(owned)
    free_pages = torch.zeros(pool_pages, dtype=torch.int64, device=dev)
    free_count = torch.zeros(1, dtype=torch.int64, device=dev)
    idx_all = perm.to(torch.int64)
    live_sampled, all_page_slots = [], []
    for bi, (p, npg) in enumerate(zip(prefixes, req_pages)):
        pg = idx_all[kv_indptr_h[bi]: kv_indptr_h[bi + 1]]
        all_page_slots.append(pg * ps)
        keep = p + len(routes[bi][sel[bi]])
        pos = torch.arange(0, keep, ps).tolist() + [keep - 1]
        live_sampled.append(pg[torch.tensor(pos) // ps] * ps + torch.tensor(pos) % ps)
    all_slots = torch.cat(all_page_slots).to(dev)
    live_slots = torch.cat(live_sampled).to(dev)
    stream = lib.stream_of(dev)
    L = lib.load()

    def prune():
        rc = L.atlas_mark_pages(lib.ptr(owned), pool_pages, lib.ptr(all_slots), int(all_slots.numel()), ps, stream)
        lib.check(rc, "atlas_mark_pages")
        rc = L.atlas_prune_pages(lib.ptr(owned), lib.ptr(live_bm), pool_pages, lib.ptr(live_slots),
                                 int(live_slots.numel()), ps, lib.ptr(free_pages), lib.ptr(free_count), stream)
        lib.check(rc, "atlas_prune_pages")

    prune()
    torch.cuda.synchronize()
    a.record()
    for _ in range(20):
        prune()
    b.record()
    torch.cuda.synchronize()
    prune_us = a.elapsed_time(b) * 1000.0 / 20
    freed = int(free_count.item())
    out = {
        "requests": requests, "nodes_per_request": nodes[0], "mean_prefix": round(sum(prefixes) / requests, 1),
        "pool_GB": round(pool.numel() * 2 / 1e9, 1), "work_items": w.current_plan.num_work,
        "attention_us_per_layer": round(attn_us, 3),
        "attention_GBps": round(attn_bytes / (attn_us * 1e-6) / 1e9, 1),
        "attention_frac": round(attn_bytes / (attn_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
        "attention_bytes_per_layer": attn_bytes,
        "commit_us": round(commit_us, 3), "commit_call_us": round(commit_call_us, 3), "commit_moved_bytes": moved,
        "commit_GBps": round(2 * moved / (commit_us * 1e-6) / 1e9, 1), "commit_staging": bool(staging),
        "commit_instances": n_inst, "hot_commit_us": round(hot_commit_us, 3),
        "hot_commit_GBps": round(2 * moved / (hot_commit_us * 1e-6) / 1e9, 1),
        "mark_and_prune_us": round(prune_us, 3), "pruned_pages": freed,
        **floors,
    }
    del pool, layers, q, outs, ws, graph, cgraph, hgraph, inst_args
    torch.cuda.empty_cache()
    return out


def commit_floors(dev, layers, inst_args, item_req, src, dst, moved, ps, side, lib):
    """Cold floors for the batched commit, each from a HIP graph over the same
    40 instances as ``commit_us``: the same K/V rows (every layer) moved by the
    commit kernel with their slots resolved through the page tables on the
    host (identity page table on the device, so no lookups before the rows),
    and a plain contiguous device copy of as many bytes (torch copy_, 40
    source / destination pairs, 1.3 GB)."""
    kv_ops = _pkg("kv_ops")
    n_inst = len(inst_args)
    slot_sets = []
    for args in inst_args:
        idx = args["kv_indices"].cpu().to(torch.int64)
        indptr = args["kv_indptr"].cpu().tolist()

        def slot(req, pos):
            return int(idx[indptr[req] + pos // ps]) * ps + pos % ps

        slot_sets.append((torch.tensor([slot(r, p) for r, p in zip(item_req, src)], device=dev),
                          torch.tensor([slot(r, p) for r, p in zip(item_req, dst)], device=dev)))

    def rows(k):
        s_t, d_t = slot_sets[k]
        kv_ops.commit_paged(layers, s_t, d_t, needs_staging=False, kv_layout=KV_LAYOUT)

    bufs = torch.empty((2 * n_inst, moved), dtype=torch.uint8, device=dev)
    bufs.fill_(1)
    with torch.cuda.stream(side):
        rows(0)
        bufs[1].copy_(bufs[0])
    torch.cuda.current_stream().wait_stream(side)
    g_rows = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_rows):
        for k in range(n_inst):
            rows(k)
    g_copy = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_copy):
        for k in range(n_inst):
            bufs[2 * k + 1].copy_(bufs[2 * k])
    out = {}
    for name, g in (("floor_same_rows_no_lookup_us", g_rows), ("floor_contiguous_copy_us", g_copy)):
        g.replay()
        torch.cuda.synchronize()
        a, b = _ev(), _ev()
        a.record()
        for _ in range(5):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        out[name] = round(a.elapsed_time(b) * 1000.0 / (5 * n_inst), 3)
    del bufs, g_rows, g_copy
    return out


def cow_leg(dev, *, requests=8, routes=9, iters=50, instances=8, profile_launches=0):
    """Drafter tail-page copy-on-write: per request, 9 forked routes share a
    partially filled 64-token tail page; 8 of them get private copies, all in
    one move launch (Llama-3.2-1B KV geometry, bf16, flat token pool).

    ``instances`` independent copy-on-write steps (disjoint source and
    destination pages, 189 MB of source plus destination rows each) are
    timed in rotation, so the working set (1.5 GB) exceeds L2 and the 256 MB
    Infinity Cache and every copy streams from and to HBM.  The same step
    repeated on one instance (``hot_*``) runs from those caches.  ``us`` is the
    device time per launch from a HIP graph; ``call_us`` the eager per-call
    time with the host work between launches."""
    kv_ops = _pkg("kv_ops")
    wl = _pkg("workloads")
    geom = wl.LLAMA_1B
    ps = 64
    pool_pages = 4096
    gen = torch.Generator().manual_seed(5)
    k_layers = [torch.empty((pool_pages * ps, geom.kv_heads, geom.head_dim), dtype=torch.bfloat16, device=dev)
                for _ in range(geom.layers)]
    v_layers = [torch.empty_like(k_layers[0]) for _ in range(geom.layers)]
    perm = torch.randperm(pool_pages, generator=gen)
    tail_lens = [int(torch.randint(1, ps, (1,), generator=gen)) for _ in range(requests)]
    sets = []
    j = 0
    for _ in range(instances):
        src, dst = [], []
        for b in range(requests):
            tail_page = int(perm[j])
            j += 1
            for _ in range(routes - 1):
                new_page = int(perm[j])
                j += 1
                src.extend(tail_page * ps + o for o in range(tail_lens[b]))
                dst.extend(new_page * ps + o for o in range(tail_lens[b]))
        sets.append((torch.tensor(dst, device=dev), torch.tensor(src, device=dev)))
    slots = int(sets[0][1].numel())
    for d_t, s_t in sets:
        kv_ops.move_slots(k_layers, v_layers, d_t, s_t)
    torch.cuda.synchronize()
    print("cow leg: instances ready", file=sys.stderr, flush=True)
    if profile_launches:
        # eager launches in rotation over the instances, for counter runs
        for i in range(profile_launches):
            d_t, s_t = sets[i % instances]
            kv_ops.move_slots(k_layers, v_layers, d_t, s_t)
            torch.cuda.synchronize()
            print(f"cow leg: move launch {i} done", file=sys.stderr, flush=True)
        return {"profile_launches": profile_launches, "slots": slots,
                "moved_bytes": slots * geom.layers * geom.token_bytes()}
    a, b = _ev(), _ev()
    # Per eager call: host work between launches included.
    a.record()
    for i in range(iters):
        d_t, s_t = sets[i % instances]
        kv_ops.move_slots(k_layers, v_layers, d_t, s_t)
    b.record()
    torch.cuda.synchronize()
    call_us = a.elapsed_time(b) * 1000.0 / iters
    # Device time of the launch, from a HIP graph of the instances in
    # rotation (no host work between launches), as the commit leg is timed.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        kv_ops.move_slots(k_layers, v_layers, sets[0][0], sets[0][1])
    torch.cuda.current_stream().wait_stream(side)
    rounds = max(1, iters // instances)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(rounds * instances):
            d_t, s_t = sets[i % instances]
            kv_ops.move_slots(k_layers, v_layers, d_t, s_t)
    hgraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(hgraph):
        for _ in range(rounds * instances):
            kv_ops.move_slots(k_layers, v_layers, sets[0][0], sets[0][1])
    graph.replay()
    hgraph.replay()
    torch.cuda.synchronize()
    a.record()
    for _ in range(3):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    print("cow leg: graph timed", file=sys.stderr, flush=True)
    us = a.elapsed_time(b) * 1000.0 / (3 * rounds * instances)
    a.record()
    for _ in range(3):
        hgraph.replay()
    b.record()
    torch.cuda.synchronize()
    hot_us = a.elapsed_time(b) * 1000.0 / (3 * rounds * instances)
    del graph, hgraph
    moved = slots * geom.layers * geom.token_bytes()
    return {"us": us, "moved_bytes": moved, "GBps": 2 * moved / (us * 1e-6) / 1e9, "slots": slots,
            "instances": instances, "working_set_bytes": 2 * moved * instances,
            "call_us": call_us, "call_GBps": 2 * moved / (call_us * 1e-6) / 1e9,
            "hot_us": hot_us, "hot_GBps": 2 * moved / (hot_us * 1e-6) / 1e9}


def decode_leg(dev, *, requests=8, routes=9, prefix_len=None, steps=8, iters=5, cascade=True, split_target=None):
    """Drafter paged decode attention (Llama-3.2-1B geometry: 16 layers, 32 q
    heads, 8 KV heads, head_dim 64; bf16, page 64): ``requests`` x ``routes``
    forked routes, one query each.  The routes of a request share its full
    prefix pages and own a private tail page (the copy-on-write copy of the
    partial prefix page plus ``steps`` decoded tokens).  Prefix lengths follow
    the fork-stress workload (128..1024 tokens) unless ``prefix_len`` is given.
    Times the 16 layers' decode attention replayed from a HIP graph; bytes are
    counted over unique pages (each shared page once) and per route."""
    da = _pkg("decode_attention")
    dw = _pkg("drafter_workload")
    geom = _pkg("workloads").LLAMA_1B
    ps = 64
    plans = dw.config5_plans(requests, ps, 0)
    prefixes = [p.prefix_len if prefix_len is None else int(prefix_len) for p in plans]
    gen = torch.Generator().manual_seed(9)
    indptr, indices, last = [0], [], []
    unique_pages = 0
    route_tokens = 0
    nxt = 0
    for pre in prefixes:
        full = pre // ps
        shared = list(range(nxt, nxt + full))
        nxt += full
        unique_pages += full
        for _ in range(routes):
            own = pre - full * ps + steps
            own_pages = (own + ps - 1) // ps
            pages = shared + list(range(nxt, nxt + own_pages))
            nxt += own_pages
            unique_pages += own_pages
            indices.extend(pages)
            indptr.append(len(indices))
            last.append(full * ps + own - (len(pages) - 1) * ps)
            route_tokens += full * ps + own
    pool_pages = nxt + 8
    perm = torch.randperm(pool_pages, generator=gen)
    phys = [int(perm[i]) for i in indices]
    batch = requests * routes
    page = (2, ps, geom.kv_heads, geom.head_dim) if KV_LAYOUT == "NHD" else (2, geom.kv_heads, ps, geom.head_dim)
    layers = [(torch.randn((pool_pages,) + page, device=dev) * 0.1).to(torch.bfloat16) for _ in range(geom.layers)]
    q = [(torch.randn((batch, geom.q_heads, geom.head_dim), device=dev) * 0.1).to(torch.bfloat16)
         for _ in range(geom.layers)]
    outs = [torch.empty_like(x) for x in q]
    ws = torch.empty(256 * 1024 * 1024, dtype=torch.uint8, device=dev)
    w = da.BatchDecodeWithPagedKVCacheWrapper(ws, KV_LAYOUT)
    w.use_cascade = cascade
    w.split_target_items = split_target
    w.plan(torch.tensor(indptr, dtype=torch.int32, device=dev), torch.tensor(phys, dtype=torch.int32, device=dev),
           torch.tensor(last, dtype=torch.int32, device=dev), geom.q_heads, geom.kv_heads, geom.head_dim, ps,
           data_type=torch.bfloat16, q_data_type=torch.bfloat16)

    def fwd():
        for l in range(geom.layers):
            w.run(q[l], layers[l], out=outs[l])

    fwd()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fwd()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fwd()
    graph.replay()
    torch.cuda.synchronize()
    a, b = _ev(), _ev()
    a.record()
    for _ in range(iters):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1000.0 / (iters * geom.layers)
    row = geom.token_bytes()  # K and V of one token, one layer
    q_bytes = 2 * batch * geom.q_heads * geom.head_dim * 2
    unique_bytes = unique_pages * ps * row + q_bytes
    route_bytes = route_tokens * row + q_bytes
    out = {
        "requests": requests, "routes_per_request": routes, "prefix_lens": sorted(set(prefixes))[:3] + (
            ["..."] if len(set(prefixes)) > 3 else []),
        "cascade_groups": w.cascade_groups, "work_items": w.current_plan.num_work,
        "merge_items": w.current_plan.num_merge,
        "us_per_layer": round(us, 3), "unique_bytes_per_layer": unique_bytes, "route_bytes_per_layer": route_bytes,
        "GBps_unique": round(unique_bytes / (us * 1e-6) / 1e9, 1),
        "frac_unique": round(unique_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
    }
    del layers, q, outs, ws, graph
    torch.cuda.empty_cache()
    return out


def frontier_leg(dev, *, rows=72, vocab=128256, k=3, iters=20):
    """One Drafter frontier depth at the 8-request x 9-route fork shape: 72
    parent rows of Llama-3.2-1B next-token logits (vocab 128256, bf16), k=3
    children per parent, the global top-3 of the 216 candidates.  Times the
    launch pair replayed from a HIP graph (device time; the logits are read
    by both launches, 18.5 MB from HBM), the whole per-depth call by wall
    clock (parent rows to the device, launch pair, one copy of the records
    back, host materialisation), and the same depth as the reference's
    sequence of torch ops on the same device."""
    fr = _pkg("flashinfer_paged.frontier")
    nat = _pkg("flashinfer_paged._frontier_native")
    types = _pkg("flashinfer_paged.types")
    lib = _pkg("_lib")
    g = torch.Generator(device=dev).manual_seed(17)
    logits = (torch.randn((rows, vocab), generator=g, device=dev) * 3.0).to(torch.bfloat16)
    routes = [types.RouteState(route_id=1 + i, stage1_root_id=1 + i // 9, parent_route_id=None,
                               materialized_leaf_node_id=None, pending_token_id=0,
                               cumulative_logprob=-0.125 * (i % 5), stage1_depth=1, stage2_depth=0,
                               kv_view=types.PrefixKVView(committed_length=64).fork()) for i in range(rows)]
    parent_info = fr._parent_info(routes, dev)

    def launch():
        return nat.frontier_topk(logits, k, parent_info=parent_info, select_mode=lib.FRONTIER_SELECT_GLOBAL,
                                 num_selected=k)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            launch()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = launch()
    torch.cuda.synchronize()
    a, b = _ev(), _ev()
    a.record()
    for _ in range(iters):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    device_us = a.elapsed_time(b) * 1000.0 / iters

    def depth():
        _, records, _ = fr._fused(routes, logits, k=k, sampling=None, relative_parent_paths=None,
                                  select_mode=lib.FRONTIER_SELECT_GLOBAL, num_selected=k)
        return fr._materialize_records(records, rows * k, k, (), 0, "not_applicable")[1]

    def torch_depth():
        # the reference's depth as torch ops: log_softmax + topk, candidate
        # columns from host lists, four stable argsorts, packed records, one copy
        lp, ids = torch.topk(torch.log_softmax(logits, dim=-1), k=k, dim=-1)
        rid = torch.tensor([r.route_id for r in routes], device=dev, dtype=torch.long).repeat_interleave(k)
        root = torch.tensor([r.stage1_root_id for r in routes], device=dev, dtype=torch.long).repeat_interleave(k)
        plp = torch.tensor([r.cumulative_logprob for r in routes], device=dev,
                           dtype=torch.float64).repeat_interleave(k)
        rank = torch.arange(k, device=dev, dtype=torch.long).repeat(rows)
        cum = plp + lp.reshape(-1).to(torch.float64)
        tok = ids.reshape(-1)
        order = torch.arange(rows * k, device=dev, dtype=torch.long)
        for values, desc in ((tok, False), (rank, False), (rid, False), (cum, True)):
            order = order.index_select(0, torch.argsort(values.index_select(0, order), dim=0, descending=desc,
                                                        stable=True))
        sel = order[:k]
        so = torch.full((rows * k,), -1, device=dev, dtype=torch.long)
        so[sel] = torch.arange(k, device=dev, dtype=torch.long)
        rec = torch.stack((torch.zeros_like(rid), rid, root, tok, rank, cum.view(torch.int64), plp.view(torch.int64),
                           so), dim=1)
        host = rec.cpu().tolist()
        return [(h[1], h[3]) for h in sorted((h for h in host if h[7] >= 0), key=lambda h: h[7])]

    def wall(fn, n):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            r = fn()
        return (time.perf_counter() - t0) * 1e6 / n, r

    call_us, chosen = wall(depth, iters)
    torch_us, chosen_t = wall(torch_depth, iters)
    assert [(c.parent_route_id, c.pending_token_id) for c in chosen] == chosen_t, "frontier selection mismatch"
    nbytes = rows * vocab * 2
    return {"rows": rows, "vocab": vocab, "k": k, "dtype": "bf16", "selection": "global top-3",
            "device_us": round(device_us, 3), "logits_bytes": nbytes,
            "GBps": round(nbytes / (device_us * 1e-6) / 1e9, 1),
            "frac": round(nbytes / (device_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
            "depth_call_us": round(call_us, 1), "torch_sequence_us": round(torch_us, 1)}


def drafter_leg(dev, *, requests=8, repeats=6, warmup=1, batched=True):
    """Drafter route-pool fork stress (Llama-3.2-1B KV geometry, bf16, page
    64): 8 requests, each forking to 9 routes at random fill levels of its
    partial tail page, 8 decode steps, commit + promote of 3 routes, prune,
    one 4-token fallback EXTEND and a decode step after it -- the route-pool
    bridge driving the native pools (device page ownership, batched
    copy-on-write, device slot allocation and page metadata).  The model is
    replaced by one all-layer K/V append per forward.  ``batched``: each
    decode step of the 8 requests is one fused frontier step (one launch for
    all 72 routes, one forward); else one bridge call per request.  Wall time
    per phase, GPU synchronised at each phase end; ``warmup`` untimed
    repetitions first (first calls, the allocator's first blocks), then the
    median over ``repeats``, each on fresh pools."""
    dw = _pkg("drafter_workload")
    npool = _pkg("flashinfer_paged.native_pool")
    geom = _pkg("workloads").LLAMA_1B
    ps = 64
    runs = []
    for rep in range(warmup + repeats):
        req_pool, kv, alloc = npool.create_native_pools(
            num_pages=640, page_size=ps, dtype=torch.bfloat16, head_num=geom.kv_heads, head_dim=geom.head_dim,
            layer_num=geom.layers, max_running_requests=128, max_context_len=4096, device=dev)
        rows = (torch.randn((2048, geom.kv_heads, geom.head_dim), device=dev) * 0.1).to(torch.bfloat16)

        model = [0.0]  # wall time inside the model stand-in since the last phase end

        def writer(slots, vids, kv=kv, rows=rows, model=model):
            t0 = time.perf_counter()
            n = int(slots.numel())
            kv.set_kv_buffer_all_layers(slots, [rows[:n]] * geom.layers, [rows[:n]] * geom.layers)
            model[0] += time.perf_counter() - t0

        # seeds 0, 1, 2 in turn: the timed repetitions cover each workload twice
        work = dw.DrafterForkWorkload(plans=dw.config5_plans(requests, ps, rep % 3), req_pool=req_pool,
                                      allocator=alloc,
                                      page_size=ps, device=dev, writer=writer, batched=batched)
        marks = []

        def on_phase(name, marks=marks, model=model):
            torch.cuda.synchronize()
            marks.append((name, time.perf_counter(), model[0]))
            model[0] = 0.0

        torch.cuda.synchronize()
        marks.append(("start", time.perf_counter(), 0.0))
        model[0] = 0.0
        work.run(on_phase)
        spans = {}
        for (_, t0, _), (name, t1, m) in zip(marks, marks[1:]):
            spans[name] = (t1 - t0) * 1e6
            spans[name + "/model"] = m * 1e6
        cow_pages = sum(r.bridge.cow_pages_copied for r in work.requests)
        cow_tokens = sum(r.bridge.cow_tokens_copied for r in work.requests)
        if rep >= warmup:
            runs.append((spans, cow_pages, cow_tokens))
        del work, req_pool, kv, alloc
    torch.cuda.empty_cache()
    decode = [statistics.fmean(sp[f"decode{t}"] for t in range(8)) for sp, _, _ in runs]
    decode_model = [statistics.fmean(sp[f"decode{t}/model"] for t in range(8)) for sp, _, _ in runs]
    return {
        "requests": requests, "routes_per_request": 9, "page_size": ps,
        "decode_step_us": round(statistics.median(decode), 1),
        "decode_step_model_standin_us": round(statistics.median(decode_model), 1),
        "decode_us_per_request_step": round(statistics.median(decode) / requests, 1),
        "decode_bridge_us_per_request_step": round(
            statistics.median(d - m for d, m in zip(decode, decode_model)) / requests, 1),
        "commit_promote_prune_us_per_request": round(statistics.median(sp["commit"] for sp, _, _ in runs) / requests,
                                                     1),
        "commit_promote_prune_us": round(statistics.median(sp["commit"] for sp, _, _ in runs), 1),
        "fallback_extend_us": round(statistics.median(sp["extend"] for sp, _, _ in runs), 1),
        "prefill_us": round(statistics.median(sp["prefill"] for sp, _, _ in runs), 1),
        "cow_pages_copied": runs[-1][1], "cow_tokens_copied": runs[-1][2],
        "batched_frontier_step": bool(batched),
        "note": "wall time of the host-driven bridge per phase (all 8 requests), model replaced by a K/V append "
                "(decode_step_model_standin_us: the part of decode_step_us spent in that append)",
    }


def cpu_baseline(step: HeadlineStep, budget_s: float):
    """Oracle float32 attention over a bounded number of the headline's layers."""
    import numpy as np

    from oracle import attention as oatt
    from oracle import paged_kv as ref

    try:
        from threadpoolctl import threadpool_info

        cores = max((int(i.get("num_threads", 1)) for i in threadpool_info()), default=1)
    except Exception:
        cores = os.cpu_count() or 1
    _, parents, _, _ = ref.dedup_tree(step.routes)
    mask = ref.ancestor_mask(parents, step.prefix_len)
    idx = step.kv_indices_host
    last = step.kv_len - (step.pages - 1) * step.ps
    times = []
    t_start = time.perf_counter()
    for l in range(step.geom.layers):
        layer = step.kv.nhd_layer(l).cpu().numpy()
        q = step.q[l].cpu().numpy()
        t0 = time.perf_counter()
        oatt.masked_attention(q, layer, [0, step.n], [0, step.pages], idx, [last], masks=[mask], dtype=np.float32)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s:
            break
    us = statistics.fmean(times) * 1e6
    return {"value": us, "unit": "µs/layer", "cores": cores, "kind": "port",
            "sample": f"oracle float32 masked attention, {len(times)} of 32 layers of the headline step "
                      f"(kv_len {step.kv_len}, {step.n} nodes)",
            "legs": cpu_kv_legs(step)}


def _median_us(fn, reps=20, warm=3):
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts) * 1e6


def cpu_kv_legs(step: HeadlineStep):
    """The reference's own torch ops for the KV legs, on the host cores
    (torch threads): the commit of the headline's selected route over 32
    layers (target_runtime.py:886-912), write_suffix_kv of its tree nodes in
    every layer (flashinfer_full_verify.py:1027-1042), the prune's live-page
    set algebra (sglang_runtime.py:507-539), and the copy-on-write of the
    8-request x 9-route fork (one move per copied page, every layer,
    sglang_runtime.py:760-785) at Llama-3.2-1B geometry, bf16, page 64.
    Median of 20 calls after 3 warm-ups, on CPU copies of the inputs."""
    from oracle import torch_path as tp

    torch.set_num_threads(os.cpu_count() or 1)
    cores = torch.get_num_threads()
    ps = step.ps
    # identity page order, as the reference's Target keeps its prefix KV
    layers = [torch.empty((step.pages, 2, ps, step.geom.kv_heads, step.geom.head_dim), dtype=torch.float16)
              for _ in range(step.geom.layers)]
    for l, layer in enumerate(layers):
        layer.copy_(step.kv.nhd_layer(l)[torch.tensor(step.kv_indices_host, device=step.dev).long()].cpu())
    k_new = [k.cpu() for k in step.k_new]
    v_new = [v.cpu() for v in step.v_new]
    _, parents, _, route_nodes = _oracle_dedup(step.routes)
    nodes = route_nodes[5 % len(route_nodes)]
    commit_us = _median_us(lambda: tp.commit_torch(layers, step.prefix_len, nodes, ps))
    append_us = _median_us(lambda: [tp.write_suffix_kv_torch(layer, k, v, step.prefix_len, ps)
                                    for layer, k, v in zip(layers, k_new, v_new)])
    owned = set(range(step.pages))
    live_path = torch.arange(step.prefix_len + len(nodes))
    prefix_slots = torch.arange(step.prefix_len)
    prune_us = _median_us(lambda: tp.prune_torch(owned, prefix_slots, [live_path], ps))
    # copy-on-write: the fork leg's shape on a compact pool (9 pages per request)
    geom = _pkg("workloads").LLAMA_1B
    cps, requests, routes = 64, 8, 9
    gen = torch.Generator().manual_seed(5)
    tail_lens = [int(torch.randint(1, cps, (1,), generator=gen)) for _ in range(requests)]
    slots = requests * routes * cps
    k_pool = [torch.randn((slots, geom.kv_heads, geom.head_dim)).to(torch.bfloat16) for _ in range(geom.layers)]
    v_pool = [torch.randn((slots, geom.kv_heads, geom.head_dim)).to(torch.bfloat16) for _ in range(geom.layers)]
    copies = []
    for b in range(requests):
        src = torch.arange(tail_lens[b]) + b * routes * cps
        for r in range(1, routes):
            copies.append((src + r * cps, src))
    cow_us = _median_us(lambda: tp.cow_copy_torch(k_pool, v_pool, copies))
    cow_bytes = 2 * sum(int(d.numel()) for d, _ in copies) * geom.layers * geom.token_bytes()
    commit_bytes = 2 * len(nodes) * step.geom.layers * step.geom.token_bytes()
    return {"cores": cores, "kind": "reference torch ops (oracle/torch_path.py)",
            "commit_us": round(commit_us, 1), "commit_GBps": round(commit_bytes / (commit_us * 1e-6) / 1e9, 2),
            "append_us": round(append_us, 1), "prune_us": round(prune_us, 1),
            "cow_8req_9routes_us": round(cow_us, 1), "cow_GBps": round(cow_bytes / (cow_us * 1e-6) / 1e9, 2),
            "sample": f"commit of {len(nodes)} tokens and append of {step.n} nodes over 32 layers of the headline "
                      f"step; prune of its {step.pages} pages; copy-on-write of {len(copies)} tail pages "
                      f"x 16 layers (1B geometry)"}


def _oracle_dedup(routes):
    from oracle import paged_kv as ref

    return ref.dedup_tree(routes)


def profile_attention(step: HeadlineStep, launches: int) -> None:
    """The headline's verify attention alone, eagerly, one layer per launch
    (the launch pair a counter run attributes to its kernels)."""
    step.outs = [torch.empty_like(q) for q in step.q]
    step.plan()
    torch.cuda.synchronize()
    plan = step.wrapper.current_plan
    print(f"profile: {plan.num_work} work items, {plan.num_merge} merge items, {launches} launches", flush=True)
    for i in range(launches):
        l = i % step.geom.layers
        step.wrapper.run(step.q[l], step.layers[l], out=step.outs[l])
        torch.cuda.synchronize()
        print(f"profile: launch {i} (layer {l}) done", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-baseline-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-legs", action="store_true")
    ap.add_argument("--legs", default="all", metavar="NAMES",
                    help="comma-separated component legs to run (config2, tree16k, batched, cow, decode, decode8k, "
                         "drafter, drafter_calls, frontier), default all")
    ap.add_argument("--split-target", type=int, default=None,
                    help="work items a verify attention plan aims at (headline and attention legs)")
    ap.add_argument("--split-granule", type=int, default=None, metavar="KEYS",
                    help="key granule of the attention splits (default: the planner's)")
    ap.add_argument("--max-rows", type=int, default=None)
    ap.add_argument("--kv-layout", choices=("HND", "NHD"), default=KV_LAYOUT,
                    help="page layout of the Target KV pools (default %(default)s)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="also run device-to-device copies of MIB MiB (calibrates HBM byte counters)")
    ap.add_argument("--commit-pool-gb", type=float, default=200.0)
    ap.add_argument("--profile-kv", type=int, default=0, metavar="N",
                    help="run N eager launches of the batched commit and of the copy-on-write move, then exit")
    ap.add_argument("--profile-attention", type=int, default=0, metavar="N",
                    help="only plan the headline step and run N eager attention launches (one per layer, "
                         "printing after each), for counter collection")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU; the path is data-parallel across requests "
                                   "and has no multi-GPU leg", "n_gpus": args.gpus}))
        sys.exit(2)
    dev = torch.device("cuda:0")
    globals()["KV_LAYOUT"] = args.kv_layout
    if args.split_target is not None:
        PLAN_TUNING["split_target_items"] = args.split_target
    if args.split_granule is not None:
        PLAN_TUNING["split_granule_keys"] = args.split_granule
    if args.profile_kv:
        # the commit and copy-on-write launches alone, eagerly, for counter
        # runs (after a copy of known size that calibrates the counters)
        if args.copy_calibration:
            src = torch.ones(args.copy_calibration << 20, dtype=torch.uint8, device=dev)
            dst = torch.empty_like(src)
            for _ in range(3):
                dst.copy_(src)
            torch.cuda.synchronize()
            del src, dst
        print(json.dumps({"commit": batched_leg(dev, pool_gb=args.commit_pool_gb, profile_launches=args.profile_kv),
                          "cow": cow_leg(dev, profile_launches=args.profile_kv)}))
        return
    step = HeadlineStep(dev, split_target=args.split_target, max_rows=args.max_rows)
    if args.copy_calibration:
        src = torch.ones(args.copy_calibration << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.profile_attention:
        profile_attention(step, args.profile_attention)
        return
    step.capture()
    print("headline: graphs captured", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        step.step()
    torch.cuda.synchronize()
    print("headline: warmup done", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        route, committed, freed = step.step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    freed = int(freed.item())
    # the step's parts timed with events, in as many further steps (outside
    # the timed region, so the event records do not add to ms_per_step)
    step.record = True
    for _ in range(args.steps):
        step.step()
    torch.cuda.synchronize()
    step.record = False
    ms_per_step = wall * 1000.0 / args.steps
    print("headline: timed steps done", file=sys.stderr, flush=True)
    attn_ms = step.attention_only(max(10, args.steps))
    attn_us = attn_ms * 1000.0
    wl = _pkg("workloads")
    bytes_layer = wl.verify_attention_bytes(step.geom, kv_len=step.kv_len, nodes=step.n, page_size=step.ps)
    achieved = bytes_layer / (attn_ms * 1e-3) / 1e9
    plan = step.wrapper.current_plan
    result = {
        "metric": METRIC,
        "value": round(attn_us, 3),
        "unit": "µs/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1)*0.1 K/V/Q, random token ids)",
        "config": {
            "workload": "forest dedup + 32-layer masked verify attention + commit + prune",
            "geometry": "Llama-3.1-8B KV (32 layers, 32 q heads, 8 kv heads, head_dim 128)",
            "prefix_len": step.prefix_len, "page_size": step.ps, "kv_layout": step.kv_layout,
            "routes": len(step.routes), "depth": 4,
            "nodes": step.n, "kv_len": step.kv_len, "work_items": plan.num_work, "merge_items": plan.num_merge,
            "tiles_per_split": plan.tiles_per_split,
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": _measured_traffic(ROOT / "profiles" / "tree_attn_forest16k_traffic.md"),
            "traffic_source": "profiles/tree_attn_forest16k_traffic.md (FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0, "
                              "copy-calibrated)",
            "kernel": "tree_attn_d128_kernel + tree_attn_merge_kernel (one verify attention launch pair)",
            "algorithmic_bytes_per_launch": bytes_layer,
        },
        "components": {
            "attention_us_per_layer": round(attn_us, 3),
            "forward_append_plus_attention_us_per_layer": round(_mean_ms(step.fwd_events) * 1000.0 / 32, 3),
            "forward_fused_us_per_layer": round(step.attention_only(20, step.graph_fwd) * 1000.0, 3),
            "forward_separate_append_us_per_layer": round(step.attention_only(20, step.graph_fwd_separate) * 1000.0,
                                                          3),
            "forward_fused_rope_us_per_layer": round(step.attention_only(20, step.graph_fwd_rope) * 1000.0, 3),
            "forward_torch_rope_then_fused_us_per_layer": round(
                step.attention_only(20, step.graph_fwd_torch_rope) * 1000.0, 3),
            "commit_us": round(_mean_ms(step.commit_events) * 1000.0, 3),
            "prune_us": round(_mean_ms(step.prune_events) * 1000.0, 3),
            "selected_route": route, "committed_tokens": committed, "pruned_pages": freed,
        },
    }
    result["components"]["committed_tokens_per_s"] = round(committed / (ms_per_step * 1e-3), 1)
    result["components"]["tree_tokens_per_s_attention"] = round(step.n / (attn_us * 1e-6 * step.geom.layers), 1)
    if not args.no_legs:
        wl = _pkg("workloads")
        legs = {
            # configuration 2 (one layer's shape: 4096 prefix, k=3 d=4 of
            # independent routes, 12 nodes, with the LSE) and the 16k-prefix
            # k=3 d=4 tree
            "config2": ("config2_4k_tree_lse", lambda: attention_leg(dev, prefix_len=4096,
                                                                     routes=wl.tree_routes(0), with_lse=True)),
            "tree16k": ("tree_16k_k3_d4", lambda: attention_leg(dev, prefix_len=16384, routes=wl.tree_routes(0),
                                                                with_lse=False)),
            "batched": ("batched_32req", lambda: batched_leg(dev, pool_gb=args.commit_pool_gb)),
            "cow": ("cow_8req_9routes", lambda: cow_leg(dev)),
            "decode": ("drafter_decode_attn", lambda: decode_leg(dev)),
            "decode8k": ("drafter_decode_attn_8k", lambda: decode_leg(dev, prefix_len=8192)),
            "drafter": ("drafter_fork_8req", lambda: drafter_leg(dev)),
            "drafter_calls": ("drafter_fork_8req_per_request_calls", lambda: drafter_leg(dev, batched=False)),
            "frontier": ("drafter_frontier_depth", lambda: frontier_leg(dev)),
        }
        chosen = list(legs) if args.legs == "all" else [x for x in args.legs.split(",") if x]
        for name in chosen:
            if name not in legs:
                raise SystemExit(f"unknown leg {name!r}; legs: {', '.join(legs)}")
            key, run = legs[name]
            result["components"][key] = run()
            print(f"leg {name} done", file=sys.stderr, flush=True)
        if "batched_32req" in result["components"]:
            result["kv_commit_GBps"] = round(result["components"]["batched_32req"]["commit_GBps"], 1)
        if "cow_8req_9routes" in result["components"]:
            result["kv_cow_GBps"] = round(result["components"]["cow_8req_9routes"]["GBps"], 1)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(step, args.cpu_baseline_seconds)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
