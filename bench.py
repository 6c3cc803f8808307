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


def _pkg(name):
    return importlib.import_module(f"0709_amd.{name}")


def _ev():
    return torch.cuda.Event(enable_timing=True)


class HeadlineStep:
    def __init__(self, dev, *, prefix_len=16384, page_size=16, seed=0, split_target=None, max_rows=None):
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
        self.routes = wl.forest_routes(seed)
        spec, _ = ffv.build_deduplicated_tree_spec_from_paths(paths=self.routes, prefix_len=prefix_len,
                                                              page_size=page_size, device=dev)
        self.n = spec.node_count
        self.kv_len = prefix_len + self.n
        self.pages = math.ceil(self.kv_len / page_size)
        self.kv = wl.make_paged_target_kv(self.geom, kv_len=self.kv_len, page_size=page_size, dtype=torch.float16,
                                          device=dev, seed=seed, spare_pages=64)
        self.layers = self.kv.layers
        self.q = wl.random_queries(self.geom, self.n, dtype=torch.float16, device=dev, seed=seed + 7)
        g = torch.Generator(device=dev).manual_seed(seed + 11)
        shp = (self.n, self.geom.kv_heads, self.geom.head_dim)
        self.k_new = [(torch.randn(shp, generator=g, device=dev) * 0.1).half() for _ in range(self.geom.layers)]
        self.v_new = [(torch.randn(shp, generator=g, device=dev) * 0.1).half() for _ in range(self.geom.layers)]
        self.verify_logits = (torch.randn((self.n, 128256), generator=g, device=dev) * 2.0).half()
        self.prefix_logits = (torch.randn((128256,), generator=g, device=dev) * 2.0).half()
        ws = torch.empty(256 * 1024 * 1024, dtype=torch.uint8, device=dev)
        self.wrapper = ffv.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
        if split_target is not None:
            self.wrapper.split_target_items = split_target
        if max_rows is not None:
            self.wrapper.max_rows_per_item = max_rows
        self.kv_indices_host = self.kv.kv_indices.cpu().tolist()
        # physical slots of the tree node positions (page table lookup on host, once)
        pos = torch.arange(prefix_len, self.kv_len)
        idx = torch.tensor(self.kv_indices_host, dtype=torch.int64)
        self.tree_slots = (idx[pos // page_size] * page_size + pos % page_size).to(dev)
        self.kv_indptr = torch.tensor([0, self.pages], dtype=torch.int32, device=dev)
        self.last = torch.tensor([self.kv_len - (self.pages - 1) * page_size], dtype=torch.int32, device=dev)
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

    def forward(self, with_append=True):
        """The per-layer device work of the verify forward: append the tree
        nodes' K/V, then masked attention (append before attention)."""
        for l in range(self.geom.layers):
            layer = self.layers[l]
            if with_append:
                self.kv_ops.append_paged([layer], [self.k_new[l]], [self.v_new[l]], dst_slots=self.tree_slots)
            self.wrapper.run(self.q[l], layer, out=self.outs[l])

    def capture(self):
        """HIP graphs of the 32-layer forward (append + attention) and of the
        attention launches alone.  plan() writes into the wrapper's persistent
        buffers, so replays use the plan of the current step."""
        self.outs = [torch.empty_like(q) for q in self.q]
        self.plan()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.forward()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
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
        # pages of the whole request (prefix + tree) are owned at verify time
        rc = lib.load().atlas_mark_pages(lib.ptr(self.owned), self.pool_pages, lib.ptr(self.all_slots),
                                         self.kv_len, self.ps, stream)
        lib.check(rc, "atlas_mark_pages")
        route_nodes = self.plan()
        self._timed(self.fwd_events, self.graph_fwd.replay)
        # scoring + best route
        backend = object.__new__(self.tr.DirectFlashInferMaskedTreeVerifyBackend)
        backend.score_weights = None
        backend.route_selection_policy = "target_best"
        backend.match_logits_dtype_rounding = True
        payloads = [self.tr.VerifyRoutePayload(route_id=i, token_ids=r, draft_logprob=0.0)
                    for i, r in enumerate(self.routes)]
        scores = backend._score_routes(routes=payloads, paths=self.routes, prefix_logits=self.prefix_logits,
                                       verify_logits=self.verify_logits, route_to_node_paths=route_nodes)
        best = backend._select_route(scores)
        nodes = route_nodes[int(best.route_id)]
        src = [self.prefix_len + x for x in nodes]
        dst = list(range(self.prefix_len, self.prefix_len + len(nodes)))
        self._timed(self.commit_events, lambda: self.kv_ops.commit_paged(
            self.layers, src, dst, kv_indptr=self.kv_indptr, kv_indices=self.kv.kv_indices))
        live = self.all_slots[: self.prefix_len + len(nodes)]
        sampled = torch.cat((live[:: self.ps], live[-1:]))

        def prune():
            rc = lib.load().atlas_prune_pages(lib.ptr(self.owned), lib.ptr(self.live), self.pool_pages,
                                              lib.ptr(sampled), int(sampled.numel()), self.ps,
                                              lib.ptr(self.free_pages), lib.ptr(self.free_count), stream)
            lib.check(rc, "atlas_prune_pages")

        self._timed(self.prune_events, prune)
        freed = int(self.free_count.item())
        return int(best.route_id), len(nodes), freed

    def attention_only(self, replays):
        torch.cuda.synchronize()
        a, b = _ev(), _ev()
        a.record()
        for _ in range(replays):
            self.graph_attn.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / (replays * self.geom.layers)


def _mean_ms(pairs):
    return statistics.fmean(a.elapsed_time(b) for a, b in pairs) if pairs else float("nan")


def commit_leg(dev, *, pool_gb=200.0, requests=32, iters=50):
    """Batched 32-request commit, 8B geometry, bf16, pages scattered over a
    pool of about ``pool_gb`` GB (32 layers x pages x 64 KiB)."""
    kv_ops = _pkg("kv_ops")
    wl = _pkg("workloads")
    geom = wl.LLAMA_8B
    ps = 16
    page_bytes = 2 * ps * geom.kv_heads * geom.head_dim * 2
    gen = torch.Generator().manual_seed(4)
    prefixes = [int(x) for x in torch.randint(1024, 16385, (requests,), generator=gen)]
    need_pages = sum(math.ceil((p + 12) / ps) for p in prefixes)
    pool = None
    while pool is None:
        pool_pages = max(need_pages + 64, int(pool_gb * 1e9 / (geom.layers * page_bytes)))
        try:
            pool = torch.empty((geom.layers, pool_pages, 2, ps, geom.kv_heads, geom.head_dim), dtype=torch.bfloat16,
                               device=dev)
        except torch.cuda.OutOfMemoryError:
            pool_gb /= 2
            if pool_gb < 1:
                raise
    perm = torch.randperm(pool_pages, generator=gen)[:need_pages].to(torch.int32)
    indptr, req, src, dst = [0], [], [], []
    for b, p in enumerate(prefixes):
        indptr.append(indptr[-1] + math.ceil((p + 12) / ps))
        nodes = sorted(int(x) for x in torch.randperm(12, generator=gen)[:4])
        nodes = [0, 1, 2, 3] if b % 3 == 0 else nodes
        for i, nd in enumerate(nodes):
            req.append(b)
            src.append(p + nd)
            dst.append(p + i)
    layers = list(pool.unbind(0))
    args = dict(kv_indptr=torch.tensor(indptr, dtype=torch.int32, device=dev), kv_indices=perm.to(dev),
                item_req=torch.tensor(req, dtype=torch.int32, device=dev))
    src_t = torch.tensor(src, device=dev)
    dst_t = torch.tensor(dst, device=dev)
    staging = kv_ops.commit_positions_need_staging(src, dst, req)
    for _ in range(5):
        kv_ops.commit_paged(layers, src_t, dst_t, needs_staging=staging, **args)
    torch.cuda.synchronize()
    a, b = _ev(), _ev()
    a.record()
    for _ in range(iters):
        kv_ops.commit_paged(layers, src_t, dst_t, needs_staging=staging, **args)
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1000.0 / iters
    moved = len(src) * geom.layers * geom.token_bytes()
    out = {"us": us, "moved_bytes": moved, "GBps": 2 * moved / (us * 1e-6) / 1e9,
           "pool_GB": round(pool.numel() * 2 / 1e9, 1), "requests": requests, "tokens": len(src)}
    del pool, layers
    torch.cuda.empty_cache()
    return out


def cow_leg(dev, *, requests=8, routes=9, iters=50):
    """Drafter tail-page copy-on-write: per request, 9 forked routes share a
    partially filled 64-token tail page; 8 of them get private copies, all in
    one move launch (Llama-3.2-1B KV geometry, bf16, flat token pool)."""
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
    src, dst = [], []
    j = 0
    for b in range(requests):
        tail_page = int(perm[j])
        j += 1
        tail_len = int(torch.randint(1, ps, (1,), generator=gen))
        for _ in range(routes - 1):
            new_page = int(perm[j])
            j += 1
            src.extend(tail_page * ps + o for o in range(tail_len))
            dst.extend(new_page * ps + o for o in range(tail_len))
    src_t = torch.tensor(src, device=dev)
    dst_t = torch.tensor(dst, device=dev)
    for _ in range(5):
        kv_ops.move_slots(k_layers, v_layers, dst_t, src_t)
    torch.cuda.synchronize()
    a, b = _ev(), _ev()
    a.record()
    for _ in range(iters):
        kv_ops.move_slots(k_layers, v_layers, dst_t, src_t)
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1000.0 / iters
    moved = len(src) * geom.layers * geom.token_bytes()
    return {"us": us, "moved_bytes": moved, "GBps": 2 * moved / (us * 1e-6) / 1e9, "slots": len(src)}


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
        layer = step.layers[l].cpu().numpy()
        q = step.q[l].cpu().numpy()
        t0 = time.perf_counter()
        oatt.masked_attention(q, layer, [0, step.n], [0, step.pages], idx, [last], masks=[mask], dtype=np.float32)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s:
            break
    us = statistics.fmean(times) * 1e6
    return {"value": us, "unit": "µs/layer", "cores": cores, "kind": "port",
            "sample": f"oracle float32 masked attention, {len(times)} of 32 layers of the headline step "
                      f"(kv_len {step.kv_len}, {step.n} nodes)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-baseline-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-legs", action="store_true")
    ap.add_argument("--split-target", type=int, default=None)
    ap.add_argument("--max-rows", type=int, default=None)
    ap.add_argument("--commit-pool-gb", type=float, default=200.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU; the path is data-parallel across requests "
                                   "and has no multi-GPU leg", "n_gpus": args.gpus}))
        sys.exit(2)
    dev = torch.device("cuda:0")
    step = HeadlineStep(dev, split_target=args.split_target, max_rows=args.max_rows)
    step.capture()
    for _ in range(args.warmup):
        step.step()
    torch.cuda.synchronize()
    step.record = True
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        route, committed, freed = step.step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1000.0 / args.steps
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
            "prefix_len": step.prefix_len, "page_size": step.ps, "routes": len(step.routes), "depth": 4,
            "nodes": step.n, "kv_len": step.kv_len, "work_items": plan.num_work, "merge_items": plan.num_merge,
            "tiles_per_split": plan.tiles_per_split,
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
            "kernel": "tree_attn_d128_kernel + tree_attn_merge_kernel (one verify attention launch pair)",
            "algorithmic_bytes_per_launch": bytes_layer,
        },
        "components": {
            "attention_us_per_layer": round(attn_us, 3),
            "forward_append_plus_attention_us_per_layer": round(_mean_ms(step.fwd_events) * 1000.0 / 32, 3),
            "commit_us": round(_mean_ms(step.commit_events) * 1000.0, 3),
            "prune_us": round(_mean_ms(step.prune_events) * 1000.0, 3),
            "selected_route": route, "committed_tokens": committed, "pruned_pages": freed,
        },
    }
    if not args.no_legs:
        result["components"]["commit_batched_32req"] = commit_leg(dev, pool_gb=args.commit_pool_gb)
        result["components"]["cow_8req_9routes"] = cow_leg(dev)
        result["kv_commit_GBps"] = round(result["components"]["commit_batched_32req"]["GBps"], 1)
        result["kv_cow_GBps"] = round(result["components"]["cow_8req_9routes"]["GBps"], 1)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(step, args.cpu_baseline_seconds)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
