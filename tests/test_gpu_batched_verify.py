"""Configuration 4 at its real shape: batched Target verify of 32 requests,
Llama-3.1-8B KV geometry (32 layers, 32 q heads, 8 KV heads, head_dim 128),
bf16, page 16, prefixes uniform in [1024, 16384], every request's pages
scattered by a random permutation over a pool larger than the requests, a
k=3 d=4 ancestor mask per request, all in one plan.

* attention: O and LSE of every request against the oracle's float64 closed
  form, within 2e-3 absolute (the reference's FlashInfer call,
  src/atlas_0709/flashinfer_full_verify.py:953-985 and :1223);
* commit: the 128-item batched commit (4 tokens per request, item_req,
  device positions, one in-place pass) copies every committed row of all 32
  layers bit for bit and leaves other rows untouched
  (src/atlas_0709/target_runtime.py:873-920);
* prune: mark and sweep over a pool of more than 95,367 pages (the page count
  of a 200 GB pool at this geometry) against the oracle's
  sorted(owned - live) (src/atlas_0709/flashinfer_paged/sglang_runtime.py:507-539).
"""

import numpy as np
import pytest
import torch

from helpers import pkg
from oracle import attention as oatt
from oracle import paged_kv as ref

pytestmark = pytest.mark.gpu

LAYERS = 32
PS = 16
# KV pool: about 1.5x the requests' pages (the scatter is what matters);
# the prune's page space is the 200 GB pool's.
KV_POOL_PAGES = 26624
PRUNE_POOL_PAGES = 95367 + 633


@pytest.fixture(scope="module")
def case(dev):
    wl = pkg("workloads")
    geom = wl.LLAMA_8B
    c = wl.batched_verify_case(pool_pages=KV_POOL_PAGES, page_size=PS)
    print(f"config 4: {len(c.prefixes)} requests, {c.need_pages} pages over a {KV_POOL_PAGES}-page pool, "
          f"mean prefix {sum(c.prefixes) / len(c.prefixes):.1f}", flush=True)
    layers = [torch.zeros((KV_POOL_PAGES, 2, PS, geom.kv_heads, geom.head_dim), dtype=torch.bfloat16, device=dev)
              for _ in range(LAYERS)]
    used = c.page_ids.to(dev)
    g = torch.Generator(device=dev).manual_seed(5)
    for layer in layers:
        layer[used] = (torch.randn((c.need_pages, 2, PS, geom.kv_heads, geom.head_dim), generator=g, device=dev)
                       * 0.1).to(torch.bfloat16)
    torch.cuda.synchronize()
    yield c, geom, layers
    del layers
    torch.cuda.empty_cache()


def _specs(c, dev):
    ffv = pkg("flashinfer_full_verify")
    return [ffv.build_deduplicated_tree_spec_from_paths(paths=r, prefix_len=p, page_size=PS, device=dev)
            for r, p in zip(c.routes, c.prefixes)]


def test_config4_attention_every_request_matches_oracle(dev, case):
    c, geom, layers = case
    ffv = pkg("flashinfer_full_verify")
    specs = _specs(c, dev)
    qo = torch.tensor(c.qo_indptr, dtype=torch.int32, device=dev)
    kv_indptr = torch.tensor(c.kv_indptr, dtype=torch.int32, device=dev)
    kv_indices = c.page_ids.to(torch.int32).to(dev)
    last = torch.tensor([k - (n - 1) * PS for k, n in zip(c.kv_lens, c.req_pages)], dtype=torch.int32, device=dev)
    flat_mask = torch.cat([sp.bool_mask for sp, _ in specs])
    ws = torch.empty(512 * 1024 * 1024, dtype=torch.uint8, device=dev)
    w = ffv.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(qo, kv_indptr, kv_indices, last, geom.q_heads, geom.kv_heads, geom.head_dim, PS, custom_mask=flat_mask,
           causal=False, q_data_type=torch.bfloat16)
    plan = w.current_plan
    assert plan.num_merge > 0 and plan.num_work > 256, "the batched plan splits keys over the device"
    g = torch.Generator(device=dev).manual_seed(6)
    nnz = c.qo_indptr[-1]
    for layer_idx in (0, LAYERS - 1):
        q = (torch.randn((nnz, geom.q_heads, geom.head_dim), generator=g, device=dev) * 0.1).to(torch.bfloat16)
        print(f"config 4 attention, layer {layer_idx}: {plan.num_work} items, {plan.num_merge} merges", flush=True)
        out, lse = w.run(q, layers[layer_idx], return_lse=True)
        torch.cuda.synchronize()
        q_h = q.float().cpu().numpy()
        out_h = out.float().cpu().numpy()
        lse_h = lse.cpu().numpy()
        worst = (0.0, 0.0)
        for b in range(len(c.prefixes)):
            pages = c.page_ids[c.kv_indptr[b]: c.kv_indptr[b + 1]].to(dev)
            kv_b = layers[layer_idx].index_select(0, pages).float().cpu().numpy()
            _, parents, _, _ = ref.dedup_tree(c.routes[b])
            mask = ref.ancestor_mask(parents, c.prefixes[b])
            q0, q1 = c.qo_indptr[b], c.qo_indptr[b + 1]
            ro, rl = oatt.masked_attention(q_h[q0:q1], kv_b, [0, q1 - q0], [0, c.req_pages[b]],
                                           list(range(c.req_pages[b])), [c.kv_lens[b] - (c.req_pages[b] - 1) * PS],
                                           masks=[mask])
            err = float(np.abs(out_h[q0:q1] - ro).max())
            lerr = float(np.abs(lse_h[q0:q1] - rl).max())
            worst = (max(worst[0], err), max(worst[1], lerr))
            assert err <= 2e-3 and lerr <= 2e-3, f"layer {layer_idx} request {b}: |dO|={err:.3g} |dlse|={lerr:.3g}"
        print(f"config 4 attention, layer {layer_idx}: worst |dO|={worst[0]:.3g} |dlse|={worst[1]:.3g}", flush=True)


def _slot(c, b, pos):
    page = int(c.page_ids[c.kv_indptr[b] + pos // PS])
    return page, pos % PS


def _rows(layers, slots, dev):
    pages = torch.tensor([p for p, _ in slots], dtype=torch.long, device=dev)
    offs = torch.tensor([o for _, o in slots], dtype=torch.long, device=dev)
    # [L, n, 2, Hkv, D] as int16 bits
    return torch.stack([layer[pages, :, offs] for layer in layers]).view(torch.int16).cpu()


def test_config4_batched_commit_bit_exact(dev, case):
    c, geom, layers = case
    kv_ops = pkg("kv_ops")
    specs = _specs(c, dev)
    item_req, src, dst = [], [], []
    for b, ((_, route_nodes), p) in enumerate(zip(specs, c.prefixes)):
        for i, nd in enumerate(route_nodes[c.selected[b]]):
            item_req.append(b)
            src.append(p + nd)
            dst.append(p + i)
    assert len(src) == 128
    assert not kv_ops.commit_positions_need_staging(src, dst, item_req)
    src_slots = [_slot(c, b, s) for b, s in zip(item_req, src)]
    dst_slots = [_slot(c, b, d) for b, d in zip(item_req, dst)]
    # untouched rows: the 16 prefix rows before every commit and the tree
    # rows that no item writes
    gen = np.random.default_rng(11)
    keep = []
    for b, p in enumerate(c.prefixes):
        for pos in sorted(set(gen.integers(0, p, 48).tolist()) | set(range(p - 16, p))):
            keep.append(_slot(c, b, pos))
        for pos in range(p + 4, c.kv_lens[b]):
            keep.append(_slot(c, b, pos))
    expect = _rows(layers, src_slots, dev)
    before_keep = _rows(layers, keep, dev)
    args = dict(kv_indptr=torch.tensor(c.kv_indptr, dtype=torch.int32, device=dev),
                kv_indices=c.page_ids.to(torch.int32).to(dev),
                item_req=torch.tensor(item_req, dtype=torch.int32, device=dev))
    print(f"config 4 commit: {len(src)} items x {LAYERS} layers, device positions, in place", flush=True)
    kv_ops.commit_paged(layers, torch.tensor(src, device=dev), torch.tensor(dst, device=dev), needs_staging=False,
                        **args)
    torch.cuda.synchronize()
    got = _rows(layers, dst_slots, dev)
    bad = (got != expect).reshape(LAYERS, len(src), -1).any(-1)
    assert not bool(bad.any()), f"committed rows differ at (layer, item) {bad.nonzero()[:8].tolist()}"
    after_keep = _rows(layers, keep, dev)
    assert torch.equal(after_keep, before_keep), "rows outside the commit destinations changed"


def test_config4_mark_and_prune_large_pool(dev, case):
    c, _, _ = case
    lib = pkg("_lib")
    L = lib.load()
    pool_pages = PRUNE_POOL_PAGES
    words = (pool_pages + 31) // 32
    owned = torch.zeros(words, dtype=torch.int32, device=dev)
    live_bm = torch.zeros_like(owned)
    free_pages = torch.zeros(pool_pages, dtype=torch.int64, device=dev)
    free_count = torch.zeros(1, dtype=torch.int64, device=dev)
    # owned: every request's pages, plus pages held elsewhere in the large
    # pool (other requests' trees) that no live path reaches
    gen = torch.Generator().manual_seed(12)
    extra = (torch.randperm(pool_pages - KV_POOL_PAGES, generator=gen)[:20000] + KV_POOL_PAGES)
    owned_pages = torch.cat((c.page_ids, extra))
    live_paths = []
    for b, p in enumerate(c.prefixes):
        keep = p + len(c.routes[b][c.selected[b]])
        pos = torch.arange(keep)
        live_paths.append((c.page_ids[c.kv_indptr[b] + pos // PS] * PS + pos % PS).tolist())
    sampled = []
    for path in live_paths:
        sampled.extend(path[::PS] + path[-1:])
    owned_slots = (owned_pages * PS).to(dev)
    live_slots = torch.tensor(sampled, dtype=torch.int64, device=dev)
    print(f"config 4 prune: {pool_pages} pages, {int(owned_pages.numel())} owned, {len(sampled)} sampled slots",
          flush=True)
    stream = lib.stream_of(dev)
    rc = L.atlas_mark_pages(lib.ptr(owned), pool_pages, lib.ptr(owned_slots), int(owned_slots.numel()), PS, stream)
    lib.check(rc, "atlas_mark_pages")
    rc = L.atlas_prune_pages(lib.ptr(owned), lib.ptr(live_bm), pool_pages, lib.ptr(live_slots),
                             int(live_slots.numel()), PS, lib.ptr(free_pages), lib.ptr(free_count), stream)
    lib.check(rc, "atlas_prune_pages")
    torch.cuda.synchronize()
    released, remaining = ref.prune({int(x) for x in owned_pages.tolist()}, None, live_paths, PS)
    n = int(free_count.item())
    assert n == len(released)
    assert free_pages[:n].cpu().tolist() == released
    bits = owned.cpu().numpy().view(np.uint32)
    still = {w * 32 + i for w in np.nonzero(bits)[0] for i in range(32) if (int(bits[w]) >> i) & 1}
    assert still == remaining
