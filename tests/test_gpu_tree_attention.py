"""Ancestor-masked paged tree attention vs the oracle's closed form.

Tolerance: 2e-3 absolute on O and LSE (fp16 / bf16), the bound the path is
specified with.  V is always drawn as N(0,1) * 0.1 (the configs' scale), which
keeps |O| below ~0.5 where one bf16 output rounding stays under 2e-3; Q and K
vary in scale.  Cases are built so that a wrong mask bit, page or split merge
moves the output by far more than the tolerance: short prefixes (the tree keys
carry a large share of the softmax mass), and long prefixes whose keys are
pushed far below the tree keys ("dominant tree"), so every query's output is
the softmax over exactly its visible ancestors.
"""

import math

import numpy as np
import pytest
import torch

from helpers import pkg
from oracle import attention as oatt
from oracle import paged_kv as ref

pytestmark = pytest.mark.gpu

ATOL = 2e-3


def _routes(gen, k, depth, share):
    routes = []
    for r in range(k):
        if routes and share:
            keep = int(torch.randint(0, depth, (1,), generator=gen))
            base = list(routes[-1][:keep])
        else:
            base = []
        while len(base) < depth:
            base.append(int(torch.randint(0, 128256, (1,), generator=gen)))
        routes.append(tuple(base))
    return routes


def _build(dev, *, seed, prefix_len, routes, hq=32, hkv=8, d=128, ps=16, dtype=torch.float16, spare_pages=7,
           scale=1.0, dominant_tree=False, permute=True):
    ffv = pkg("flashinfer_full_verify")
    gen = torch.Generator().manual_seed(seed)
    spec, route_nodes = ffv.build_deduplicated_tree_spec_from_paths(
        paths=routes, prefix_len=prefix_len, page_size=ps, device=dev
    )
    n = spec.node_count
    kv_len = prefix_len + n
    pages = math.ceil(kv_len / ps)
    pool = pages + spare_pages
    order = torch.randperm(pool, generator=gen)[:pages] if permute else torch.arange(pages)
    kv = torch.randn((pool, 2, ps, hkv, d), generator=gen) * scale
    kv[:, 1] = torch.randn((pool, ps, hkv, d), generator=gen) * 0.1
    q = torch.randn((n, hq, d), generator=gen) * scale
    if dominant_tree:
        # All queries near u; prefix keys near -u, tree keys near +u.  With
        # |u| = 12 a prefix key scores ~25 (natural log) below a tree key, so
        # 16k prefix keys hold < 1e-6 of the softmax mass.
        u = torch.randn(d, generator=gen)
        u = u / u.norm() * 12.0
        q = u + 0.3 * torch.randn((n, hq, d), generator=gen)
        flat_k = kv[order, 0].reshape(pages * ps, hkv, d)
        flat_k[:prefix_len] = -u + 0.3 * torch.randn((prefix_len, hkv, d), generator=gen)
        flat_k[prefix_len:kv_len] = u + 0.3 * torch.randn((n, hkv, d), generator=gen)
        kv[order, 0] = flat_k.reshape(pages, ps, hkv, d)
    kv = kv.to(dtype)
    q = q.to(dtype)
    _, parents, _, _ = ref.dedup_tree(routes)
    mask = ref.ancestor_mask(parents, prefix_len)
    return dict(spec=spec, q=q, kv=kv, order=order.to(torch.int32), pages=pages, kv_len=kv_len, n=n, mask=mask,
                hq=hq, hkv=hkv, d=d, ps=ps, dtype=dtype, route_nodes=route_nodes)


def _hnd(kv):
    """NHD pages [pool, 2, ps, Hkv, D] as HND pages [pool, 2, Hkv, ps, D]."""
    return kv.permute(0, 1, 3, 2, 4).contiguous()


def _run_and_check(dev, c, *, split_target=None, use_packed=False, atol=ATOL, max_rows=None, layout="NHD"):
    ta = pkg("tree_attention")
    ffv = pkg("flashinfer_full_verify")
    ws = torch.empty(128 * 1024 * 1024, dtype=torch.uint8, device=dev)
    w = ta.BatchPrefillWithPagedKVCacheWrapper(ws, layout)
    if split_target is not None:
        w.split_target_items = split_target
    if max_rows is not None:
        w.max_rows_per_item = max_rows
    last = ffv.last_page_len(c["kv_len"], c["ps"])
    mask_kw = (
        {"packed_custom_mask": ffv.packbits(c["spec"].bool_mask, bitorder="little")}
        if use_packed else {"custom_mask": c["spec"].bool_mask}
    )
    w.plan(
        torch.tensor([0, c["n"]], dtype=torch.int32, device=dev),
        torch.tensor([0, c["pages"]], dtype=torch.int32, device=dev),
        c["order"].to(dev),
        torch.tensor([last], dtype=torch.int32, device=dev),
        c["hq"], c["hkv"], c["d"], c["ps"], causal=False, pos_encoding_mode="NONE",
        q_data_type=c["dtype"], kv_data_type=c["dtype"], **mask_kw,
    )
    kv = c["kv"] if layout == "NHD" else _hnd(c["kv"])
    out, lse = w.run(c["q"].to(dev), kv.to(dev), return_lse=True)
    torch.cuda.synchronize()
    ro, rl = oatt.masked_attention(
        c["q"].float().numpy().astype(np.float64), c["kv"].float().numpy().astype(np.float64),
        [0, c["n"]], [0, c["pages"]], c["order"].tolist(), [last], masks=[c["mask"]],
    )
    o = out.float().cpu().numpy()
    l = lse.cpu().numpy()
    err_o = float(np.abs(o - ro).max())
    err_l = float(np.abs(l - rl).max())
    assert err_o <= atol, f"max |O - ref| = {err_o}"
    assert err_l <= atol, f"max |lse - ref| = {err_l}"
    c.setdefault("outs", {})[(layout, split_target)] = (out.cpu(), lse.cpu())
    return w, o, ro


@pytest.mark.parametrize("prefix_len", [0, 1, 5, 16, 61, 64, 100, 257])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_tree_short_prefix(dev, prefix_len, dtype):
    gen = torch.Generator().manual_seed(prefix_len)
    routes = _routes(gen, 3, 4, share=True)
    c = _build(dev, seed=10 + prefix_len, prefix_len=prefix_len, routes=routes, dtype=dtype)
    _run_and_check(dev, c)
    c = _build(dev, seed=20 + prefix_len, prefix_len=prefix_len, routes=routes, dtype=dtype, dominant_tree=True)
    _run_and_check(dev, c)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_config2_geometry_4096_prefix_no_shared_prefix(dev, dtype):
    """8B attention geometry, prefix 4096 in permuted pages, k=3 d=4 (12 nodes)."""
    gen = torch.Generator().manual_seed(0)
    routes = _routes(gen, 3, 4, share=False)
    c = _build(dev, seed=0, prefix_len=4096, routes=routes, dtype=dtype, scale=0.1, spare_pages=300)
    assert c["n"] == 12
    _run_and_check(dev, c)
    c = _build(dev, seed=1, prefix_len=4096, routes=routes, dtype=dtype, dominant_tree=True, spare_pages=300)
    _run_and_check(dev, c)


@pytest.mark.parametrize("split_target", [1, 64, 512, 4096])
def test_forest_16k_prefix_dominant_tree_all_split_levels(dev, split_target):
    """Forest of 9 routes (shared prefixes, <= 36 nodes) over a 16k prefix; the
    tree keys dominate so mask, paging and split-merge errors are visible."""
    gen = torch.Generator().manual_seed(3)
    routes = _routes(gen, 9, 4, share=True)
    c = _build(dev, seed=3, prefix_len=16384, routes=routes, dominant_tree=True, spare_pages=50)
    assert c["n"] <= 36
    w, o, ro = _run_and_check(dev, c, split_target=split_target)
    plan = w.current_plan
    if split_target == 1:
        assert plan.num_merge == 0
    if split_target >= 512:
        assert plan.num_merge > 0


@pytest.mark.parametrize("max_rows", [16, 48, 64, 100, 192])
def test_row_blocking_variants(dev, max_rows):
    """Rows of a KV head split over several work items (each re-reading the
    keys) give the same result as one block."""
    gen = torch.Generator().manual_seed(21)
    routes = _routes(gen, 9, 4, share=True)
    c = _build(dev, seed=21, prefix_len=2000, routes=routes, dominant_tree=True)
    w, _, _ = _run_and_check(dev, c, max_rows=max_rows)
    assert w.current_plan.max_rows <= max(16, max_rows)


@pytest.mark.parametrize("n_routes,max_rows", [(2, 32), (6, 96), (9, 144), (10, 160), (11, 176), (16, 256)])
@pytest.mark.parametrize("split_target", [None, 1])
def test_row_tile_counts_cover_every_wave_layout(dev, n_routes, max_rows, split_target):
    """One row block of T = 2, 6, 9, 10, 11, 16 tiles (n_routes disjoint routes
    of depth 4, four query heads per KV head): leftover tiles split by keys into
    halves (2, 6, 10) or quarters (9), two tiles per wave (11, 16); with the
    keys split over work items (partial states merged) and without."""
    gen = torch.Generator().manual_seed(40 + n_routes)
    routes = [tuple(int(x) for x in torch.randint(0, 128256, (4,), generator=gen)) for _ in range(n_routes)]
    c = _build(dev, seed=40 + n_routes, prefix_len=2000, routes=routes, dominant_tree=split_target is None)
    assert c["n"] * 4 == max_rows
    w, _, _ = _run_and_check(dev, c, max_rows=max_rows, split_target=split_target)
    assert w.current_plan.max_rows == max_rows
    assert (w.current_plan.num_merge > 0) == (split_target is None)


def test_forest_16k_unit_scale(dev):
    gen = torch.Generator().manual_seed(4)
    routes = _routes(gen, 9, 4, share=True)
    c = _build(dev, seed=4, prefix_len=16384, routes=routes, spare_pages=11)
    _run_and_check(dev, c)


def test_packed_mask_little_bit_order(dev):
    gen = torch.Generator().manual_seed(5)
    routes = _routes(gen, 3, 4, share=True)
    c = _build(dev, seed=5, prefix_len=77, routes=routes)
    _run_and_check(dev, c, use_packed=True)


def test_identical_routes_and_single_node(dev):
    c = _build(dev, seed=6, prefix_len=33, routes=[(7, 8), (7, 8)])
    assert c["n"] == 2
    _run_and_check(dev, c)
    c = _build(dev, seed=7, prefix_len=500, routes=[(9,)], dominant_tree=True)
    _run_and_check(dev, c)


@pytest.mark.parametrize("hq,hkv,d,ps", [(32, 8, 64, 16), (32, 8, 128, 64), (8, 8, 128, 16), (16, 2, 64, 32)])
def test_geometry_variants(dev, hq, hkv, d, ps):
    gen = torch.Generator().manual_seed(hq + d + ps)
    routes = _routes(gen, 3, 4, share=True)
    c = _build(dev, seed=8, prefix_len=300, routes=routes, hq=hq, hkv=hkv, d=d, ps=ps)
    _run_and_check(dev, c)
    c = _build(dev, seed=9, prefix_len=3000, routes=routes, hq=hq, hkv=hkv, d=d, ps=ps, dominant_tree=True)
    _run_and_check(dev, c)


def test_batched_ragged_requests_mixed_masks(dev):
    """Several requests (ragged prefixes, scattered pages) in one plan: tree
    masks per request, compared against the oracle request by request."""
    ta = pkg("tree_attention")
    ffv = pkg("flashinfer_full_verify")
    gen = torch.Generator().manual_seed(11)
    hq, hkv, d, ps = 32, 8, 128, 16
    prefixes = [1024, 37, 5000, 16, 2048]
    specs, qs, masks = [], [], []
    pages_per, lasts, kv_lens = [], [], []
    for i, p in enumerate(prefixes):
        routes = _routes(gen, 3, 4, share=bool(i % 2))
        spec, _ = ffv.build_deduplicated_tree_spec_from_paths(paths=routes, prefix_len=p, page_size=ps, device=dev)
        _, parents, _, _ = ref.dedup_tree(routes)
        specs.append(spec)
        masks.append(ref.ancestor_mask(parents, p))
        qs.append(torch.randn((spec.node_count, hq, d), generator=gen))
        kv_lens.append(p + spec.node_count)
        pages_per.append(math.ceil(kv_lens[-1] / ps))
        lasts.append(ffv.last_page_len(kv_lens[-1], ps))
    total_pages = sum(pages_per)
    pool = total_pages + 40
    perm = torch.randperm(pool, generator=gen)[:total_pages].to(torch.int32)
    kv = torch.randn((pool, 2, ps, hkv, d), generator=gen)
    kv[:, 1] *= 0.1
    kv = kv.to(torch.float16)
    q = torch.cat(qs).to(torch.float16)
    qo = [0]
    for s in specs:
        qo.append(qo[-1] + s.node_count)
    kvp = [0]
    for p in pages_per:
        kvp.append(kvp[-1] + p)
    flat_mask = torch.cat([torch.from_numpy(m.reshape(-1)) for m in masks]).to(dev)
    ws = torch.empty(64 * 1024 * 1024, dtype=torch.uint8, device=dev)
    w = ta.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(torch.tensor(qo, dtype=torch.int32, device=dev), torch.tensor(kvp, dtype=torch.int32, device=dev),
           perm.to(dev), torch.tensor(lasts, dtype=torch.int32, device=dev), hq, hkv, d, ps,
           custom_mask=flat_mask, q_data_type=torch.float16)
    out, lse = w.run(q.to(dev), kv.to(dev), return_lse=True)
    torch.cuda.synchronize()
    ro, rl = oatt.masked_attention(q.float().numpy().astype(np.float64), kv.float().numpy().astype(np.float64),
                                   qo, kvp, perm.tolist(), lasts, masks=masks)
    assert float(np.abs(out.float().cpu().numpy() - ro).max()) <= ATOL
    assert float(np.abs(lse.cpu().numpy() - rl).max()) <= ATOL


def test_causal_and_unmasked_modes(dev):
    ta = pkg("tree_attention")
    gen = torch.Generator().manual_seed(12)
    hq, hkv, d, ps = 16, 4, 128, 16
    qo_len, kv_len = 20, 700
    pages = math.ceil(kv_len / ps)
    kv = torch.randn((pages + 3, 2, ps, hkv, d), generator=gen)
    kv[:, 1] *= 0.1
    kv = kv.to(torch.float16)
    q = torch.randn((qo_len, hq, d), generator=gen).to(torch.float16)
    perm = torch.randperm(pages + 3, generator=gen)[:pages].to(torch.int32)
    last = kv_len - (pages - 1) * ps
    ws = torch.empty(16 * 1024 * 1024, dtype=torch.uint8, device=dev)
    for causal in (False, True):
        w = ta.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
        w.plan(torch.tensor([0, qo_len], dtype=torch.int32), torch.tensor([0, pages], dtype=torch.int32),
               perm.to(dev), torch.tensor([last], dtype=torch.int32), hq, hkv, d, ps, causal=causal)
        out, lse = w.run(q.to(dev), kv.to(dev), return_lse=True)
        torch.cuda.synchronize()
        ro, rl = oatt.masked_attention(q.float().numpy().astype(np.float64), kv.float().numpy().astype(np.float64),
                                       [0, qo_len], [0, pages], perm.tolist(), [last], causal=causal)
        assert float(np.abs(out.float().cpu().numpy() - ro).max()) <= ATOL
        assert float(np.abs(lse.cpu().numpy() - rl).max()) <= ATOL


def test_reference_plan_helper_and_kv_tuple(dev):
    """plan_prefill_wrapper's keyword ladder drives the wrapper; run accepts a
    (K, V) tuple of [pages, page_size, Hkv, D] caches."""
    ffv = pkg("flashinfer_full_verify")
    from types import SimpleNamespace

    gen = torch.Generator().manual_seed(13)
    routes = _routes(gen, 3, 4, share=True)
    c = _build(dev, seed=13, prefix_len=160, routes=routes, permute=False, spare_pages=0)
    args = SimpleNamespace(workspace_mb=8, device=dev, page_size=16, use_packed_custom_mask=False)
    cfg = SimpleNamespace(num_attention_heads=32, num_key_value_heads=8, head_dim=128, hidden_size=4096)
    w = ffv.make_prefill_wrapper(args=args)
    ffv.plan_prefill_wrapper(w, c["spec"], args=args, config=cfg, dtype=torch.float16)
    kvd = c["kv"].to(dev)
    out = ffv.first_tensor(w.run(c["q"].to(dev), kvd))
    out2 = w.run(c["q"].to(dev), (kvd[:, 0], kvd[:, 1]))
    torch.cuda.synchronize()
    ro, _ = oatt.masked_attention(c["q"].float().numpy().astype(np.float64), c["kv"].float().numpy().astype(np.float64),
                                  [0, c["n"]], [0, c["pages"]], list(range(c["pages"])), [ffv.last_page_len(c["kv_len"], 16)],
                                  masks=[c["mask"]])
    assert float(np.abs(out.float().cpu().numpy() - ro).max()) <= ATOL
    assert torch.equal(out, out2)


@pytest.mark.parametrize("split_target", [None, 1, 64])
def test_page_windows_match_page_table_path(dev, split_target):
    """Plan-time page-id windows: each item's window holds the ids of its first
    64 pages (clamped to its last page), the plan's page table and mask words
    equal the caller's, and attention with the windows is bit-equal
    to attention reading the page table after the work item.  Split target 1
    gives one split of ~330 pages per KV head, so the kernel still loads later
    windows from the page table."""
    ta = pkg("tree_attention")
    ffv = pkg("flashinfer_full_verify")
    gen = torch.Generator().manual_seed(31)
    routes = _routes(gen, 9, 4, share=True)
    c = _build(dev, seed=31, prefix_len=5000, routes=routes, spare_pages=20)
    last = ffv.last_page_len(c["kv_len"], c["ps"])
    q, kv = c["q"].to(dev), c["kv"].to(dev)
    results = []
    for use in (True, False):
        ws = torch.empty(64 * 1024 * 1024, dtype=torch.uint8, device=dev)
        w = ta.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
        w.use_page_windows = use
        if split_target is not None:
            w.split_target_items = split_target
        w.plan(
            torch.tensor([0, c["n"]], dtype=torch.int32, device=dev),
            torch.tensor([0, c["pages"]], dtype=torch.int32, device=dev),
            c["order"].to(dev), torch.tensor([last], dtype=torch.int32, device=dev),
            c["hq"], c["hkv"], c["d"], c["ps"], causal=False, custom_mask=c["spec"].bool_mask,
            q_data_type=c["dtype"],
        )
        out, lse = w.run(q, kv, return_lse=True)
        torch.cuda.synchronize()
        results.append((w.current_plan, out.cpu(), lse.cpu()))
    (plan, out_a, lse_a), (plan_b, out_b, lse_b) = results
    assert plan.page_windows is not None and plan_b.page_windows is None
    assert torch.equal(out_a, out_b) and torch.equal(lse_a, lse_b)
    order = c["order"].tolist()
    words = c["spec"].tree_mask.cpu().tolist()
    for p in (plan, plan_b):
        # the one-launch plan install copied the page table and the mask words
        assert p.kv_indices[: len(order)].cpu().tolist() == order
        assert p.tree_mask[: len(words)].cpu().tolist() == words
    win = plan.page_windows.cpu().view(-1, 64)
    meta = plan.meta.cpu()
    ps = c["ps"]
    for i in range(plan.num_work):
        item = meta[16 * i : 16 * i + 16].tolist()
        kv_start, kv_end, kv_len, page_offset = item[4], item[5], item[9], item[11]
        end = min(kv_end, kv_len)
        t0 = min(kv_start, end)
        if t0 < end:
            p0, lp = t0 // ps, (end - 1) // ps
            assert win[i].tolist() == [order[page_offset + min(p0 + l, lp)] for l in range(64)], f"item {i}"


@pytest.mark.parametrize("prefix_len,split_target", [(16384, None), (16384, 1), (300, None), (4000, 4096)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_append_matches_append_then_attention(dev, prefix_len, split_target, dtype):
    """run(append_key_states=, append_value_states=) writes the tree nodes'
    K/V rows at positions prefix_len + i inside the attention launch: the
    cache equals the one a separate append leaves (bit-exact), and the
    output equals the separate append + attention (bit-exact) and the oracle
    (2e-3).  Split target 1 leaves one split per KV head; 4096 splits the
    tree positions over several items."""
    ta = pkg("tree_attention")
    ffv = pkg("flashinfer_full_verify")
    kv_ops = pkg("kv_ops")
    gen = torch.Generator().manual_seed(prefix_len + 3)
    routes = _routes(gen, 9, 4, share=True)
    c = _build(dev, seed=prefix_len + 5, prefix_len=prefix_len, routes=routes, dtype=dtype, spare_pages=9)
    n, ps, hkv, d = c["n"], c["ps"], c["hkv"], c["d"]
    k_new = (torch.randn((n, hkv, d), generator=gen) * 0.5).to(dtype)
    v_new = (torch.randn((n, hkv, d), generator=gen) * 0.1).to(dtype)
    order = c["order"].tolist()
    pos = [prefix_len + i for i in range(n)]
    slots = torch.tensor([order[p // ps] * ps + p % ps for p in pos], dtype=torch.int64, device=dev)
    last = ffv.last_page_len(c["kv_len"], ps)
    results = []
    for fused in (False, True):
        kv = c["kv"].to(dev)
        w = ta.BatchPrefillWithPagedKVCacheWrapper(torch.empty(64 << 20, dtype=torch.uint8, device=dev), "NHD")
        if split_target is not None:
            w.split_target_items = split_target
        w.plan(torch.tensor([0, n], dtype=torch.int32, device=dev),
               torch.tensor([0, c["pages"]], dtype=torch.int32, device=dev), c["order"].to(dev),
               torch.tensor([last], dtype=torch.int32, device=dev), c["hq"], hkv, d, ps,
               custom_mask=c["spec"].bool_mask, q_data_type=dtype)
        assert w.current_plan.fused_append
        if fused:
            out, lse = w.run(c["q"].to(dev), kv, return_lse=True, append_key_states=k_new.to(dev),
                             append_value_states=v_new.to(dev))
        else:
            kv_ops.append_paged([kv], [k_new.to(dev)], [v_new.to(dev)], dst_slots=slots)
            out, lse = w.run(c["q"].to(dev), kv, return_lse=True)
        torch.cuda.synchronize()
        results.append((kv.cpu(), out.cpu(), lse.cpu()))
    (kv_a, out_a, lse_a), (kv_b, out_b, lse_b) = results
    assert torch.equal(kv_a.view(torch.int16), kv_b.view(torch.int16))
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16)) and torch.equal(lse_a, lse_b)
    ro, rl = oatt.masked_attention(c["q"].double().numpy(), kv_b.double().numpy(), [0, n], [0, c["pages"]],
                                   order, [last], masks=[c["mask"]])
    assert float(np.abs(out_b.float().numpy() - ro).max()) <= ATOL
    assert float(np.abs(lse_b.numpy() - rl).max()) <= ATOL


def test_fused_append_batched_requests_and_refusals(dev):
    """Two ragged requests in one plan (causal mode, each appending its own
    newest rows), then the cases the fused append refuses: several row blocks
    per KV head (the rows could be read by another block before they are
    written) and head_dim 64."""
    ta = pkg("tree_attention")
    gen = torch.Generator().manual_seed(77)
    hq, hkv, d, ps = 32, 8, 128, 16
    qo_lens, kv_lens = [5, 11], [700, 2100]
    pages = [math.ceil(k / ps) for k in kv_lens]
    pool = sum(pages) + 5
    perm = torch.randperm(pool, generator=gen).tolist()
    table = [perm[: pages[0]], perm[pages[0]: pages[0] + pages[1]]]
    kv = (torch.randn((pool, 2, ps, hkv, d), generator=gen) * 0.3).half()
    q = (torch.randn((sum(qo_lens), hq, d), generator=gen) * 0.3).half()
    k_new = (torch.randn((sum(qo_lens), hkv, d), generator=gen) * 0.3).half()
    v_new = (torch.randn((sum(qo_lens), hkv, d), generator=gen) * 0.1).half()
    qo = [0, qo_lens[0], sum(qo_lens)]
    kvp = [0, pages[0], sum(pages)]
    last = [k - (p - 1) * ps for k, p in zip(kv_lens, pages)]
    w = ta.BatchPrefillWithPagedKVCacheWrapper(torch.empty(64 << 20, dtype=torch.uint8, device=dev), "NHD")
    w.plan(torch.tensor(qo, dtype=torch.int32), torch.tensor(kvp, dtype=torch.int32),
           torch.tensor(table[0] + table[1], dtype=torch.int32, device=dev), torch.tensor(last, dtype=torch.int32),
           hq, hkv, d, ps, causal=True, q_data_type=torch.float16)
    kv_dev = kv.to(dev)
    out = w.run(q.to(dev), kv_dev, append_key_states=k_new.to(dev), append_value_states=v_new.to(dev))
    torch.cuda.synchronize()
    expect = kv.clone()
    for b in range(2):
        for i in range(qo_lens[b]):
            p = kv_lens[b] - qo_lens[b] + i
            expect[table[b][p // ps], 0, p % ps] = k_new[qo[b] + i]
            expect[table[b][p // ps], 1, p % ps] = v_new[qo[b] + i]
    got = kv_dev.cpu()
    assert torch.equal(got.view(torch.int16), expect.view(torch.int16))
    ro, _ = oatt.masked_attention(q.double().numpy(), expect.double().numpy(), qo, kvp, table[0] + table[1], last,
                                  causal=True)
    assert float(np.abs(out.float().cpu().numpy() - ro).max()) <= ATOL
    # several row blocks per KV head: refused
    w.max_rows_per_item = 16
    w.plan(torch.tensor(qo, dtype=torch.int32), torch.tensor(kvp, dtype=torch.int32),
           torch.tensor(table[0] + table[1], dtype=torch.int32, device=dev), torch.tensor(last, dtype=torch.int32),
           hq, hkv, d, ps, causal=True, q_data_type=torch.float16)
    assert not w.current_plan.fused_append
    with pytest.raises(NotImplementedError):
        w.run(q.to(dev), kv_dev, append_key_states=k_new.to(dev), append_value_states=v_new.to(dev))
    # head_dim 64: refused
    w64 = ta.BatchPrefillWithPagedKVCacheWrapper(torch.empty(8 << 20, dtype=torch.uint8, device=dev), "NHD")
    w64.plan(torch.tensor([0, 2], dtype=torch.int32), torch.tensor([0, 1], dtype=torch.int32),
             torch.tensor([0], dtype=torch.int32, device=dev), torch.tensor([5], dtype=torch.int32),
             8, 8, 64, 16, causal=True, q_data_type=torch.float16)
    assert not w64.current_plan.fused_append


def _rope_tables(positions: torch.Tensor, d: int, dtype: torch.dtype, theta: float = 500000.0):
    """cos / sin rows as the reference builds them without a rotary module
    (flashinfer_full_verify.py:242-256): fp32 angles, rounded to the dtype."""
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    emb = torch.cat((torch.outer(positions.float(), inv),) * 2, dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def _torch_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """apply_rope_with_cos_sin (flashinfer_full_verify.py:324-333) as 16-bit tensor ops."""
    h = x.shape[-1] // 2
    return (x * cos[:, None, :]) + (torch.cat((-x[..., h:], x[..., :h]), dim=-1) * sin[:, None, :])


@pytest.mark.parametrize("prefix_len,split_target", [(16384, None), (300, None), (4000, 4096)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_rope_matches_reference_rope_then_append(dev, prefix_len, split_target, dtype):
    """run(..., rope_cos_sin=(cos, sin)) given the projections before the
    rotary embedding (positions prefix_len + depth, as the reference's verify
    step builds them, flashinfer_full_verify.py:1197-1213): the cache holds
    the K rows that the reference's rotation + write_suffix_kv leave and the
    oracle's per-op rounding gives (bit-exact), and the output equals the
    attention of the torch-rotated queries (bit-exact) and the oracle (2e-3)."""
    from oracle import rope as orope

    ta = pkg("tree_attention")
    ffv = pkg("flashinfer_full_verify")
    kv_ops = pkg("kv_ops")
    gen = torch.Generator().manual_seed(prefix_len + 11)
    routes = _routes(gen, 9, 4, share=True)
    c = _build(dev, seed=prefix_len + 13, prefix_len=prefix_len, routes=routes, dtype=dtype, spare_pages=9)
    n, ps, hkv, d, hq = c["n"], c["ps"], c["hkv"], c["d"], c["hq"]
    q_raw = (torch.randn((n, hq, d), generator=gen) * 2.0).to(dtype)
    k_raw = (torch.randn((n, hkv, d), generator=gen) * 2.0).to(dtype)
    v_new = (torch.randn((n, hkv, d), generator=gen) * 0.1).to(dtype)
    cos, sin = _rope_tables(prefix_len + c["spec"].depths.cpu(), d, dtype)
    cos_d, sin_d = cos.to(dev), sin.to(dev)
    q_rot = _torch_rope(q_raw.to(dev), cos_d, sin_d)
    k_rot = _torch_rope(k_raw.to(dev), cos_d, sin_d)
    odt = "f16" if dtype == torch.float16 else "bf16"
    k_or = orope.apply_rope(k_raw.float().numpy(), cos.float().numpy(), sin.float().numpy(), odt)
    assert np.array_equal(k_rot.float().cpu().numpy(), k_or)
    order = c["order"].tolist()
    slots = torch.tensor([order[p // ps] * ps + p % ps for p in range(prefix_len, prefix_len + n)],
                         dtype=torch.int64, device=dev)
    last = ffv.last_page_len(c["kv_len"], ps)
    results = []
    for fused in (False, True):
        kv = c["kv"].to(dev)
        w = ta.BatchPrefillWithPagedKVCacheWrapper(torch.empty(64 << 20, dtype=torch.uint8, device=dev), "NHD")
        if split_target is not None:
            w.split_target_items = split_target
        w.plan(torch.tensor([0, n], dtype=torch.int32, device=dev),
               torch.tensor([0, c["pages"]], dtype=torch.int32, device=dev), c["order"].to(dev),
               torch.tensor([last], dtype=torch.int32, device=dev), hq, hkv, d, ps,
               custom_mask=c["spec"].bool_mask, q_data_type=dtype)
        if fused:
            out, lse = w.run(q_raw.to(dev), kv, return_lse=True, append_key_states=k_raw.to(dev),
                             append_value_states=v_new.to(dev), rope_cos_sin=(cos_d, sin_d))
        else:
            kv_ops.append_paged([kv], [k_rot], [v_new.to(dev)], dst_slots=slots)
            out, lse = w.run(q_rot, kv, return_lse=True)
        torch.cuda.synchronize()
        results.append((kv.cpu(), out.cpu(), lse.cpu()))
    (kv_a, out_a, lse_a), (kv_b, out_b, lse_b) = results
    assert torch.equal(kv_a.view(torch.int16), kv_b.view(torch.int16))
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16)) and torch.equal(lse_a, lse_b)
    ro, rl = oatt.masked_attention(q_rot.double().cpu().numpy(), kv_b.double().numpy(), [0, n], [0, c["pages"]],
                                   order, [last], masks=[c["mask"]])
    assert float(np.abs(out_b.float().numpy() - ro).max()) <= ATOL
    assert float(np.abs(lse_b.numpy() - rl).max()) <= ATOL


def test_fused_rope_batched_requests_and_refusals(dev):
    """Two ragged causal requests whose cos / sin rows follow their own
    positions (table row = query row): the cache gets the oracle-rotated K
    rows and V rows unchanged, and the output matches the oracle on the
    oracle-rotated queries.  Then the refusals: RoPE without the fused
    append, tables of another dtype, too few table rows."""
    from oracle import rope as orope

    ta = pkg("tree_attention")
    gen = torch.Generator().manual_seed(91)
    hq, hkv, d, ps = 32, 8, 128, 32
    qo_lens, kv_lens = [6, 13], [900, 2500]
    pages = [math.ceil(k / ps) for k in kv_lens]
    pool = sum(pages) + 3
    perm = torch.randperm(pool, generator=gen).tolist()
    table = [perm[: pages[0]], perm[pages[0]: pages[0] + pages[1]]]
    dt = torch.bfloat16
    kv = (torch.randn((pool, 2, ps, hkv, d), generator=gen) * 0.3).to(dt)
    q = (torch.randn((sum(qo_lens), hq, d), generator=gen) * 0.5).to(dt)
    k_new = (torch.randn((sum(qo_lens), hkv, d), generator=gen) * 0.5).to(dt)
    v_new = (torch.randn((sum(qo_lens), hkv, d), generator=gen) * 0.1).to(dt)
    positions = torch.cat([torch.arange(k - l, k) for k, l in zip(kv_lens, qo_lens)])
    cos, sin = _rope_tables(positions, d, dt)
    qo = [0, qo_lens[0], sum(qo_lens)]
    kvp = [0, pages[0], sum(pages)]
    last = [k - (p - 1) * ps for k, p in zip(kv_lens, pages)]
    w = ta.BatchPrefillWithPagedKVCacheWrapper(torch.empty(64 << 20, dtype=torch.uint8, device=dev), "NHD")
    w.plan(torch.tensor(qo, dtype=torch.int32), torch.tensor(kvp, dtype=torch.int32),
           torch.tensor(table[0] + table[1], dtype=torch.int32, device=dev), torch.tensor(last, dtype=torch.int32),
           hq, hkv, d, ps, causal=True, q_data_type=dt)
    kv_dev = kv.to(dev)
    out = w.run(q.to(dev), kv_dev, append_key_states=k_new.to(dev), append_value_states=v_new.to(dev),
                rope_cos_sin=(cos.to(dev), sin.to(dev)))
    torch.cuda.synchronize()
    k_rot = torch.from_numpy(orope.apply_rope(k_new.float().numpy(), cos.float().numpy(), sin.float().numpy(),
                                              "bf16")).to(dt)
    q_rot = orope.apply_rope(q.float().numpy(), cos.float().numpy(), sin.float().numpy(), "bf16")
    expect = kv.clone()
    for b in range(2):
        for i in range(qo_lens[b]):
            p = kv_lens[b] - qo_lens[b] + i
            expect[table[b][p // ps], 0, p % ps] = k_rot[qo[b] + i]
            expect[table[b][p // ps], 1, p % ps] = v_new[qo[b] + i]
    assert torch.equal(kv_dev.cpu().view(torch.int16), expect.view(torch.int16))
    ro, _ = oatt.masked_attention(q_rot.astype(np.float64), expect.double().numpy(), qo, kvp,
                                  table[0] + table[1], last, causal=True)
    assert float(np.abs(out.float().cpu().numpy() - ro).max()) <= ATOL
    with pytest.raises(NotImplementedError):
        w.run(q.to(dev), kv_dev, rope_cos_sin=(cos.to(dev), sin.to(dev)))
    with pytest.raises(TypeError):
        w.run(q.to(dev), kv_dev, append_key_states=k_new.to(dev), append_value_states=v_new.to(dev),
              rope_cos_sin=(cos.half().to(dev), sin.half().to(dev)))
    with pytest.raises(ValueError):
        w.run(q.to(dev), kv_dev, append_key_states=k_new.to(dev), append_value_states=v_new.to(dev),
              rope_cos_sin=(cos[:-1].to(dev), sin[:-1].to(dev)))



@pytest.mark.parametrize("inference", [False, True])
def test_plan_sees_index_tensors_changed_in_place(dev, inference):
    """The tree builder's index tensors carry their host values; a plan reads
    those only while the tensor is unchanged.  After an in-place write the
    plan reads the device values again (here: a longer last page, so one more
    key per row, checked against the oracle).  The same holds when the spec
    is built and changed under torch.inference_mode, as the Target verify
    does."""
    import contextlib

    ta = pkg("tree_attention")
    ffv = pkg("flashinfer_full_verify")
    gen = torch.Generator().manual_seed(31)
    routes = _routes(gen, 3, 4, share=True)
    ctx = torch.inference_mode() if inference else contextlib.nullcontext()
    with ctx:
        c = _build(dev, seed=31, prefix_len=300, routes=routes, permute=False, spare_pages=1)
        _plan_changed_in_place(dev, ta, ffv, c)


def _plan_changed_in_place(dev, ta, ffv, c):
    spec = c["spec"]
    assert spec.kv_last_page_len._atlas_host_values[0] == [ffv.last_page_len(c["kv_len"], 16)]
    ws = torch.empty(16 * 1024 * 1024, dtype=torch.uint8, device=dev)
    w = ta.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(spec.qo_indptr, spec.kv_indptr, spec.kv_indices, spec.kv_last_page_len, c["hq"], c["hkv"], c["d"], 16,
           causal=True, q_data_type=torch.float16)
    assert w.current_plan.kv_lens == [c["kv_len"]]
    # a last page one key longer reads one more row of the same page (the
    # cache buffer holds whole pages)
    old_last = ffv.last_page_len(c["kv_len"], 16)
    assert old_last < 16
    spec.kv_last_page_len.add_(1)
    w.plan(spec.qo_indptr, spec.kv_indptr, spec.kv_indices, spec.kv_last_page_len, c["hq"], c["hkv"], c["d"], 16,
           causal=True, q_data_type=torch.float16)
    kv_len = c["kv_len"] + 1
    assert w.current_plan.kv_lens == [kv_len]
    out = w.run(c["q"].to(dev), c["kv"].to(dev))
    torch.cuda.synchronize()
    n = c["n"]
    causal = np.zeros((n, kv_len), dtype=bool)
    for i in range(n):
        causal[i, : kv_len - n + i + 1] = True
    ro, _ = oatt.masked_attention(c["q"].float().numpy().astype(np.float64), c["kv"].float().numpy().astype(np.float64),
                                  [0, n], [0, c["pages"]], list(range(c["pages"])), [old_last + 1], masks=[causal])
    assert float(np.abs(out.float().cpu().numpy() - ro).max()) <= ATOL


def test_replans_reuse_and_refresh_the_work_list(dev):
    """Planning the same shape again reuses the work decomposition and skips
    the metadata upload; a different shape in between re-uploads it.  Every
    run matches the oracle."""
    gen = torch.Generator().manual_seed(37)
    routes = _routes(gen, 3, 4, share=True)
    ta = pkg("tree_attention")
    ffv = pkg("flashinfer_full_verify")
    ws = torch.empty(64 * 1024 * 1024, dtype=torch.uint8, device=dev)
    w = ta.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    cases = [_build(dev, seed=40 + i, prefix_len=p, routes=routes) for i, p in enumerate((5000, 700, 5000))]
    decomps = []
    for c in cases:
        last = ffv.last_page_len(c["kv_len"], c["ps"])
        w.plan(torch.tensor([0, c["n"]], dtype=torch.int32, device=dev),
               torch.tensor([0, c["pages"]], dtype=torch.int32, device=dev), c["order"].to(dev),
               torch.tensor([last], dtype=torch.int32, device=dev), c["hq"], c["hkv"], c["d"], c["ps"],
               custom_mask=c["spec"].bool_mask, causal=False, q_data_type=c["dtype"])
        decomps.append(w._decomp_cache[1])
        out, lse = w.run(c["q"].to(dev), c["kv"].to(dev), return_lse=True)
        torch.cuda.synchronize()
        ro, rl = oatt.masked_attention(
            c["q"].float().numpy().astype(np.float64), c["kv"].float().numpy().astype(np.float64),
            [0, c["n"]], [0, c["pages"]], c["order"].tolist(), [last], masks=[c["mask"]])
        assert float(np.abs(out.float().cpu().numpy() - ro).max()) <= ATOL
        assert float(np.abs(lse.cpu().numpy() - rl).max()) <= ATOL
    assert decomps[0] is not decomps[1] and decomps[1] is not decomps[2]
    assert np.array_equal(decomps[0]["meta"], decomps[2]["meta"])
    # the same inputs twice in a row reuse the decomposition object
    c = cases[2]
    last = ffv.last_page_len(c["kv_len"], c["ps"])
    w.plan(torch.tensor([0, c["n"]], dtype=torch.int32), torch.tensor([0, c["pages"]], dtype=torch.int32),
           c["order"].to(dev), torch.tensor([last], dtype=torch.int32), c["hq"], c["hkv"], c["d"], c["ps"],
           custom_mask=c["spec"].bool_mask, causal=False, q_data_type=c["dtype"])
    assert w._decomp_cache[1] is decomps[2]


@pytest.mark.parametrize("seed", range(12))
def test_random_request_mixes_match_oracle(dev, seed):
    """Seeded random batches: 1-4 requests, each with its own route tree (1-5
    routes of depth 1-5, shared prefixes or not) over a prefix of 0-3000
    tokens on scattered pages; one of several head layouts, head dims 64 or
    128, pages of 1, 16 or 64 tokens, fp16 or bf16, sometimes a forced split
    target or row cap.  Every request's O and LSE within 2e-3 of the
    oracle."""
    ta = pkg("tree_attention")
    ffv = pkg("flashinfer_full_verify")
    pick = np.random.default_rng(1000 + seed)
    gen = torch.Generator().manual_seed(seed)
    hq, hkv = [(32, 8), (8, 8), (16, 2), (32, 4)][int(pick.integers(4))]
    d = int(pick.choice([64, 128]))
    ps = int(pick.choice([1, 16, 64]))
    dtype = [torch.float16, torch.bfloat16][int(pick.integers(2))]
    batch = int(pick.integers(1, 5))
    specs, qs, masks, pages_per, lasts = [], [], [], [], []
    for i in range(batch):
        routes = _routes(gen, int(pick.integers(1, 6)), int(pick.integers(1, 6)), share=bool(pick.integers(2)))
        prefix = int(pick.integers(0, 3001))
        spec, _ = ffv.build_deduplicated_tree_spec_from_paths(paths=routes, prefix_len=prefix, page_size=ps,
                                                              device=dev)
        _, parents, _, _ = ref.dedup_tree(routes)
        specs.append(spec)
        masks.append(ref.ancestor_mask(parents, prefix))
        qs.append(torch.randn((spec.node_count, hq, d), generator=gen))
        kv_len = prefix + spec.node_count
        pages_per.append(math.ceil(kv_len / ps))
        lasts.append(ffv.last_page_len(kv_len, ps))
    total = sum(pages_per)
    pool = total + 11
    perm = torch.randperm(pool, generator=gen)[:total].to(torch.int32)
    kv = torch.randn((pool, 2, ps, hkv, d), generator=gen)
    kv[:, 1] *= 0.1
    kv = kv.to(dtype)
    q = torch.cat(qs).to(dtype)
    qo, kvp = [0], [0]
    for s, p in zip(specs, pages_per):
        qo.append(qo[-1] + s.node_count)
        kvp.append(kvp[-1] + p)
    flat_mask = torch.cat([torch.from_numpy(m.reshape(-1)) for m in masks]).to(dev)
    w = ta.BatchPrefillWithPagedKVCacheWrapper(torch.empty(64 << 20, dtype=torch.uint8, device=dev), "NHD")
    w.split_target_items = [None, None, 1, 64, 600][int(pick.integers(5))]
    w.max_rows_per_item = [None, None, 32][int(pick.integers(3))]
    w.plan(torch.tensor(qo, dtype=torch.int32, device=dev), torch.tensor(kvp, dtype=torch.int32, device=dev),
           perm.to(dev), torch.tensor(lasts, dtype=torch.int32, device=dev), hq, hkv, d, ps,
           custom_mask=flat_mask, q_data_type=dtype)
    out, lse = w.run(q.to(dev), kv.to(dev), return_lse=True)
    torch.cuda.synchronize()
    ro, rl = oatt.masked_attention(q.float().numpy().astype(np.float64), kv.float().numpy().astype(np.float64),
                                   qo, kvp, perm.tolist(), lasts, masks=masks)
    case = f"seed {seed}: hq {hq} hkv {hkv} d {d} ps {ps} {dtype} batch {batch}"
    assert float(np.abs(out.float().cpu().numpy() - ro).max()) <= ATOL, case
    assert float(np.abs(lse.cpu().numpy() - rl).max()) <= ATOL, case


@pytest.mark.parametrize("n_routes,prefix_len,split_target", [
    (17, 300, None),    # 68 nodes: two tiles of words, unaligned tree start
    (32, 64, 1024),     # 128 nodes from a tile boundary, many splits
    (64, 4000, 240),    # 256 nodes after a long prefix: the tree spans five tiles of the last splits
    (64, 16, 4096),     # 256 nodes after a tiny prefix, most items masked
])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_wide_trees_beyond_64_columns(dev, n_routes, prefix_len, split_target, dtype):
    """Trees of 65 to 256 nodes (one visibility word per 64-key tile of the
    tree region), with and without splits, against the oracle; the dominant
    tree case puts almost all softmax mass on each row's own ancestors, so a
    wrong word or bit shows in full."""
    gen = torch.Generator().manual_seed(n_routes + prefix_len)
    routes = _routes(gen, n_routes, 4, share=False)
    for dominant in (False, True):
        c = _build(dev, seed=n_routes + prefix_len + dominant, prefix_len=prefix_len, routes=routes, dtype=dtype,
                   dominant_tree=dominant)
        assert c["n"] > 64
        w, _, _ = _run_and_check(dev, c, split_target=split_target)
        plan = w.current_plan
        assert plan.mask_words >= 2
        assert plan.mask_words == (c["kv_len"] - 1) // 64 - prefix_len // 64 + 1


def test_wide_tree_masks_batched_with_narrow_and_dense_paths(dev):
    """A batch mixing a 130-node tree with 12-node trees in one plan (the
    dense mask path: every request in the per-tile layout), and a 68-node tree
    planned from a packed mask, against the oracle request by request; also
    the head_dim 64 kernel on a wide tree."""
    ta = pkg("tree_attention")
    ffv = pkg("flashinfer_full_verify")
    gen = torch.Generator().manual_seed(21)
    for d, hq, hkv in ((128, 32, 8), (64, 32, 8)):
        ps = 16
        prefixes = [700, 37, 2100]
        route_sets = [_routes(gen, 3, 4, share=True), _routes(gen, 33, 4, share=False), _routes(gen, 3, 4, share=False)]
        specs, qs, masks, kv_lens, pages_per, lasts = [], [], [], [], [], []
        for p, routes in zip(prefixes, route_sets):
            spec, _ = ffv.build_deduplicated_tree_spec_from_paths(paths=routes, prefix_len=p, page_size=ps,
                                                                  device=dev)
            _, parents, _, _ = ref.dedup_tree(routes)
            specs.append(spec)
            masks.append(ref.ancestor_mask(parents, p))
            qs.append(torch.randn((spec.node_count, hq, d), generator=gen))
            kv_lens.append(p + spec.node_count)
            pages_per.append(math.ceil(kv_lens[-1] / ps))
            lasts.append(ffv.last_page_len(kv_lens[-1], ps))
        assert specs[1].node_count > 128
        total_pages = sum(pages_per)
        pool = total_pages + 40
        perm = torch.randperm(pool, generator=gen)[:total_pages].to(torch.int32)
        kv = torch.randn((pool, 2, ps, hkv, d), generator=gen)
        kv[:, 1] *= 0.1
        kv = kv.to(torch.float16)
        q = torch.cat(qs).to(torch.float16)
        qo, kvp = [0], [0]
        for s_, p_ in zip(specs, pages_per):
            qo.append(qo[-1] + s_.node_count)
            kvp.append(kvp[-1] + p_)
        flat_mask = torch.cat([torch.from_numpy(m.reshape(-1)) for m in masks]).to(dev)
        ws = torch.empty(64 * 1024 * 1024, dtype=torch.uint8, device=dev)
        w = ta.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
        w.plan(torch.tensor(qo, dtype=torch.int32, device=dev), torch.tensor(kvp, dtype=torch.int32, device=dev),
               perm.to(dev), torch.tensor(lasts, dtype=torch.int32, device=dev), hq, hkv, d, ps,
               custom_mask=flat_mask, q_data_type=torch.float16)
        assert w.current_plan.mask_words >= 2
        out, lse = w.run(q.to(dev), kv.to(dev), return_lse=True)
        torch.cuda.synchronize()
        ro, rl = oatt.masked_attention(q.float().numpy().astype(np.float64), kv.float().numpy().astype(np.float64),
                                       qo, kvp, perm.tolist(), lasts, masks=masks)
        assert float(np.abs(out.float().cpu().numpy() - ro).max()) <= ATOL, d
        assert float(np.abs(lse.cpu().numpy() - rl).max()) <= ATOL, d
    # one request, a packed mask (no attached window: derived from the mask)
    routes = _routes(gen, 17, 4, share=False)
    c = _build(dev, seed=5, prefix_len=500, routes=routes)
    _run_and_check(dev, c, use_packed=True)


def test_wide_tree_mask_refused_beyond_its_width(dev):
    """A mask whose non-visible region spans more columns than the per-tile
    layout covers is refused at plan time."""
    ta = pkg("tree_attention")
    n, kv = 2, ta.MAX_WIDE_TREE_WIDTH + 70
    mask = torch.ones((n, kv), dtype=torch.bool)
    mask[0, 5] = False
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=dev)
    w = ta.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    pages = math.ceil(kv / 16)
    with pytest.raises(NotImplementedError, match="spans more than"):
        w.plan(torch.tensor([0, n], dtype=torch.int32, device=dev), torch.tensor([0, pages], dtype=torch.int32,
               device=dev), torch.arange(pages, dtype=torch.int32, device=dev),
               torch.tensor([kv - (pages - 1) * 16], dtype=torch.int32, device=dev), 32, 8, 128, 16,
               custom_mask=mask.reshape(-1).to(dev), q_data_type=torch.float16)


@pytest.mark.parametrize("case", ["forest16k", "forest16k_split1", "short61_bf16", "d64_ps32", "wide130_bf16",
                                  "causal_free_4k"])
def test_hnd_pages_match_oracle_and_nhd_bit_for_bit(dev, case):
    """HND pages [pool, 2, Hkv, ps, D] (each KV head's keys of a page one
    contiguous run) holding the NHD case's values: within 2e-3 of the fp64
    oracle and bit-equal to the NHD run, on the head_dim-128 kernel (one
    split and many), the generic kernel (head_dim 64, page 32), a wide tree
    and a short prefix."""
    gen = torch.Generator().manual_seed(91)
    kw, split = {}, None
    if case.startswith("forest16k"):
        routes, prefix = _routes(gen, 9, 4, share=True), 16384
        split = 1 if case.endswith("split1") else None
    elif case == "short61_bf16":
        routes, prefix, kw = _routes(gen, 4, 3, share=True), 61, dict(dtype=torch.bfloat16)
    elif case == "d64_ps32":
        routes, prefix, kw = _routes(gen, 6, 4, share=True), 3000, dict(hq=16, hkv=2, d=64, ps=32)
    elif case == "wide130_bf16":
        routes, prefix, kw = _routes(gen, 26, 5, share=False), 5000, dict(dtype=torch.bfloat16)
    else:
        routes, prefix = _routes(gen, 3, 4, share=False), 4096
    c = _build(dev, seed=92, prefix_len=prefix, routes=routes, **kw)
    _run_and_check(dev, c, split_target=split, layout="NHD")
    _run_and_check(dev, c, split_target=split, layout="HND")
    (o_n, l_n), (o_h, l_h) = c["outs"][("NHD", split)], c["outs"][("HND", split)]
    assert torch.equal(o_n.view(torch.int16), o_h.view(torch.int16)) and torch.equal(l_n, l_h)


@pytest.mark.parametrize("prefix_len", [16384, 300])
def test_hnd_fused_rope_append_matches_nhd(dev, prefix_len):
    """The fused RoPE + append + attention launch on HND pages writes the
    same rows (read back as NHD) and returns the same output, bit for bit,
    as on NHD pages."""
    ta = pkg("tree_attention")
    ffv = pkg("flashinfer_full_verify")
    dtype = torch.float16
    gen = torch.Generator().manual_seed(prefix_len + 5)
    routes = _routes(gen, 9, 4, share=True)
    c = _build(dev, seed=prefix_len + 6, prefix_len=prefix_len, routes=routes, dtype=dtype, spare_pages=9)
    n, ps, hkv, d, hq = c["n"], c["ps"], c["hkv"], c["d"], c["hq"]
    q_raw = (torch.randn((n, hq, d), generator=gen) * 2.0).to(dtype).to(dev)
    k_raw = (torch.randn((n, hkv, d), generator=gen) * 2.0).to(dtype).to(dev)
    v_new = (torch.randn((n, hkv, d), generator=gen) * 0.1).to(dtype).to(dev)
    cos, sin = _rope_tables(prefix_len + c["spec"].depths.cpu(), d, dtype)
    last = ffv.last_page_len(c["kv_len"], ps)
    results = []
    for layout in ("NHD", "HND"):
        kv = (c["kv"] if layout == "NHD" else _hnd(c["kv"])).to(dev)
        w = ta.BatchPrefillWithPagedKVCacheWrapper(torch.empty(64 << 20, dtype=torch.uint8, device=dev), layout)
        w.plan(torch.tensor([0, n], dtype=torch.int32, device=dev),
               torch.tensor([0, c["pages"]], dtype=torch.int32, device=dev), c["order"].to(dev),
               torch.tensor([last], dtype=torch.int32, device=dev), hq, hkv, d, ps,
               custom_mask=c["spec"].bool_mask, q_data_type=dtype)
        out, lse = w.run(q_raw, kv, return_lse=True, append_key_states=k_raw, append_value_states=v_new,
                         rope_cos_sin=(cos.to(dev), sin.to(dev)))
        torch.cuda.synchronize()
        results.append(((kv if layout == "NHD" else kv.permute(0, 1, 3, 2, 4)).cpu(), out.cpu(), lse.cpu()))
    (kv_a, out_a, lse_a), (kv_b, out_b, lse_b) = results
    assert torch.equal(kv_a.view(torch.int16), kv_b.contiguous().view(torch.int16))
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16)) and torch.equal(lse_a, lse_b)


@pytest.mark.parametrize("n_routes,depth,prefix,dedup", [(9, 4, 16384, True), (3, 4, 0, True), (1, 1, 7, False),
                                                         (40, 4, 100, True), (300, 5, 64, True), (6, 3, 61, False)])
def test_device_tree_spec_equals_host_spec(dev, n_routes, depth, prefix, dedup):
    """A tree spec built for the device (one atlas_tree_spec_upload launch
    copies the buffer from the pinned ring and fills the dense mask in the
    same allocation; a spec larger than the ring's quarter is copied first)
    equals the one built for the host, tensor for tensor, and the oracle's
    ancestor mask; the plan's cached window and tile words ride along, and an
    in-place change of the device mask is seen by the plan (version counter)."""
    import random

    ffv = pkg("flashinfer_full_verify")
    ta = pkg("tree_attention")
    rng = random.Random(n_routes * 31 + depth)
    paths = [tuple(rng.randrange(6) for _ in range(depth)) for _ in range(n_routes)]
    build = ffv.build_deduplicated_tree_spec_from_paths if dedup else ffv.build_tree_spec_from_paths
    outs = [build(paths=paths, prefix_len=prefix, page_size=16, device=d) for d in (dev, "cpu")]
    (gpu, cpu) = [o[0] if dedup else o for o in outs]
    torch.cuda.synchronize()
    for name in ("flat_token_ids", "depths", "bool_mask", "qo_indptr", "kv_indptr", "kv_indices", "kv_last_page_len"):
        assert torch.equal(getattr(gpu, name).cpu(), getattr(cpu, name)), name
    assert (gpu.node_count, gpu.kv_len, gpu.total_pages, gpu.parent_indices) == \
        (cpu.node_count, cpu.kv_len, cpu.total_pages, cpu.parent_indices)
    _, parents, _, _ = ref.dedup_tree(paths) if dedup else (None, cpu.parent_indices, None, None)
    mask = ref.ancestor_mask(list(parents), prefix)
    assert gpu.bool_mask.cpu().numpy().tolist() == mask.reshape(-1).tolist()
    n, kv = gpu.node_count, gpu.kv_len
    if n <= 64:
        assert torch.equal(gpu.tree_mask.cpu(), cpu.tree_mask)
        assert ta._cached_tree_window(gpu.bool_mask, [n], [kv]) is not None
        gpu.bool_mask[kv * (n - 1) + prefix] = not bool(gpu.bool_mask[kv * (n - 1) + prefix])
        assert ta._cached_tree_window(gpu.bool_mask, [n], [kv]) is None
    elif n <= 1024:
        assert ta._cached_tree_tiles(gpu.bool_mask, [n], [kv]) is not None


@pytest.mark.parametrize("source", ["mapped", "device", "in_place"])
def test_tree_spec_upload_copies_and_fills(dev, source):
    """atlas_tree_spec_upload from mapped pinned memory, from another device
    buffer, and in place (mask only): the spec bytes arrive unchanged (an odd
    length, so the last 16-byte chunk is partial) and the dense mask has the
    prefix columns set and the tree block after them."""
    import numpy as np

    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    rng = np.random.default_rng(7)
    n, prefix = 13, 70
    spec = rng.integers(0, 256, size=1000 + n * n, dtype=np.uint8)
    spec[-n * n:] = rng.integers(0, 2, size=n * n)
    nbytes = int(spec.nbytes)
    dst = torch.full((nbytes + 15,), 0xEE, dtype=torch.uint8, device=dev)
    mask = torch.full((n * (prefix + n) + 5,), 0xEE, dtype=torch.uint8, device=dev)
    stream = lib_mod.stream_of(dev)
    print(f"tree spec upload: {source}", flush=True)

    def launch(src):
        lib_mod.check(lib.atlas_tree_spec_upload(src, nbytes, n, prefix, lib_mod.ptr(dst), lib_mod.ptr(mask), stream),
                      "atlas_tree_spec_upload")

    if source == "mapped":
        assert lib_mod.staging().stage(spec, dev, launch)
    elif source == "device":
        launch(lib_mod.ptr(torch.from_numpy(spec).to(dev)))
    else:
        dst[:nbytes].copy_(torch.from_numpy(spec))
        launch(lib_mod.ptr(dst))
    torch.cuda.synchronize()
    assert dst[:nbytes].cpu().numpy().tobytes() == spec.tobytes()
    assert dst[nbytes:].tolist() == [0xEE] * 15
    block = spec[-n * n:].reshape(n, n)
    want = np.concatenate([np.ones((n, prefix), dtype=np.uint8), block], axis=1).reshape(-1)
    got = mask.cpu().numpy()
    assert got[: want.size].tobytes() == want.tobytes() and got[want.size:].tolist() == [0xEE] * 5
