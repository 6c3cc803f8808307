"""Paged decode attention (one query per request) vs the oracle's closed form.

The decode wrapper plans a batch of single-query requests on the same paged
kernels as the verify attention.  Cases mirror the Drafter's use: forked routes
of a request share their prefix pages and own private tail pages (copy-on-write
copies), with ragged lengths.  Tolerance 2e-3 absolute on O and LSE
(fp16 / bf16), V drawn as N(0,1) * 0.1 as in the configs.
"""

import math
import types

import numpy as np
import pytest
import torch

from helpers import pkg
from oracle import attention as oatt

pytestmark = pytest.mark.gpu

ATOL = 2e-3


def _routes_batch(gen, *, requests, routes, prefix_range, extra_range, ps, pool_pages):
    """Page tables of forked routes: per request a shared run of full prefix
    pages, then per route a private tail (its own pages) of random length."""
    perm = torch.randperm(pool_pages, generator=gen).tolist()
    nxt = 0
    indptr, indices, last, kv_lens = [0], [], [], []
    for _ in range(requests):
        prefix = int(torch.randint(prefix_range[0], prefix_range[1] + 1, (1,), generator=gen))
        full = prefix // ps
        shared = perm[nxt : nxt + full]
        nxt += full
        for _ in range(routes):
            own = prefix - full * ps + int(torch.randint(extra_range[0], extra_range[1] + 1, (1,), generator=gen))
            own_pages = max(1, math.ceil(own / ps)) if own else 0
            pages = shared + perm[nxt : nxt + own_pages]
            nxt += own_pages
            kv_len = full * ps + own
            if kv_len == 0:
                pages, kv_len = perm[nxt : nxt + 1], 1
                nxt += 1
            indices.extend(pages)
            indptr.append(len(indices))
            last.append(kv_len - (len(pages) - 1) * ps)
            kv_lens.append(kv_len)
    assert nxt <= pool_pages
    return indptr, indices, last, kv_lens


def _check(dev, *, seed, requests, routes, prefix_range, extra_range, hq, hkv, d, ps, dtype, split=None,
           sm_scale=None, use_forward=False, cascade=True):
    da = pkg("decode_attention")
    gen = torch.Generator().manual_seed(seed)
    pool_pages = requests * (prefix_range[1] // ps + 1) + requests * routes * (extra_range[1] // ps + 2) + 4
    indptr, indices, last, kv_lens = _routes_batch(gen, requests=requests, routes=routes, prefix_range=prefix_range,
                                                   extra_range=extra_range, ps=ps, pool_pages=pool_pages)
    batch = requests * routes
    kv = torch.randn((pool_pages, 2, ps, hkv, d), generator=gen)
    kv[:, 1] *= 0.1
    q = torch.randn((batch, hq, d), generator=gen)
    kv, q = kv.to(dtype), q.to(dtype)
    ws = torch.empty(64 * 1024 * 1024, dtype=torch.uint8, device=dev)
    w = da.BatchDecodeWithPagedKVCacheWrapper(ws, "NHD")
    w.use_cascade = cascade
    if split is not None:
        w.split_target_items = split
    w.begin_forward(torch.tensor(indptr, dtype=torch.int32, device=dev),
                    torch.tensor(indices, dtype=torch.int32, device=dev),
                    torch.tensor(last, dtype=torch.int32, device=dev), hq, hkv, d, ps,
                    data_type=dtype, q_data_type=dtype, non_blocking=True)
    kv_dev = kv.to(dev)
    # the Drafter passes (K, V) views of its token pools as [pages, page_size, Hkv, D]
    paged = (kv_dev[:, 0], kv_dev[:, 1])
    if use_forward:
        out = w.forward(q.to(dev), paged, sm_scale=sm_scale, logits_soft_cap=None, k_scale=None, v_scale=1.0)
        lse = None
    else:
        out, lse = w.run(q.to(dev), paged, return_lse=True)
    torch.cuda.synchronize()
    ro, rl = oatt.masked_attention(q.double().numpy(), kv.double().numpy(), list(range(batch + 1)), indptr, indices,
                                   last, sm_scale=sm_scale)
    err = float(np.abs(out.float().cpu().numpy() - ro).max())
    assert err <= ATOL, f"max |O - ref| = {err}"
    if lse is not None:
        lerr = float(np.abs(lse.cpu().numpy() - rl).max())
        assert lerr <= ATOL, f"max |lse - ref| = {lerr}"
    return w, kv_lens


@pytest.mark.parametrize("d,ps", [(64, 64), (64, 16), (128, 16), (128, 64)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_forked_routes_shared_prefix(dev, d, ps, dtype):
    """8 requests x 9 routes (the Drafter's fork stress shape), prefixes of
    128..1024 tokens, private tails of 1..72 tokens: every request's routes
    form one cascade group (shared prefix pass + per-route tails, merged)."""
    w, _ = _check(dev, seed=d + ps, requests=8, routes=9, prefix_range=(128, 1024), extra_range=(1, 72), hq=32,
                  hkv=8, d=d, ps=ps, dtype=dtype)
    assert w.cascade_groups == 8
    assert w.current_plan.num_merge > 0


@pytest.mark.parametrize("d", [64, 128])
def test_forked_routes_without_cascade(dev, d):
    """The same batches with every route streaming its whole page list."""
    w, _ = _check(dev, seed=30 + d, requests=4, routes=9, prefix_range=(128, 1024), extra_range=(1, 72), hq=32,
                  hkv=8, d=d, ps=64, dtype=torch.bfloat16, cascade=False)
    assert w.cascade_groups == 0


@pytest.mark.parametrize("split", [None, 1, 4096])
def test_cascade_long_shared_prefix(dev, split):
    """Long shared prefixes (3k-9k tokens) split over work items, groups of
    up to 12 routes (48 packed rows per KV head), plus routes that share
    nothing (one-route requests) in the same batch."""
    w, _ = _check(dev, seed=41, requests=3, routes=12, prefix_range=(3000, 9000), extra_range=(1, 100), hq=32,
                  hkv=8, d=64, ps=64, dtype=torch.bfloat16, split=split)
    assert w.cascade_groups == 3
    w, _ = _check(dev, seed=42, requests=5, routes=1, prefix_range=(3000, 9000), extra_range=(1, 100), hq=32,
                  hkv=8, d=128, ps=16, dtype=torch.float16, split=split)
    assert w.cascade_groups == 0


@pytest.mark.parametrize("split", [None, 1, 4096])
def test_long_contexts_split_and_unsplit(dev, split):
    """Contexts of 3k-9k tokens: keys split over work items (merged) or not."""
    w, _ = _check(dev, seed=7, requests=2, routes=3, prefix_range=(3000, 9000), extra_range=(0, 40), hq=32, hkv=8,
                  d=64, ps=64, dtype=torch.bfloat16, split=split, cascade=False)
    if split == 1:
        assert w.current_plan.num_merge == 0
    if split == 4096:
        assert w.current_plan.num_merge > 0


def test_single_token_contexts_and_gqa_variants(dev):
    _check(dev, seed=11, requests=3, routes=2, prefix_range=(0, 0), extra_range=(1, 1), hq=16, hkv=2, d=128, ps=16,
           dtype=torch.float16)
    _check(dev, seed=12, requests=2, routes=2, prefix_range=(0, 40), extra_range=(0, 9), hq=8, hkv=8, d=64, ps=32,
           dtype=torch.bfloat16)


def test_forward_sm_scale_and_unsupported_options(dev):
    """SGLang's forward(): its sm_scale replaces the plan's; soft-capping and
    KV scales other than 1 are refused; run before plan raises."""
    w, _ = _check(dev, seed=13, requests=2, routes=3, prefix_range=(64, 300), extra_range=(1, 20), hq=32, hkv=8,
                  d=64, ps=64, dtype=torch.bfloat16, sm_scale=0.05, use_forward=True)
    q = torch.zeros((6, 32, 64), dtype=torch.bfloat16, device=dev)
    kv = torch.zeros((64, 2, 64, 8, 64), dtype=torch.bfloat16, device=dev)
    with pytest.raises(NotImplementedError):
        w.forward(q, kv, logits_soft_cap=30.0)
    with pytest.raises(NotImplementedError):
        w.run(q, kv, k_scale=2.0)
    da = pkg("decode_attention")
    fresh = da.BatchDecodeWithPagedKVCacheWrapper(torch.empty(1024, dtype=torch.uint8, device=dev))
    with pytest.raises(RuntimeError):
        fresh.run(q, kv)


def test_reference_plan_helper(dev):
    """flashinfer_full_verify.plan_decode_wrapper (one request over pages
    0..n-1, keyword retry ladder) on the drop-in wrapper."""
    ffv = pkg("flashinfer_full_verify")
    args = types.SimpleNamespace(workspace_mb=16, device=dev, page_size=16, flashinfer_backend="auto")
    config = types.SimpleNamespace(hidden_size=32 * 64, num_attention_heads=32, num_key_value_heads=8, head_dim=64)
    w = ffv.make_decode_wrapper(args=args)
    seq = 300
    ffv.plan_decode_wrapper(w, seq_len=seq, args=args, config=config, dtype=torch.float16)
    gen = torch.Generator().manual_seed(14)
    pages = math.ceil(seq / 16)
    kv = (torch.randn((pages, 2, 16, 8, 64), generator=gen) * 0.5).half()
    q = (torch.randn((1, 32, 64), generator=gen) * 0.5).half()
    out = w.run(q.to(dev), kv.to(dev))
    torch.cuda.synchronize()
    ro, _ = oatt.masked_attention(q.double().numpy(), kv.double().numpy(), [0, 1], [0, pages], list(range(pages)),
                                  [seq - (pages - 1) * 16])
    assert float(np.abs(out.float().cpu().numpy() - ro).max()) <= ATOL


def test_cascade_graph_replays_match_eager(dev):
    """The Drafter's decode attention over forked routes (cascade plan:
    shared-prefix splits, per-route tails, merge), 3 layers captured in a HIP
    graph and replayed several times with eager work, synchronisations and a
    re-plan of the same batch in between: every replay equals the eager
    result bit for bit, and the eager result is within 2e-3 of the oracle."""
    da = pkg("decode_attention")
    gen = torch.Generator().manual_seed(31)
    hq, hkv, d, ps, layers = 32, 8, 64, 64, 3
    requests, routes = 4, 9
    pool_pages = 4 * (1024 // ps + 1) + 36 * 3 + 4
    indptr, indices, last, kv_lens = _routes_batch(gen, requests=requests, routes=routes, prefix_range=(300, 1024),
                                                   extra_range=(1, 9), ps=ps, pool_pages=pool_pages)
    batch = requests * routes
    kvs = [torch.randn((pool_pages, 2, ps, hkv, d), generator=gen) for _ in range(layers)]
    for kv in kvs:
        kv[:, 1] *= 0.1
    qs = [torch.randn((batch, hq, d), generator=gen) for _ in range(layers)]
    kvs = [kv.to(torch.bfloat16).to(dev) for kv in kvs]
    qs = [q.to(torch.bfloat16).to(dev) for q in qs]
    ws = torch.empty(64 * 1024 * 1024, dtype=torch.uint8, device=dev)
    w = da.BatchDecodeWithPagedKVCacheWrapper(ws, "NHD", use_cuda_graph=True)

    def plan():
        w.plan(torch.tensor(indptr, dtype=torch.int32, device=dev), torch.tensor(indices, dtype=torch.int32, device=dev),
               torch.tensor(last, dtype=torch.int32, device=dev), hq, hkv, d, ps, data_type=torch.bfloat16,
               q_data_type=torch.bfloat16)

    outs = [torch.empty_like(q) for q in qs]

    def forward():
        for l in range(layers):
            w.run(qs[l], kvs[l], out=outs[l])

    plan()
    assert w.cascade_groups == requests
    forward()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    for l in range(layers):
        ro, _ = oatt.masked_attention(qs[l].float().cpu().numpy().astype(np.float64),
                                      kvs[l].float().cpu().numpy().astype(np.float64),
                                      list(range(batch + 1)), indptr, indices, last)
        assert float(np.abs(eager[l].float().cpu().numpy() - ro).max()) <= ATOL
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        forward()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        forward()
    for rep in range(4):
        for o in outs:
            o.zero_()
        if rep % 2:
            plan()  # the same batch planned again into the persistent buffers
        scratch = torch.randn(1 << 20, device=dev).sum()  # unrelated eager work
        graph.replay()
        torch.cuda.synchronize()
        assert float(scratch) == float(scratch)
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {rep} differs from eager"


@pytest.mark.parametrize("seed", range(8))
def test_random_forked_tables_match_oracle(dev, seed):
    """Seeded random decode batches: families of routes sharing a random
    number of leading full pages (each route with its own tail pages), single
    routes between them, scattered page ids; one of several head layouts,
    head dims 64 or 128, pages of 16 or 64 tokens, fp16 or bf16, sometimes a
    forced split target.  O and LSE within 2e-3 of the oracle."""
    da = pkg("decode_attention")
    pick = np.random.default_rng(700 + seed)
    gen = torch.Generator().manual_seed(seed)
    hq, hkv = [(32, 8), (8, 8), (16, 2), (32, 4)][int(pick.integers(4))]
    d = int(pick.choice([64, 128]))
    ps = int(pick.choice([16, 64]))
    dtype = [torch.float16, torch.bfloat16][int(pick.integers(2))]
    page_lists, last = [], []
    nxt = 0
    for _ in range(int(pick.integers(1, 5))):
        n_routes = 1 if pick.random() < 0.3 else int(pick.integers(2, 10))
        family = list(range(nxt, nxt + int(pick.integers(0, 40))))
        nxt += len(family)
        for _ in range(n_routes):
            keep = family[: int(pick.integers(max(0, len(family) - 3), len(family) + 1))]
            own = int(pick.integers(1, 4))
            page_lists.append(keep + list(range(nxt, nxt + own)))
            nxt += own
            last.append(int(pick.integers(1, ps + 1)))
    pool = nxt + 7
    phys = torch.randperm(pool, generator=gen).tolist()
    indices = [phys[p] for pages in page_lists for p in pages]
    indptr = [0]
    for pages in page_lists:
        indptr.append(indptr[-1] + len(pages))
    batch = len(page_lists)
    kv = torch.randn((pool, 2, ps, hkv, d), generator=gen)
    kv[:, 1] *= 0.1
    q = torch.randn((batch, hq, d), generator=gen)
    kv, q = kv.to(dtype), q.to(dtype)
    w = da.BatchDecodeWithPagedKVCacheWrapper(torch.empty(64 << 20, dtype=torch.uint8, device=dev), "NHD")
    w.split_target_items = [None, None, 64, 1024][int(pick.integers(4))]
    w.plan(torch.tensor(indptr, dtype=torch.int32, device=dev), torch.tensor(indices, dtype=torch.int32, device=dev),
           torch.tensor(last, dtype=torch.int32, device=dev), hq, hkv, d, ps, data_type=dtype, q_data_type=dtype)
    out, lse = w.run(q.to(dev), kv.to(dev), return_lse=True)
    torch.cuda.synchronize()
    ro, rl = oatt.masked_attention(q.double().numpy(), kv.double().numpy(), list(range(batch + 1)), indptr, indices,
                                   last)
    case = f"seed {seed}: hq {hq} hkv {hkv} d {d} ps {ps} {dtype} routes {batch} cascade groups {w.cascade_groups}"
    assert float(np.abs(out.float().cpu().numpy() - ro).max()) <= ATOL, case
    assert float(np.abs(lse.cpu().numpy() - rl).max()) <= ATOL, case


@pytest.mark.parametrize("d,ps,cascade,as_tuple", [(64, 64, True, True), (64, 16, False, False), (128, 64, True, False),
                                                   (128, 16, True, True), (64, 64, False, True)])
def test_hnd_pages_equal_nhd_pages(dev, d, ps, cascade, as_tuple):
    """Decode attention over HND pages ([pages, 2, Hkv, page_size, D], or the
    (K, V) views [pages, Hkv, page_size, D] the Drafter passes) gives the
    bits of the same batch over NHD pages holding the same values: the
    head_dim-64 kernel (page 64 and 16) and the head_dim-128 kernel, cascade
    plans and one item per route, O and LSE; the NHD result is checked
    against the oracle in this file's other tests, and here once more."""
    da = pkg("decode_attention")
    gen = torch.Generator().manual_seed(d * 7 + ps)
    requests, routes, hq, hkv = 3, 4, 8, 2
    pool_pages = requests * (700 // ps + 1) + requests * routes * (90 // ps + 2) + 4
    indptr, indices, last, kv_lens = _routes_batch(gen, requests=requests, routes=routes, prefix_range=(100, 700),
                                                   extra_range=(0, 90), ps=ps, pool_pages=pool_pages)
    batch = requests * routes
    kv = (torch.randn((pool_pages, 2, ps, hkv, d), generator=gen) * 0.5).to(torch.bfloat16)
    q = torch.randn((batch, hq, d), generator=gen).to(torch.bfloat16)
    results = {}
    for layout in ("NHD", "HND"):
        cache = (kv if layout == "NHD" else kv.permute(0, 1, 3, 2, 4)).contiguous().to(dev)
        paged = (cache[:, 0], cache[:, 1]) if as_tuple else cache
        ws = torch.empty(32 * 1024 * 1024, dtype=torch.uint8, device=dev)
        w = da.BatchDecodeWithPagedKVCacheWrapper(ws, layout)
        w.use_cascade = cascade
        w.plan(torch.tensor(indptr, dtype=torch.int32, device=dev), torch.tensor(indices, dtype=torch.int32, device=dev),
               torch.tensor(last, dtype=torch.int32, device=dev), hq, hkv, d, ps, data_type=torch.bfloat16,
               q_data_type=torch.bfloat16)
        out, lse = w.run(q.to(dev), paged, return_lse=True)
        torch.cuda.synchronize()
        results[layout] = (out.cpu(), lse.cpu())
    (on, ln), (oh, lh) = results["NHD"], results["HND"]
    assert torch.equal(on.view(torch.int16), oh.view(torch.int16)) and torch.equal(ln, lh)
    ro, rl = oatt.masked_attention(q.double().numpy(), kv.double().numpy(), list(range(batch + 1)), indptr, indices,
                                   last)
    assert float(np.abs(on.float().numpy() - ro).max()) <= ATOL
    assert float(np.abs(ln.numpy() - rl).max()) <= ATOL
