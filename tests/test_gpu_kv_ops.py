"""KV append / move / commit kernels vs the oracle: bit-exact."""

import math

import numpy as np
import pytest
import torch

from helpers import bits16, pkg
from oracle import paged_kv as ref

pytestmark = pytest.mark.gpu


def _rand(gen, shape, dtype):
    return (torch.randn(shape, generator=gen) * 0.5).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("layers,heads,dim", [(2, 8, 64), (3, 8, 128), (1, 2, 64), (17, 8, 64), (9, 8, 128)])
def test_move_slots_matches_values_dst_eq_src(dev, dtype, layers, heads, dim):
    kv = pkg("kv_ops")
    gen = torch.Generator().manual_seed(1)
    slots = 512
    k_cpu = [_rand(gen, (slots, heads, dim), dtype) for _ in range(layers)]
    v_cpu = [_rand(gen, (slots, heads, dim), dtype) for _ in range(layers)]
    perm = torch.randperm(slots, generator=gen)
    src = perm[:40]
    dst = perm[100:140]
    k_dev = [t.to(dev) for t in k_cpu]
    v_dev = [t.to(dev) for t in v_cpu]
    kv.move_slots(k_dev, v_dev, dst.to(dev), src.to(dev))
    torch.cuda.synchronize()
    k_np = [bits16(t) for t in k_cpu]
    v_np = [bits16(t) for t in v_cpu]
    ref.move_kv(k_np, v_np, dst.tolist(), src.tolist())
    for a, b in zip(k_dev + v_dev, k_np + v_np):
        np.testing.assert_array_equal(bits16(a), b)


def test_move_slots_empty_and_reference_move_list(dev):
    kv = pkg("kv_ops")
    # tests/test_tail_page_cow.py:77-79: one COW move ([40, 41, 42] <- [0, 1, 2]).
    k = torch.arange(512 * 8, dtype=torch.float16).reshape(512, 1, 8).to(dev)
    v = (-torch.arange(512 * 8, dtype=torch.float16)).reshape(512, 1, 8).to(dev)
    kv.move_slots([k], [v], torch.tensor([], dtype=torch.long, device=dev), torch.tensor([], dtype=torch.long, device=dev))
    kv.move_slots([k], [v], torch.tensor([40, 41, 42], device=dev), torch.tensor([0, 1, 2], device=dev))
    torch.cuda.synchronize()
    assert torch.equal(k[40:43].cpu(), k[0:3].cpu())
    assert torch.equal(v[40:43].cpu(), v[0:3].cpu())
    assert torch.equal(k[43].cpu(), torch.arange(43 * 8, 44 * 8, dtype=torch.float16).reshape(1, 8))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_append_paged_write_suffix_matches_oracle(dev, dtype):
    ffv = pkg("flashinfer_full_verify")
    gen = torch.Generator().manual_seed(2)
    pages, ps, h, d = 9, 16, 8, 128
    cache_cpu = _rand(gen, (pages, 2, ps, h, d), dtype)
    key = _rand(gen, (13, h, d), dtype)
    val = _rand(gen, (13, h, d), dtype)
    cache = cache_cpu.to(dev)
    ffv.write_suffix_kv(cache, key_states=key.to(dev), value_states=val.to(dev), prefix_len=101, page_size=ps)
    torch.cuda.synchronize()
    expect = bits16(cache_cpu).copy()
    ref.write_suffix(expect, bits16(key), bits16(val), 101)
    np.testing.assert_array_equal(bits16(cache), expect)


def test_prefix_layer_to_paged_kv_reference_literal(dev):
    # tests/test_target_kv_commit.py:58-73 (float32 literal rows, here fp16).
    ffv = pkg("flashinfer_full_verify")
    key = torch.arange(5, dtype=torch.float16).reshape(1, 1, 5, 1).repeat(1, 1, 1, 8).to(dev)
    value = (100 + torch.arange(5, dtype=torch.float16)).reshape(1, 1, 5, 1).repeat(1, 1, 1, 8).to(dev)
    cache = ffv.prefix_layer_to_paged_kv(key=key, value=value, prefix_len=5, node_count=2, page_size=4)
    torch.cuda.synchronize()
    c = cache.cpu()
    assert c.shape == (2, 2, 4, 1, 8)
    assert [c[p // 4, 0, p % 4, 0, 0].item() for p in range(5)] == [0, 1, 2, 3, 4]
    assert [c[p // 4, 1, p % 4, 0, 0].item() for p in range(5)] == [100, 101, 102, 103, 104]
    assert float(c[1, :, 1:].abs().sum()) == 0.0


@pytest.mark.parametrize("node_ids", [(0, 2), (0, 1, 4, 5), (6, 7, 8, 9), (0, 1, 2, 3)])
@pytest.mark.parametrize("permuted", [False, True])
def test_commit_matches_gather_clone_scatter(dev, node_ids, permuted):
    kv = pkg("kv_ops")
    gen = torch.Generator().manual_seed(3)
    layers, pages, ps, h, d = 4, 12, 16, 8, 128
    cpu = [_rand(gen, (pages, 2, ps, h, d), torch.float16) for _ in range(layers)]
    prefix_len = 150
    indices = torch.randperm(pages, generator=gen).to(torch.int32) if permuted else None
    devs = [t.to(dev) for t in cpu]
    src = [prefix_len + n for n in node_ids]
    dst = list(range(prefix_len, prefix_len + len(node_ids)))
    kv.commit_paged(
        devs, src, dst,
        kv_indptr=None if indices is None else torch.tensor([0, pages], dtype=torch.int32, device=dev),
        kv_indices=None if indices is None else indices.to(dev),
    )
    torch.cuda.synchronize()
    expect = [bits16(t).copy() for t in cpu]
    ref.commit(expect, prefix_len, node_ids, None if indices is None else indices.tolist())
    for a, b in zip(devs, expect):
        np.testing.assert_array_equal(bits16(a), b)


def test_commit_aliasing_uses_staging(dev):
    kv = pkg("kv_ops")
    assert kv.commit_positions_need_staging([10, 12], [9, 10])
    assert not kv.commit_positions_need_staging([10, 12], [10, 11])
    gen = torch.Generator().manual_seed(4)
    cpu = [_rand(gen, (6, 2, 4, 2, 64), torch.float16) for _ in range(3)]
    devs = [t.to(dev) for t in cpu]
    # dst 5 is the source of item 1: a one-pass copy would race.
    src, dst = [7, 5, 9], [4, 5, 6]
    src2, dst2 = [5, 9, 2], [8, 5, 7]
    kv.commit_paged(devs, src2, dst2)
    kv.commit_paged(devs, src, dst)
    torch.cuda.synchronize()
    expect = [bits16(t).copy() for t in cpu]
    for layer in expect:
        for s_list, d_list in ((src2, dst2), (src, dst)):
            rows = [layer[s // 4, :, s % 4].copy() for s in s_list]
            for r, d_ in zip(rows, d_list):
                layer[d_ // 4, :, d_ % 4] = r
    for a, b in zip(devs, expect):
        np.testing.assert_array_equal(bits16(a), b)


def test_batched_commit_device_positions(dev):
    """Several requests with their own page tables in one launch."""
    kv = pkg("kv_ops")
    gen = torch.Generator().manual_seed(5)
    layers, pool, ps, h, d = 3, 64, 16, 8, 64
    cpu = [_rand(gen, (pool, 2, ps, h, d), torch.bfloat16) for _ in range(layers)]
    perm = torch.randperm(pool, generator=gen).to(torch.int32)
    indptr = torch.tensor([0, 20, 41, 64], dtype=torch.int32)
    prefixes = [300, 17, 320]
    nodes = [(0, 2, 5), (1, 3), (0, 1, 2, 3)]
    req, src, dst = [], [], []
    for b, (p, ns) in enumerate(zip(prefixes, nodes)):
        for i, n in enumerate(ns):
            req.append(b)
            src.append(p + n)
            dst.append(p + i)
    devs = [t.to(dev) for t in cpu]
    kv.commit_paged(
        devs, torch.tensor(src, device=dev), torch.tensor(dst, device=dev), kv_indptr=indptr.to(dev),
        kv_indices=perm.to(dev), item_req=torch.tensor(req, dtype=torch.int32, device=dev),
    )
    torch.cuda.synchronize()
    expect = [bits16(t).copy() for t in cpu]
    for b, (p, ns) in enumerate(zip(prefixes, nodes)):
        pt = perm[int(indptr[b]) : int(indptr[b + 1])].tolist()
        ref.commit(expect, p, ns, pt)
    for a, e in zip(devs, expect):
        np.testing.assert_array_equal(bits16(a), e)


@pytest.mark.parametrize("as_tensors", [False, True])
def test_commit_long_route_many_layers(dev, as_tensors):
    """A 200-node route over 6 layers: more items than fit the kernel argument
    block, layers not a multiple of the per-launch layer group, aliasing
    source/destination positions (staged)."""
    kv = pkg("kv_ops")
    gen = torch.Generator().manual_seed(6)
    layers, pages, ps, h, d = 6, 40, 16, 8, 128
    cpu = [_rand(gen, (pages, 2, ps, h, d), torch.bfloat16) for _ in range(layers)]
    perm = torch.randperm(pages, generator=gen).to(torch.int32)
    prefix_len = 130
    node_ids = sorted(torch.randperm(400, generator=gen)[:200].tolist())
    src = [prefix_len + n for n in node_ids]
    dst = list(range(prefix_len, prefix_len + len(node_ids)))
    assert kv.commit_positions_need_staging(src, dst)
    devs = [t.to(dev) for t in cpu]
    s_arg, d_arg = (torch.tensor(src, device=dev), torch.tensor(dst, device=dev)) if as_tensors else (src, dst)
    kv.commit_paged(devs, s_arg, d_arg, kv_indptr=torch.tensor([0, pages], dtype=torch.int32, device=dev),
                    kv_indices=perm.to(dev))
    torch.cuda.synchronize()
    expect = [bits16(t).copy() for t in cpu]
    ref.commit(expect, prefix_len, node_ids, perm.tolist())
    for a, b in zip(devs, expect):
        np.testing.assert_array_equal(bits16(a), b)


def test_commit_disjoint_device_positions_without_staging(dev):
    """Disjoint source and destination sets with staging switched off, over
    several requests, more items than fit the kernel argument block."""
    kv = pkg("kv_ops")
    gen = torch.Generator().manual_seed(7)
    layers, pages, ps, h, d = 5, 48, 16, 4, 64
    cpu = [_rand(gen, (pages, 2, ps, h, d), torch.float16) for _ in range(layers)]
    perm = torch.randperm(pages, generator=gen).to(torch.int32)
    indptr = [0, 16, 32, 48]
    req, src, dst = [], [], []
    for b in range(3):
        for i in range(40):
            req.append(b)
            src.append(128 + 3 * i)      # positions 128..245 of request b
            dst.append(2 * i)            # positions 0..78
    assert not kv.commit_positions_need_staging(src, dst, req)
    devs = [t.to(dev) for t in cpu]
    kv.commit_paged(devs, torch.tensor(src, device=dev), torch.tensor(dst, device=dev),
                    kv_indptr=torch.tensor(indptr, dtype=torch.int32, device=dev), kv_indices=perm.to(dev),
                    item_req=torch.tensor(req, dtype=torch.int32, device=dev), needs_staging=False)
    torch.cuda.synchronize()
    expect = [bits16(t).copy() for t in cpu]
    for layer in expect:
        for r, s, t in zip(req, src, dst):
            pt = perm[indptr[r]: indptr[r + 1]].tolist()
            layer[pt[t // ps], :, t % ps] = layer[pt[s // ps], :, s % ps]
    for a, b in zip(devs, expect):
        np.testing.assert_array_equal(bits16(a), b)


def test_append_token_pool_set_kv_buffer(dev):
    kv = pkg("kv_ops")
    gen = torch.Generator().manual_seed(6)
    layers, slots, h, d = 4, 256, 8, 64
    k_cpu = [_rand(gen, (slots, h, d), torch.float16) for _ in range(layers)]
    v_cpu = [_rand(gen, (slots, h, d), torch.float16) for _ in range(layers)]
    rows_k = [_rand(gen, (9, h, d), torch.float16) for _ in range(layers)]
    rows_v = [_rand(gen, (9, h, d), torch.float16) for _ in range(layers)]
    loc = torch.randperm(slots, generator=gen)[:9]
    k_dev = [t.to(dev) for t in k_cpu]
    v_dev = [t.to(dev) for t in v_cpu]
    kv.append_token_pool(k_dev, v_dev, [t.to(dev) for t in rows_k], [t.to(dev) for t in rows_v], loc.to(dev))
    torch.cuda.synchronize()
    k_np = [bits16(t).copy() for t in k_cpu]
    v_np = [bits16(t).copy() for t in v_cpu]
    ref.set_kv(k_np, v_np, loc.tolist(), [bits16(t) for t in rows_k], [bits16(t) for t in rows_v])
    for a, b in zip(k_dev + v_dev, k_np + v_np):
        np.testing.assert_array_equal(bits16(a), b)


def test_kv_ops_reject_cpu_tensors():
    kv = pkg("kv_ops")
    k = torch.zeros(4, 1, 8, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="HIP device"):
        kv.move_slots([k], [k], torch.tensor([1]), torch.tensor([0]))


def test_kv_kernels_graph_replays_match_eager(dev):
    """A batched commit without staging (device positions, several
    requests), an aliasing commit through the staging workspace and a
    copy-on-write move, captured in one HIP graph and replayed several times
    from the same starting pools, with eager work and synchronisations in
    between: every replay leaves the pools bit-equal to the eager run."""
    kv = pkg("kv_ops")
    gen = torch.Generator().manual_seed(17)
    layers, pages, ps, h, d = 4, 48, 16, 8, 64
    pools = [_rand(gen, (pages, 2, ps, h, d), torch.bfloat16).to(dev) for _ in range(layers)]
    perm = torch.randperm(pages, generator=gen).to(torch.int32).to(dev)
    indptr = torch.tensor([0, 16, 32, 48], dtype=torch.int32, device=dev)
    req, src, dst = [], [], []
    for b in range(3):
        for i in range(4):
            req.append(b)
            src.append(200 + 3 * i)
            dst.append(190 + i)
    req_t = torch.tensor(req, dtype=torch.int32, device=dev)
    src_t, dst_t = torch.tensor(src, device=dev), torch.tensor(dst, device=dev)
    alias_src, alias_dst = torch.tensor([5, 6, 7], device=dev), torch.tensor([6, 7, 8], device=dev)  # overlapping
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=dev)
    tok_k = [_rand(gen, (512, h, d), torch.bfloat16).to(dev) for _ in range(layers)]
    tok_v = [_rand(gen, (512, h, d), torch.bfloat16).to(dev) for _ in range(layers)]
    cow_src, cow_dst = torch.arange(0, 40, device=dev), torch.arange(100, 140, device=dev)

    def work():
        kv.commit_paged(pools, src_t, dst_t, kv_indptr=indptr, kv_indices=perm, item_req=req_t, needs_staging=False)
        kv.commit_paged(pools, alias_src, alias_dst, kv_indptr=indptr[:2], kv_indices=perm, workspace=ws,
                        needs_staging=True)
        kv.move_slots(tok_k, tok_v, cow_dst, cow_src)

    start = [t.clone() for t in pools + tok_k + tok_v]

    def restore():
        for t, s in zip(pools + tok_k + tok_v, start):
            t.copy_(s)

    work()
    torch.cuda.synchronize()
    eager = [t.clone() for t in pools + tok_k + tok_v]
    assert not all(torch.equal(a, b) for a, b in zip(eager, start))
    restore()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        work()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        work()
    for rep in range(4):
        restore()
        scratch = torch.randn(1 << 20, device=dev).sum()  # unrelated eager work
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert float(scratch) == float(scratch)
        for a, e in zip(pools + tok_k + tok_v, eager):
            assert torch.equal(a, e), f"replay {rep} differs from the eager run"


@pytest.mark.parametrize("seed", range(8))
def test_random_commits_match_gather_then_scatter(dev, seed):
    """Seeded random commits: 1-5 layers, pages of 1, 16 or 64 tokens, 1-4
    requests with their own scattered page tables, 1-70 items with distinct
    destinations whose sources may overlap them (the staging decision is the
    library's own for host lists), given as host lists or device tensors.
    Every layer equals the reference's gather-clone-scatter bit for bit."""
    kv = pkg("kv_ops")
    pick = np.random.default_rng(500 + seed)
    gen = torch.Generator().manual_seed(seed)
    layers = int(pick.integers(1, 6))
    ps = int(pick.choice([1, 16, 64]))
    h, d = [(8, 64), (8, 128), (2, 64)][int(pick.integers(3))]
    nreq = int(pick.integers(1, 5))
    lens = [int(pick.integers(8, 400)) for _ in range(nreq)]
    pages_per = [math.ceil(n / ps) for n in lens]
    pool = sum(pages_per) + 5
    perm = torch.randperm(pool, generator=gen)[: sum(pages_per)].to(torch.int32)
    indptr = [0]
    for p in pages_per:
        indptr.append(indptr[-1] + p)
    req, src, dst = [], [], []
    for b, n in enumerate(lens):
        k = int(pick.integers(0, min(n, 20) + 1))
        dsts = pick.choice(n, size=k, replace=False)
        for t in dsts:
            req.append(b)
            src.append(int(pick.integers(0, n)))
            dst.append(int(t))
    if not req:
        req, src, dst = [0], [0], [min(1, lens[0] - 1)]
    cpu = [_rand(gen, (pool, 2, ps, h, d), torch.float16) for _ in range(layers)]
    devs = [t.to(dev) for t in cpu]
    as_tensors = bool(pick.integers(2))
    args = (torch.tensor(src, device=dev), torch.tensor(dst, device=dev)) if as_tensors else (src, dst)
    item_req = torch.tensor(req, dtype=torch.int32, device=dev) if as_tensors else req
    kv.commit_paged(devs, *args, kv_indptr=torch.tensor(indptr, dtype=torch.int32, device=dev),
                    kv_indices=perm.to(dev), item_req=item_req)
    torch.cuda.synchronize()
    expect = [bits16(t).copy() for t in cpu]
    for layer in expect:
        rows = []
        for r, s in zip(req, src):  # gather every source first (clone), then scatter
            pt = perm[indptr[r]: indptr[r + 1]].tolist()
            rows.append(layer[pt[s // ps], :, s % ps].copy())
        for r, t, row in zip(req, dst, rows):
            pt = perm[indptr[r]: indptr[r + 1]].tolist()
            layer[pt[t // ps], :, t % ps] = row
    case = f"seed {seed}: layers {layers} ps {ps} h {h} d {d} requests {nreq} items {len(req)} tensors {as_tensors}"
    for a, e in zip(devs, expect):
        np.testing.assert_array_equal(bits16(a), e, err_msg=case)


def test_host_staging_ring_keeps_every_pending_upload(dev):
    """Uploads through a small pinned ring (four 1 KiB quarters) that wraps
    many times while its copies are still queued behind device work: every
    upload arrives intact (a quarter is rewritten only after the copies out
    of it ran), also when the stream changes between uploads."""
    lib = pkg("_lib")
    ring = lib.HostStaging(4096)
    rng = np.random.default_rng(5)
    side = torch.cuda.Stream()
    sent, got = [], []
    for i in range(300):
        if i % 50 == 0:
            # keep the device busy so copies stay queued while the host runs ahead
            big = torch.randn((2048, 2048), device=dev)
            big @ big
        n = int(rng.integers(1, 1000))
        host = rng.integers(0, 256, size=n, dtype=np.uint8)
        sent.append(host)
        if i % 7 == 3:
            with torch.cuda.stream(side):
                got.append(ring.upload(host, dev))
        elif i % 5 == 1:
            # into a caller's buffer (a slice of a larger tensor)
            out = torch.empty(n + 16, dtype=torch.uint8, device=dev)[8 : 8 + n]
            got.append(ring.upload(host, dev, out=out))
            assert got[-1] is out
        else:
            got.append(ring.upload(host, dev))
    torch.cuda.synchronize()
    for h, d in zip(sent, got):
        assert np.array_equal(d.cpu().numpy(), h)
    vals = [int(x) for x in rng.integers(-2**62, 2**62, size=33)]
    assert lib.upload_i64(vals, dev).cpu().tolist() == vals


@pytest.mark.parametrize("heads,dim,staged,as_tensors", [(8, 128, False, False), (8, 64, False, True),
                                                        (2, 128, True, False), (8, 128, True, True),
                                                        (1, 64, False, False)])
def test_hnd_append_and_commit_match_nhd(dev, heads, dim, staged, as_tensors):
    """HND pages [pages, 2, Hkv, ps, D] (a token's row split by KV head):
    append_paged at positions and at slots, and commit_paged (in place,
    staged through the workspace, host-list and device-tensor positions)
    leave the same values, read back as NHD, as the same calls on NHD pages,
    which match the oracle elsewhere in this file (2 KiB, 1 KiB and 256-byte
    rows: both one-wave row paths and the vector loop)."""
    kv = pkg("kv_ops")
    gen = torch.Generator().manual_seed(heads * dim + staged)
    layers, pages, ps = 3, 10, 16
    nhd = [_rand(gen, (pages, 2, ps, heads, dim), torch.float16) for _ in range(layers)]
    k_new = [_rand(gen, (5, heads, dim), torch.float16) for _ in range(layers)]
    v_new = [_rand(gen, (5, heads, dim), torch.float16) for _ in range(layers)]
    indices = torch.randperm(pages, generator=gen).to(torch.int32)
    slots = torch.tensor([int(indices[p // ps]) * ps + p % ps for p in (40, 41, 57, 58, 100)], dtype=torch.int64)
    if staged:
        src, dst = [100, 90, 120, 95], [90, 95, 101, 102]  # dst 90 and 95 are sources of other items
    else:
        src, dst = [100, 103, 120, 95], [90, 91, 92, 93]
    results = []
    for layout in ("NHD", "HND"):
        caches = [(t if layout == "NHD" else t.permute(0, 1, 3, 2, 4)).contiguous().to(dev) for t in nhd]
        kv.append_paged(caches, [x.to(dev) for x in k_new], [x.to(dev) for x in v_new], start_pos=3,
                        kv_layout=layout)
        kv.append_paged(caches, [x.to(dev) for x in k_new], [x.to(dev) for x in v_new], dst_slots=slots.to(dev),
                        kv_layout=layout)
        pos = (torch.tensor(src, device=dev), torch.tensor(dst, device=dev)) if as_tensors else (src, dst)
        kv.commit_paged(caches, *pos, kv_indptr=torch.tensor([0, pages], dtype=torch.int32, device=dev),
                        kv_indices=indices.to(dev), kv_layout=layout)
        torch.cuda.synchronize()
        results.append([(c if layout == "NHD" else c.permute(0, 1, 3, 2, 4)).cpu().contiguous() for c in caches])
    for a, b in zip(*results):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    # the calls changed the cache (the comparison is not vacuous)
    assert not torch.equal(results[0][0].view(torch.int16), nhd[0].view(torch.int16))


def test_hnd_layout_geometry_and_refusals(dev):
    """HND geometry: token stride D, head stride page_size * D; a layout name
    outside NHD / HND is refused."""
    kv = pkg("kv_ops")
    hnd = torch.zeros((4, 2, 8, 16, 128), dtype=torch.float16, device=dev)
    geom, v_off = kv.paged_layer_geometry(hnd, "HND")
    assert (geom.page_size, geom.token_stride, geom.head_stride, geom.head_bytes, geom.row_bytes) == \
        (16, 256, 16 * 256, 256, 8 * 256)
    assert v_off == 8 * 16 * 256 and geom.page_stride == 2 * v_off
    nhd_geom, _ = kv.paged_layer_geometry(torch.zeros((4, 2, 16, 8, 128), dtype=torch.float16, device=dev))
    assert nhd_geom.token_stride == 8 * 256 and nhd_geom.head_stride == 256
    with pytest.raises(ValueError, match="kv_layout"):
        kv.paged_layer_geometry(hnd, "NDH")
