"""Prune / ownership / allocator-slot / paged-metadata kernels vs the oracle
(bit-exact integer results)."""

import itertools

import numpy as np
import pytest
import torch

from helpers import pkg
from oracle import paged_kv as ref

pytestmark = pytest.mark.gpu


def _lib():
    return pkg("_lib")


def _bitmap(pages_set, num_pages, dev):
    words = np.zeros((num_pages + 31) // 32, dtype=np.uint32)
    for p in pages_set:
        words[p >> 5] |= np.uint32(1 << (p & 31))
    return torch.from_numpy(words.view(np.int32)).to(dev)


def _set_from_bitmap(bm):
    w = bm.cpu().numpy().view(np.uint32)
    return {i * 32 + b for i, x in enumerate(w) for b in range(32) if (int(x) >> b) & 1}


def _prune(dev, owned, live_slots, num_pages, ps):
    lib = _lib()
    owned_bm = _bitmap(owned, num_pages, dev)
    live_bm = torch.zeros_like(owned_bm)
    free = torch.full((num_pages,), -1, dtype=torch.int64, device=dev)
    cnt = torch.zeros(1, dtype=torch.int64, device=dev)
    slots = torch.tensor(live_slots, dtype=torch.int64, device=dev)
    rc = lib.load().atlas_prune_pages(lib.ptr(owned_bm), lib.ptr(live_bm), num_pages, lib.ptr(slots),
                                      len(live_slots), ps, lib.ptr(free), lib.ptr(cnt), lib.stream_of(dev))
    lib.check(rc, "prune")
    torch.cuda.synchronize()
    n = int(cnt.item())
    return free[:n].cpu().tolist(), _set_from_bitmap(owned_bm)


def test_prune_reference_literal(dev):
    # tests/test_tail_page_cow.py:241-277 -> freed page 11 (slot 44), owned {0, 10}
    prefix = [0, 1, 40]
    route = [0, 1, 40, 41]
    sampled = prefix[::4] + route[::4] + route[-1:]
    freed, owned = _prune(dev, {0, 10, 11}, sampled, 64, 4)
    assert freed == [11] and owned == {0, 10}
    assert [p * 4 for p in freed] == [44]


@pytest.mark.parametrize("num_pages", [1, 31, 32, 33, 4096, 95367])
def test_prune_random_matches_oracle(dev, num_pages):
    rng = np.random.default_rng(num_pages)
    ps = 16
    owned = set(rng.choice(num_pages, size=min(num_pages, 3000), replace=False).tolist())
    paths = []
    for _ in range(9):
        pages = rng.choice(num_pages, size=min(num_pages, 8), replace=False)
        length = int(rng.integers(1, len(pages) * ps + 1))
        paths.append([int(pages[i // ps]) * ps + i % ps for i in range(length)])
    sampled = [s for p in paths for s in (p[::ps] + p[-1:])]
    freed, left = _prune(dev, owned, sampled, num_pages, ps)
    exp_freed, exp_left = ref.prune(owned, None, paths, ps)
    assert freed == exp_freed and left == exp_left


@pytest.mark.parametrize("num_pages,n_slots,ps", [
    (524288, 3000, 16),   # one workgroup: the largest bitmap kept in LDS
    (4096, 4096, 16),     # one workgroup: the most slots it takes
    (4096, 4000, 24),     # one workgroup, page size not a power of two
    (524289, 3000, 16),   # clear + mark + sweep launches: bitmap too large for LDS
    (4096, 4097, 16),     # the same launches: more slots than one workgroup takes
])
def test_prune_fused_and_multi_launch_paths(dev, num_pages, n_slots, ps):
    """Both prune paths give releasable = sorted(owned - live), owned &= live
    (sglang_runtime.py:507-539) and leave the live bitmap set; slots that are
    negative or past the pool are ignored."""
    lib = _lib()
    rng = np.random.default_rng(num_pages + n_slots + ps)
    owned = set(rng.choice(num_pages, size=min(num_pages, 20000), replace=False).tolist())
    slots = rng.integers(-ps, (num_pages + 8) * ps, size=n_slots)
    slots[::97] = -1
    live = {int(x) // ps for x in slots if 0 <= x < num_pages * ps}
    owned_bm = _bitmap(owned, num_pages, dev)
    live_bm = torch.full_like(owned_bm, -1)
    free = torch.full((num_pages,), -1, dtype=torch.int64, device=dev)
    cnt = torch.zeros(1, dtype=torch.int64, device=dev)
    slots_t = torch.tensor(slots, dtype=torch.int64, device=dev)
    rc = lib.load().atlas_prune_pages(lib.ptr(owned_bm), lib.ptr(live_bm), num_pages, lib.ptr(slots_t),
                                      n_slots, ps, lib.ptr(free), lib.ptr(cnt), lib.stream_of(dev))
    lib.check(rc, "prune")
    torch.cuda.synchronize()
    n = int(cnt.item())
    assert free[:n].cpu().tolist() == sorted(owned - live)
    assert _set_from_bitmap(owned_bm) == owned & live
    assert _set_from_bitmap(live_bm) == live


@pytest.mark.parametrize("read_back", [False, True])
@pytest.mark.parametrize("num_pages,num_paths,ps", [(4096, 10, 16), (95367, 64, 64), (524288, 3, 16),
                                                      (3000, 7, 24), (64, 1, 4)])
def test_prune_by_paths_matches_oracle_and_sample_list(dev, num_pages, num_paths, ps, read_back):
    """atlas_prune_pages_paths samples each path's page-start slots (and, for
    paths with their bit in the mask, the last slot) inside the launch: the
    released pages, the owned bitmap and the live bitmap equal the oracle's
    prune of the same paths and atlas_prune_pages over the sample list
    (sglang_runtime.py:507-539).  Empty paths and a prefix without its last
    slot are included.  ``read_back``: atlas_prune_pages_paths_gather, the
    same prune whose launch then copies its own released-page count and the
    page starts of path 0 to mapped host memory."""
    lib = _lib()
    rng = np.random.default_rng(num_pages * 7 + num_paths)
    owned = set(rng.choice(num_pages, size=min(num_pages, 5000), replace=False).tolist())
    paths, last = [], []
    for i in range(num_paths):
        pages = rng.choice(num_pages, size=min(num_pages, 40), replace=False)
        length = 0 if i == 1 else int(rng.integers(1, len(pages) * ps + 1))
        paths.append([int(pages[j // ps]) * ps + j % ps for j in range(length)])
        last.append(i != 0)  # path 0 plays the prefix: page starts only
    sampled = [s for p, l in zip(paths, last) for s in (p[::ps] + (p[-1:] if l else []))]
    exp_freed, exp_left = _prune(dev, owned, sampled, num_pages, ps)
    ref_freed, ref_left = ref.prune(owned, paths[0] or None, [p for p in paths[1:] if p], ps)
    assert (exp_freed, exp_left) == (ref_freed, ref_left)

    owned_bm = _bitmap(owned, num_pages, dev)
    live_bm = torch.full_like(owned_bm, -1)
    free = torch.full((num_pages,), -1, dtype=torch.int64, device=dev)
    cnt = torch.zeros(1, dtype=torch.int64, device=dev)
    tensors = [torch.tensor(p, dtype=torch.int64, device=dev) for p in paths]
    arr = (lib.SlotPath * num_paths)()
    mask = 0
    for i, t in enumerate(tensors):
        arr[i].slots, arr[i].len = (t.data_ptr() if t.numel() else None), t.numel()
        mask |= (1 << i) if last[i] else 0
    print(f"prune by paths: {num_pages} pages, {num_paths} paths, page {ps}, read_back={read_back}", flush=True)
    if read_back:
        starts = tensors[0][::ps]
        segs = (lib.I64Segment * 2)()
        for i, t in enumerate((cnt, starts)):
            segs[i].src, segs[i].count, segs[i].stride = t.data_ptr(), t.numel(), t.stride(0)
        mapped = lib.MappedReadback(2 * (1 + starts.numel() + 4))
        vals = mapped.np.view(np.int64)
        vals[:] = -9
        rc = lib.load().atlas_prune_pages_paths_gather(lib.ptr(owned_bm), lib.ptr(live_bm), num_pages, arr,
                                                       num_paths, mask, ps, lib.ptr(free), lib.ptr(cnt), segs, 2,
                                                       mapped.device_ptr, lib.stream_of(dev))
    else:
        rc = lib.load().atlas_prune_pages_paths(lib.ptr(owned_bm), lib.ptr(live_bm), num_pages, arr, num_paths,
                                                mask, ps, lib.ptr(free), lib.ptr(cnt), lib.stream_of(dev))
    lib.check(rc, "prune by paths")
    torch.cuda.synchronize()
    n = int(cnt.item())
    if read_back:
        # the launch's own count, then path 0's page starts, nothing after them
        k = int(starts.numel())
        assert vals[0] == n == len(exp_freed)
        assert vals[1:1 + k].tolist() == paths[0][::ps] and vals[1 + k:].tolist() == [-9] * 4
    assert free[:n].cpu().tolist() == exp_freed
    assert _set_from_bitmap(owned_bm) == exp_left
    assert _set_from_bitmap(live_bm) == {s // ps for s in sampled}


def test_prune_empty_live_frees_everything_ascending(dev):
    owned = {5, 3, 900, 64, 31, 32}
    freed, left = _prune(dev, owned, [], 1000, 16)
    assert freed == sorted(owned) and left == set()


def test_mark_pages(dev):
    lib = _lib()
    bm = torch.zeros(4, dtype=torch.int32, device=dev)
    slots = torch.tensor([0, 17, 18, 127, 64, -1, 5000], dtype=torch.int64, device=dev)
    rc = lib.load().atlas_mark_pages(lib.ptr(bm), 120, lib.ptr(slots), 7, 16, lib.stream_of(dev))
    lib.check(rc, "mark")
    torch.cuda.synchronize()
    # slot -> page: 0, 1, 1, 7, 4; -1 and page 312 (>= 120) are ignored
    assert _set_from_bitmap(bm) == {0, 1, 4, 7}


def test_alloc_decode_and_extend_match_allocator_policy(dev):
    lib = _lib()
    ps = 16
    rng = np.random.default_rng(7)
    free_pages = [int(x) for x in rng.permutation(np.arange(1, 200))]
    alloc = ref.PagedAllocator(num_pages=199, page_size=ps)
    alloc.free_pages = list(free_pages)
    seq = [int(x) for x in rng.integers(1, 300, size=70)]
    last = [int(x) for x in rng.integers(0, 4000, size=70)]
    expect = alloc.alloc_decode(seq, last)
    fp = torch.tensor(free_pages, dtype=torch.int64, device=dev)
    out = torch.empty(70, dtype=torch.int64, device=dev)
    # Keep every argument tensor referenced until the launch is enqueued: a
    # temporary freed earlier can be handed to the next upload.
    seq_t = torch.tensor(seq, device=dev)
    last_t = torch.tensor(last, device=dev)
    rc = lib.load().atlas_alloc_decode_slots(lib.ptr(seq_t), lib.ptr(last_t), lib.ptr(fp), ps, 70, lib.ptr(out),
                                             lib.stream_of(dev))
    lib.check(rc, "alloc_decode")
    torch.cuda.synchronize()
    assert out.cpu().tolist() == expect
    # extend
    alloc2 = ref.PagedAllocator(num_pages=199, page_size=ps)
    alloc2.free_pages = list(free_pages)
    pre = [int(x) for x in rng.integers(0, 100, size=9)]
    seqe = [p + int(x) for p, x in zip(pre, rng.integers(1, 70, size=9))]
    laste = [int(rng.integers(1, 100)) * ps + (p - 1) % ps if p else -1 for p in pre]
    expect = alloc2.alloc_extend(pre, seqe, laste)
    n = sum(s - p for p, s in zip(pre, seqe))
    out = torch.empty(n, dtype=torch.int64, device=dev)
    pre_t = torch.tensor(pre, device=dev)
    seqe_t = torch.tensor(seqe, device=dev)
    laste_t = torch.tensor(laste, device=dev)
    rc = lib.load().atlas_alloc_extend_slots(lib.ptr(pre_t), lib.ptr(seqe_t), lib.ptr(laste_t), lib.ptr(fp), ps, 9,
                                             lib.ptr(out), lib.stream_of(dev))
    lib.check(rc, "alloc_extend")
    torch.cuda.synchronize()
    assert out.cpu().tolist() == expect


def _slot_path(page_ids, length, page_size=16):
    return [p * page_size + o for p in page_ids for o in range(page_size)][:length]


def test_paged_metadata_reference_literals(dev):
    # tests/test_paged_attention_metadata.py:24-52
    pm = pkg("flashinfer_paged.paged_metadata")
    lengths = [1, 15, 16, 17, 31, 32]
    paths = [torch.tensor(_slot_path([11 + 3 * i, 31 + 5 * i], n), device=dev) for i, n in enumerate(lengths)]
    md = pm.build_flashinfer_paged_kv_metadata(paths, page_size=16)
    counts = [(n + 15) // 16 for n in lengths]
    assert md.kv_indptr.tolist() == list(itertools.accumulate([0] + counts))
    assert md.kv_last_page_len.tolist() == [1, 15, 16, 1, 15, 16]
    assert md.seq_lens.tolist() == lengths
    assert md.token_index_count == sum(lengths) and md.page_index_count == sum(counts)
    assert md.layout_validated
    md.assert_layout_valid()
    exp = ref.paged_metadata([p.tolist() for p in paths], 16)
    assert md.kv_page_indices.tolist() == exp.kv_page_indices
    long = torch.tensor(_slot_path(list(range(100, 612)), 8192), device=dev)
    md = pm.build_flashinfer_paged_kv_metadata([long], page_size=16, sync_check=True)
    assert md.token_index_count == 8192 and md.page_index_count == 512
    assert md.kv_indptr.tolist() == [0, 512] and md.kv_last_page_len.tolist() == [16]


@pytest.mark.parametrize("bad", [[161, 162, 163], [160, 161, 165], list(range(160, 176)) + [193]])
def test_paged_metadata_invalid_layout_raises_on_check(dev, bad):
    # tests/test_paged_attention_metadata.py:55-67 (raised on the host, no device assert)
    pm = pkg("flashinfer_paged.paged_metadata")
    md = pm.build_flashinfer_paged_kv_metadata([torch.tensor(bad, device=dev)], page_size=16)
    with pytest.raises(RuntimeError, match="page-aligned"):
        md.assert_layout_valid()
    with pytest.raises(RuntimeError):
        pm.build_flashinfer_paged_kv_metadata([torch.tensor(bad, device=dev)], page_size=16, sync_check=True)


def test_paged_metadata_random_paths_match_oracle(dev):
    pm = pkg("flashinfer_paged.paged_metadata")
    rng = np.random.default_rng(9)
    for ps in (1, 4, 16, 64):
        paths = []
        for _ in range(72):
            pages = rng.choice(5000, size=6, replace=False)
            length = int(rng.integers(1, 6 * ps + 1))
            paths.append(_slot_path([int(x) for x in pages], length, ps))
        md = pm.build_flashinfer_paged_kv_metadata([torch.tensor(p, device=dev) for p in paths], page_size=ps,
                                                   sync_check=True)
        exp = ref.paged_metadata(paths, ps)
        assert md.kv_page_indices.tolist() == exp.kv_page_indices
        assert md.kv_indptr.tolist() == exp.kv_indptr
        assert md.kv_last_page_len.tolist() == exp.kv_last_page_len
        assert md.seq_lens.tolist() == exp.seq_lens


def test_paged_metadata_argument_errors(dev):
    pm = pkg("flashinfer_paged.paged_metadata")
    with pytest.raises(ValueError):
        pm.build_flashinfer_paged_kv_metadata([torch.tensor([0], device=dev)], page_size=0)
    with pytest.raises(ValueError):
        pm.build_flashinfer_paged_kv_metadata([], page_size=16)
    with pytest.raises(TypeError):
        pm.build_flashinfer_paged_kv_metadata([torch.tensor([0.0], device=dev)], page_size=16)
    with pytest.raises(ValueError):
        pm.build_flashinfer_paged_kv_metadata([torch.zeros(0, dtype=torch.long, device=dev)], page_size=16)


@pytest.mark.parametrize("num_pages,n_slots", [(4096, 900), (524289, 3000)])
def test_mark_and_prune_graph_replays(dev, num_pages, n_slots):
    """Ownership marks and a prune (one workgroup, or the clear + mark + sweep
    launches of a pool too large for LDS) captured in one HIP graph and
    replayed from the same starting bitmaps, with eager work in between:
    every replay gives the eager run's owned bitmap, free list and count,
    which equal the oracle's."""
    lib = _lib()
    rng = np.random.default_rng(num_pages + 1)
    ps = 16
    owned0 = set(rng.choice(num_pages, size=min(num_pages // 2, 5000), replace=False).tolist())
    new_pages = rng.choice(num_pages, size=64, replace=False).tolist()
    owned_bm = _bitmap(owned0, num_pages, dev)
    start = owned_bm.clone()
    live_bm = torch.zeros_like(owned_bm)
    free = torch.full((num_pages,), -1, dtype=torch.int64, device=dev)
    cnt = torch.zeros(1, dtype=torch.int64, device=dev)
    marks = torch.tensor([p * ps + 3 for p in new_pages], dtype=torch.int64, device=dev)
    live = torch.tensor(rng.integers(0, num_pages * ps, size=n_slots).tolist(), dtype=torch.int64, device=dev)
    L = lib.load()

    def work():
        lib.check(L.atlas_mark_pages(lib.ptr(owned_bm), num_pages, lib.ptr(marks), int(marks.numel()), ps,
                                     lib.stream_of(dev)), "mark")
        lib.check(L.atlas_prune_pages(lib.ptr(owned_bm), lib.ptr(live_bm), num_pages, lib.ptr(live), n_slots, ps,
                                      lib.ptr(free), lib.ptr(cnt), lib.stream_of(dev)), "prune")

    work()
    torch.cuda.synchronize()
    n = int(cnt.item())
    eager = (owned_bm.clone(), free[:n].clone(), n)
    exp_freed, exp_left = ref.prune(owned0 | set(new_pages), None,
                                    [[int(s)] for s in live.cpu().tolist()], ps)
    assert free[:n].cpu().tolist() == exp_freed and _set_from_bitmap(owned_bm) == exp_left
    owned_bm.copy_(start)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        work()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        work()
    for rep in range(4):
        owned_bm.copy_(start)
        free.fill_(-1)
        cnt.zero_()
        scratch = torch.randn(1 << 20, device=dev).sum()  # unrelated eager work
        graph.replay()
        torch.cuda.synchronize()
        assert float(scratch) == float(scratch)
        assert int(cnt.item()) == eager[2], f"replay {rep}: count differs"
        assert torch.equal(owned_bm, eager[0]) and torch.equal(free[: eager[2]], eager[1]), f"replay {rep} differs"


@pytest.mark.parametrize("target", ["mapped", "device"])
def test_gather_i64_segments(dev, target):
    """atlas_gather_i64: contiguous, strided, single-value and empty
    segments concatenated in order, into mapped host memory and into device
    memory; nothing past the values is written."""
    import numpy as np

    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    a = torch.arange(100, 140, dtype=torch.int64, device=dev)
    b = torch.arange(-500, 0, dtype=torch.int64, device=dev)[::7]  # strided view
    c = torch.tensor([1 << 40], dtype=torch.int64, device=dev)
    e = a[:0]
    parts = [a, e, b, c, a[5:9]]
    want = np.concatenate([p.cpu().numpy() for p in parts]).tolist()
    segs = (lib_mod.I64Segment * len(parts))()
    for i, t in enumerate(parts):
        segs[i].src, segs[i].count, segs[i].stride = t.data_ptr(), t.numel(), t.stride(0)
    print(f"gather_i64 into {target}: {len(want)} values", flush=True)
    if target == "mapped":
        buf = lib_mod.MappedReadback(2 * (len(want) + 8))
        vals = buf.np.view(np.int64)
        vals[:] = -7
        out = buf.device_ptr
    else:
        dst = torch.full((len(want) + 8,), -7, dtype=torch.int64, device=dev)
        out = dst.data_ptr()
    lib_mod.check(lib.atlas_gather_i64(segs, len(parts), out, lib_mod.stream_of(dev)), "atlas_gather_i64")
    torch.cuda.synchronize()
    got = vals.tolist() if target == "mapped" else dst.tolist()
    assert got[: len(want)] == want and got[len(want):] == [-7] * 8
