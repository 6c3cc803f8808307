"""Host-side tree construction of the product (trie, TreeSpec, bitmasks, plan
helpers) against the reference literals and the oracle.  CPU only."""

import numpy as np
import pytest
import torch

from helpers import pkg
from oracle import paged_kv as ref


def test_dedup_literals():
    # tests/test_tree_dedup.py:6-35
    ffv = pkg("flashinfer_full_verify")
    tokens, parents, depths, routes = ffv.build_deduplicated_path_tree_tokens(
        [(10, 20, 30, 40), (10, 20, 31, 41), (11, 21, 32, 42)], device="cpu"
    )
    assert tokens.tolist() == [10, 20, 30, 40, 31, 41, 11, 21, 32, 42]
    assert parents == [-1, 0, 1, 2, 1, 4, -1, 6, 7, 8]
    assert depths.tolist() == [0, 1, 2, 3, 2, 3, 0, 1, 2, 3]
    assert routes == [[0, 1, 2, 3], [0, 1, 4, 5], [6, 7, 8, 9]]
    tokens, parents, depths, routes = ffv.build_deduplicated_path_tree_tokens([(7, 8), (7, 8)], device="cpu")
    assert tokens.tolist() == [7, 8] and parents == [-1, 0] and routes == [[0, 1], [0, 1]]


@pytest.mark.parametrize("bad", [[], [(1, 2), (3,)], [()]])
def test_dedup_rejects_bad_paths(bad):
    ffv = pkg("flashinfer_full_verify")
    with pytest.raises(ValueError):
        ffv.build_deduplicated_path_tree_tokens(bad, device="cpu")


def test_tree_spec_matches_oracle_mask_and_metadata():
    ffv = pkg("flashinfer_full_verify")
    rng = np.random.default_rng(0)
    for trial in range(20):
        k = int(rng.integers(1, 10))
        depth = int(rng.integers(1, 5))
        paths = [tuple(int(x) for x in rng.integers(0, 3, size=depth)) for _ in range(k)]
        prefix = int(rng.integers(0, 70))
        spec, routes = ffv.build_deduplicated_tree_spec_from_paths(paths=paths, prefix_len=prefix, page_size=16,
                                                                   device="cpu")
        tokens, parents, _, oroutes = ref.dedup_tree(paths)
        mask = ref.ancestor_mask(parents, prefix)
        assert routes == oroutes
        assert spec.bool_mask.numpy().tolist() == mask.reshape(-1).tolist()
        assert spec.packed_mask.numpy().tolist() == ref.packbits(mask).tolist()
        n = len(tokens)
        assert spec.kv_len == prefix + n and spec.node_count == n
        assert spec.total_pages == (prefix + n + 15) // 16
        assert spec.kv_last_page_len.tolist() == [ffv.last_page_len(prefix + n, 16)]
        assert spec.kv_indices.tolist() == list(range(spec.total_pages))
        # compact bitmask agrees with the dense mask's tree columns
        bits = spec.tree_mask.numpy().astype(np.uint64)
        for i in range(n):
            row = [(int(bits[i]) >> j) & 1 for j in range(n)]
            assert row == mask[i, prefix:].astype(int).tolist()


def test_undeduplicated_tree_spec():
    ffv = pkg("flashinfer_full_verify")
    spec = ffv.build_tree_spec_from_paths(paths=[(1, 2), (1, 3)], prefix_len=3, page_size=4, device="cpu")
    assert spec.node_count == 4 and spec.parent_indices == [-1, 0, -1, 2]


def test_tree_mask_from_dense_window_detection():
    ta = pkg("tree_attention")
    _, parents, _, _ = ref.dedup_tree([(1, 2, 3), (1, 5, 6), (9, 9, 9)])
    mask = torch.from_numpy(ref.ancestor_mask(parents, 40))
    col0, bits = ta.tree_mask_from_dense(mask)
    assert col0 == 40
    for i in range(mask.shape[0]):
        assert [(int(bits[i]) >> j) & 1 for j in range(mask.shape[1] - 40)] == mask[i, 40:].int().tolist()
    # A mask whose hidden region spans more than 64 columns is not a tree window.
    wide = torch.ones((2, 200), dtype=torch.bool)
    wide[0, 10] = False
    assert ta.tree_mask_from_dense(wide) is None
    # all-visible mask
    col0, bits = ta.tree_mask_from_dense(torch.ones((3, 50), dtype=torch.bool))
    assert col0 == 50


def test_packbits_and_unpack_roundtrip():
    ffv = pkg("flashinfer_full_verify")
    ta = pkg("tree_attention")
    rng = np.random.default_rng(1)
    x = torch.from_numpy(rng.random(101) > 0.4)
    assert ffv.packbits(x).tolist() == np.packbits(x.numpy()).tolist()
    little = ffv.packbits(x, bitorder="little")
    assert ta.unpack_bits_little(little, 101).tolist() == x.tolist()


def test_ancestor_bitmasks_arbitrary_order():
    ffv = pkg("flashinfer_full_verify")
    # parent after child: bitmask still the ancestor closure
    parents = [2, -1, 1]
    bits = ffv.ancestor_bitmasks(parents)
    assert bits == [0b111, 0b010, 0b110]


def test_plan_argument_validation_without_gpu():
    ta = pkg("tree_attention")
    w = ta.BatchPrefillWithPagedKVCacheWrapper(torch.empty(16, dtype=torch.uint8), "NHD")
    with pytest.raises(RuntimeError, match="HIP device"):
        w.plan(torch.tensor([0, 1]), torch.tensor([0, 1]), torch.tensor([0]), torch.tensor([1]), 4, 2, 64, 16)
    assert ta.BatchPrefillWithPagedKVCacheWrapper(torch.empty(16, dtype=torch.uint8), "HND").kv_layout == "HND"
    with pytest.raises(NotImplementedError):
        ta.BatchPrefillWithPagedKVCacheWrapper(torch.empty(16, dtype=torch.uint8), "NDH")


def test_cached_tree_window_validated_against_plan():
    ffv = pkg("flashinfer_full_verify")
    ta = pkg("tree_attention")
    spec = ffv.build_tree_spec_from_paths(paths=[(1, 2, 3), (1, 5, 6)], prefix_len=20, page_size=4, device="cpu")
    n, kv = spec.node_count, spec.kv_len
    mask = spec.bool_mask
    col0, bits = ta._cached_tree_window(mask, [n], [kv])
    assert col0 == 20 and bits.tolist() == spec.tree_mask.tolist()
    # a plan of another shape, or of several requests, does not take the window
    assert ta._cached_tree_window(mask, [n], [kv + 1]) is None
    assert ta._cached_tree_window(mask, [n - 1], [kv]) is None
    assert ta._cached_tree_window(mask, [n, 1], [kv, kv]) is None
    # an in-place change of the mask invalidates it; the dense path then agrees
    # (undeduplicated: node 3 is the second path's root, node 4 its child)
    mask[4 * kv + 23] = False  # row 4 no longer sees tree node 3
    assert ta._cached_tree_window(mask, [n], [kv]) is None
    col0, bits2 = ta.tree_mask_from_dense(mask.view(n, kv))
    assert col0 == 20 and int(bits[4]) == 0b11000 and int(bits2[4]) == 0b10000


def test_cached_values_under_inference_mode():
    """The Target builds its tree spec under torch.inference_mode.  The
    builder's tensors are still normal tensors with version counters, so the
    attached host values and window are taken while unchanged and dropped
    after an in-place write made in inference mode; a host copy attached to
    an inference tensor (no counter) is never trusted."""
    ffv = pkg("flashinfer_full_verify")
    ta = pkg("tree_attention")
    with torch.inference_mode():
        spec, _ = ffv.build_deduplicated_tree_spec_from_paths(paths=[(1, 2, 3), (1, 5, 6)], prefix_len=20,
                                                              page_size=4, device="cpu")
        assert not spec.bool_mask.is_inference() and not spec.kv_last_page_len.is_inference()
        got = ta._cached_tree_window(spec.bool_mask, [spec.node_count], [spec.kv_len])
        assert got is not None and got[0] == 20 and got[1].tolist() == spec.tree_mask.tolist()
        assert ta._cached_tree_window(spec.bool_mask, [spec.node_count], [spec.kv_len + 3]) is None
        assert ta._cached_host_values(spec.kv_last_page_len) == [spec.kv_len - 4 * (spec.total_pages - 1)]
        spec.kv_last_page_len.add_(1)
        spec.bool_mask[spec.kv_len + 20] = False
        assert ta._cached_host_values(spec.kv_last_page_len) is None
        assert ta._cached_tree_window(spec.bool_mask, [spec.node_count], [spec.kv_len]) is None
        foreign = ffv.with_host_values(torch.tensor([0, 5], dtype=torch.int32), [0, 5])
        assert foreign.is_inference() and ta._cached_host_values(foreign) is None
        mask = torch.ones(spec.node_count * spec.kv_len, dtype=torch.bool)
        mask._atlas_tree_window = (20, spec.tree_mask, ffv.tensor_version(mask))
        assert ta._cached_tree_window(mask, [spec.node_count], [spec.kv_len]) is None
    # the host lists then come from the tensors themselves
    assert ta._host_lists(foreign)[0] == [0, 5]


def test_wide_tree_tile_words_match_brute_force():
    """Per-tile mask words of trees wider than 64 columns: the builder's host
    words, the plan's words derived from the dense mask and a brute-force
    reading of the oracle's dense ancestor mask agree bit for bit (prefixes on
    and off a tile boundary, 68 to 255 nodes)."""
    import random

    import numpy as np

    from oracle import paged_kv as ref

    ffv = pkg("flashinfer_full_verify")
    ta = pkg("tree_attention")
    rng = random.Random(3)
    for n_routes, prefix in ((17, 100), (32, 64), (64, 1000), (40, 0)):
        paths = [tuple(rng.randrange(500) for _ in range(4)) for _ in range(n_routes)]
        spec, _ = ffv.build_deduplicated_tree_spec_from_paths(paths=paths, prefix_len=prefix, page_size=16,
                                                              device="cpu")
        n, kv = spec.node_count, spec.kv_len
        assert n > 64
        _, parents, _, _ = ref.dedup_tree(paths)
        dense = ref.ancestor_mask(parents, prefix)
        t0 = prefix // 64
        ntiles = (kv - 1) // 64 - t0 + 1
        brute = np.zeros((n, ntiles), dtype=np.uint64)
        for i in range(n):
            for j in range(ntiles):
                word = 0
                for b in range(64):
                    key = 64 * (t0 + j) + b
                    if key < kv and dense[i, key]:
                        word |= 1 << b
                brute[i, j] = word
        col0, words, _ = spec.bool_mask._atlas_tree_tiles
        assert col0 == prefix and np.array_equal(words.numpy().view(np.uint64), brute)
        c2, w2 = ta.tree_tile_words_from_dense(torch.from_numpy(dense))
        assert c2 == prefix and np.array_equal(w2.numpy().view(np.uint64), brute)
        assert ta._cached_tree_tiles(spec.bool_mask, [n], [kv]) is not None
        assert ta._cached_tree_tiles(spec.bool_mask, [n], [kv + 64]) is None
        assert ta._cached_tree_window(spec.bool_mask, [n], [kv]) is None
    # beyond the per-tile layout's width: refused
    wide = torch.ones((2, ta.MAX_WIDE_TREE_WIDTH + 10), dtype=torch.bool)
    wide[0, 3] = False
    assert ta.tree_tile_words_from_dense(wide) is None


def _lib_build(paths, prefix_len, page_size, dedup, out_bytes=None):
    """Call atlas_tree_spec_build directly with a buffer of exactly
    atlas_tree_spec_bytes (or ``out_bytes``) bytes."""
    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    arr = np.asarray(paths, dtype=np.int64)
    k, depth = arr.shape
    need = lib.atlas_tree_spec_bytes(k, depth, prefix_len, page_size)
    out = np.zeros(need if out_bytes is None else out_bytes, dtype=np.uint8)
    parents = np.full(k * depth, -7, dtype=np.int32)
    routes = np.full(k * depth, -7, dtype=np.int32)
    info = np.zeros(8, dtype=np.int64)
    rc = lib.atlas_tree_spec_build(arr.ctypes.data, k, depth, int(dedup), prefix_len, page_size, out.ctypes.data,
                                   out.nbytes, parents.ctypes.data, routes.ctypes.data, info.ctypes.data)
    return rc, need, out, parents, routes, info


def test_native_tree_builder_matches_oracle_across_mask_regimes():
    """The library's host builder against the oracle's trie and ancestor mask:
    route -> node paths, parents, token ids, depths, the packed int32 block
    and the tree block of the dense mask, for trees of up to 64 nodes (one
    word per node), up to 1024 (tile words) and beyond (block only), with and
    without deduplication; the buffer bound holds in every case."""
    import random

    rng = random.Random(11)
    cases = [(9, 4, 3, 0), (3, 4, 2, 37), (40, 4, 6, 64), (300, 4, 40, 1000), (300, 5, 400, 17), (1, 1, 5, 0)]
    for k, depth, vocab, prefix in cases:
        paths = [tuple(rng.randrange(vocab) for _ in range(depth)) for _ in range(k)]
        for dedup in (True, False):
            rc, need, out, parents, routes, info = _lib_build(paths, prefix, 16, dedup)
            assert rc == 0
            n, kv_len, pages, last, n_words, tiles, n32, nbytes = info.tolist()
            assert nbytes <= need
            if dedup:
                tokens, oparents, odepths, oroutes = ref.dedup_tree(paths)
                assert routes.reshape(k, depth).tolist() == oroutes
            else:
                tokens = [t for p in paths for t in p]
                odepths = [d for _ in paths for d in range(depth)]
                oparents = [-1 if d == 0 else i - 1 for i, d in enumerate(odepths)]
            assert n == len(tokens) and parents[:n].tolist() == list(oparents)
            assert out[: 8 * n].view(np.int64).tolist() == list(tokens)
            assert out[8 * n : 16 * n].view(np.int64).tolist() == list(odepths)
            assert kv_len == prefix + n and pages == (kv_len + 15) // 16 and last == kv_len - 16 * (pages - 1)
            assert n_words == (n if n <= 64 else n * tiles if n <= 1024 else 0) and (tiles > 0) == (64 < n <= 1024)
            i32 = out[16 * n + 8 * n_words : 16 * n + 8 * n_words + 4 * n32].view(np.int32)
            assert n32 % 2 == 0 and i32[:5].tolist() == [0, n, 0, pages, last]
            assert i32[5 : 5 + pages].tolist() == list(range(pages)) and not i32[5 + pages :].any()
            mask = ref.ancestor_mask(list(oparents), prefix)
            block = out[16 * n + 8 * n_words + 4 * n32 : nbytes].reshape(n, n)
            assert np.array_equal(block.astype(bool), mask[:, prefix:])
            if n <= 64:
                assert out[16 * n : 16 * n + 8 * n].view(np.uint64).tolist() == [
                    int(sum(1 << j for j in range(n) if mask[i, prefix + j])) for i in range(n)]


def test_native_tree_builder_bound_and_refusals():
    """atlas_tree_spec_bytes bounds every tree of the shape, also when
    deduplication brings a tree of more than 1024 path positions into the
    tile-word range; a buffer one byte short, an empty path list, a zero
    depth and NULL outputs are refused with ATLAS_EINVAL."""
    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    # 1100 path positions, 1024 nodes after deduplication (all share token 0 at depth 0)
    paths = [(0, 1 + i // 3, 1 + i % 3) for i in range(341)] + [(0, 1000, 1001)] * 26
    paths = paths[:366] + [(0, 2000, 2001)]
    rc, need, _, _, _, info = _lib_build(paths, 5000, 16, True)
    assert rc == 0 and info[7] <= need and 64 < info[0] <= 1024
    rc, *_ = _lib_build(paths, 5000, 16, True, out_bytes=int(info[7]) - 1)
    assert rc == lib_mod.ATLAS_EINVAL and b"out buffer holds" in lib.atlas_last_error()
    assert lib.atlas_tree_spec_bytes(0, 4, 0, 16) == -1 and lib.atlas_tree_spec_bytes(3, 0, 0, 16) == -1
    assert lib.atlas_tree_spec_bytes(3, 4, -1, 16) == -1 and lib.atlas_tree_spec_bytes(3, 4, 0, 0) == -1
    arr = np.zeros((2, 3), dtype=np.int64)
    info = np.zeros(8, dtype=np.int64)
    rc = lib.atlas_tree_spec_build(arr.ctypes.data, 2, 3, 1, 0, 16, None, 1 << 20, None, None, info.ctypes.data)
    assert rc == lib_mod.ATLAS_EINVAL and b"NULL" in lib.atlas_last_error()
    rc = lib.atlas_tree_spec_build(arr.ctypes.data, 0, 3, 1, 0, 16, None, 0, None, None, None)
    assert rc == lib_mod.ATLAS_EINVAL and b"empty" in lib.atlas_last_error()


def test_tree_spec_builders_accept_tensor_and_numpy_paths():
    ffv = pkg("flashinfer_full_verify")
    paths = [(10, 20, 30), (10, 20, 31), (11, 21, 32)]
    want, routes = ffv.build_deduplicated_tree_spec_from_paths(paths=paths, prefix_len=5, page_size=4, device="cpu")
    for alt in (torch.tensor(paths), np.asarray(paths), [list(p) for p in paths]):
        got, r2 = ffv.build_deduplicated_tree_spec_from_paths(paths=alt, prefix_len=5, page_size=4, device="cpu")
        assert r2 == routes and torch.equal(got.bool_mask, want.bool_mask)
        assert got.flat_token_ids.tolist() == [10, 20, 30, 31, 11, 21, 32]
    # a later build does not change an earlier spec (the builder reuses host buffers)
    before = want.bool_mask.clone(), want.flat_token_ids.clone()
    ffv.build_deduplicated_tree_spec_from_paths(paths=[(1, 2, 3)] * 4, prefix_len=9, page_size=4, device="cpu")
    assert torch.equal(before[0], want.bool_mask) and torch.equal(before[1], want.flat_token_ids)


def _paths_strategy():
    from hypothesis import strategies as st

    return st.integers(1, 6).flatmap(lambda depth: st.lists(
        st.lists(st.integers(0, 3), min_size=depth, max_size=depth).map(tuple), min_size=1, max_size=14))


def test_tree_spec_builders_match_oracle_on_random_shapes():
    """Property test of the spec builders (the library's host builder behind
    them) against the oracle's trie and ancestor mask: small token alphabets
    (so routes share prefixes and repeat), depth 1 to 6, prefixes on and off
    64-key tiles, page sizes 1 to 64."""
    from hypothesis import HealthCheck, given, settings
    from hypothesis import strategies as st

    ffv = pkg("flashinfer_full_verify")

    @settings(max_examples=150, deadline=None, suppress_health_check=[HealthCheck.too_slow])
    @given(paths=_paths_strategy(), prefix=st.integers(0, 200), ps=st.sampled_from([1, 4, 16, 64]),
           dedup=st.booleans())
    def check(paths, prefix, ps, dedup):
        if dedup:
            spec, routes = ffv.build_deduplicated_tree_spec_from_paths(paths=paths, prefix_len=prefix, page_size=ps,
                                                                      device="cpu")
            tokens, parents, depths, oroutes = ref.dedup_tree(paths)
            assert routes == oroutes
        else:
            spec = ffv.build_tree_spec_from_paths(paths=paths, prefix_len=prefix, page_size=ps, device="cpu")
            tokens = [t for p in paths for t in p]
            depths = [d for p in paths for d in range(len(p))]
            parents = [-1 if d == 0 else i - 1 for i, d in enumerate(depths)]
        n = len(tokens)
        assert spec.flat_token_ids.tolist() == list(tokens) and spec.parent_indices == list(parents)
        assert spec.depths.tolist() == list(depths)
        mask = ref.ancestor_mask(list(parents), prefix)
        assert spec.bool_mask.numpy().tolist() == mask.reshape(-1).tolist()
        kv_len = prefix + n
        pages = -(-kv_len // ps)
        assert (spec.node_count, spec.kv_len, spec.total_pages) == (n, kv_len, pages)
        assert spec.kv_last_page_len.tolist() == [kv_len - (pages - 1) * ps]
        assert spec.qo_indptr.tolist() == [0, n] and spec.kv_indptr.tolist() == [0, pages]
        assert spec.kv_indices.tolist() == list(range(pages))

    check()
