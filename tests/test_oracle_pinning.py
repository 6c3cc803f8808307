"""Pin the oracle: reference test literals, closed forms, brute force and
library routines that a plausible mistake in the oracle would fail."""

import hashlib
import itertools
import math

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import paged_kv as ref
from oracle import scoring as osc


# ---------------------------------------------------------------- a1 metadata
def _slot_path(page_ids, length, page_size=16):
    slots = [p * page_size + o for p in page_ids for o in range(page_size)]
    return slots[:length]


def test_metadata_reference_literals():
    # tests/test_paged_attention_metadata.py:24-42
    lengths = [1, 15, 16, 17, 31, 32]
    paths = [_slot_path([11 + 3 * i, 31 + 5 * i], n) for i, n in enumerate(lengths)]
    md = ref.paged_metadata(paths, 16)
    counts = [(n + 15) // 16 for n in lengths]
    assert md.kv_indptr == list(itertools.accumulate([0] + counts))
    assert md.kv_last_page_len == [1, 15, 16, 1, 15, 16]
    assert md.seq_lens == lengths
    assert md.token_index_count == sum(lengths)
    assert len(md.kv_page_indices) == sum(counts)
    assert md.layout_ok
    # page ids are the physical pages of each path
    flat = [p for i, n in enumerate(lengths) for p in [11 + 3 * i, 31 + 5 * i][: counts[i]]]
    assert md.kv_page_indices == flat


def test_metadata_long_prefix_literal():
    # tests/test_paged_attention_metadata.py:45-52
    md = ref.paged_metadata([_slot_path(list(range(100, 612)), 8192)], 16)
    assert md.token_index_count == 8192 and len(md.kv_page_indices) == 512
    assert md.kv_indptr == [0, 512] and md.kv_last_page_len == [16]


@pytest.mark.parametrize("path", [[161, 162, 163], [160, 161, 165], list(range(160, 176)) + [193]])
def test_metadata_rejects_invalid_layouts(path):
    # tests/test_paged_attention_metadata.py:55-67
    assert not ref.paged_metadata([path], 16).layout_ok


def test_metadata_errors():
    with pytest.raises(ValueError):
        ref.paged_metadata([[1]], 0)
    with pytest.raises(ValueError):
        ref.paged_metadata([], 16)
    with pytest.raises(ValueError):
        ref.paged_metadata([[]], 16)


# ---------------------------------------------------------------- a2 dedup
def test_dedup_reference_literals():
    # tests/test_tree_dedup.py:6-25
    tokens, parents, depths, routes = ref.dedup_tree([(10, 20, 30, 40), (10, 20, 31, 41), (11, 21, 32, 42)])
    assert tokens == [10, 20, 30, 40, 31, 41, 11, 21, 32, 42]
    assert parents == [-1, 0, 1, 2, 1, 4, -1, 6, 7, 8]
    assert depths == [0, 1, 2, 3, 2, 3, 0, 1, 2, 3]
    assert routes == [[0, 1, 2, 3], [0, 1, 4, 5], [6, 7, 8, 9]]


def test_dedup_identical_routes_literal():
    # tests/test_tree_dedup.py:28-35
    tokens, parents, depths, routes = ref.dedup_tree([(7, 8), (7, 8)])
    assert tokens == [7, 8] and parents == [-1, 0] and depths == [0, 1] and routes == [[0, 1], [0, 1]]


def test_dedup_brute_force_unique_prefixes():
    rng = np.random.default_rng(0)
    for _ in range(50):
        paths = [tuple(int(x) for x in rng.integers(0, 3, size=4)) for _ in range(9)]
        tokens, parents, depths, routes = ref.dedup_tree(paths)
        prefixes = {p[: i + 1] for p in paths for i in range(4)}
        assert len(tokens) == len(prefixes)
        for path, nodes in zip(paths, routes):
            for i, node in enumerate(nodes):
                # reconstruct the prefix through parents
                chain, cur = [], node
                while cur >= 0:
                    chain.append(tokens[cur])
                    cur = parents[cur]
                assert tuple(reversed(chain)) == path[: i + 1]
                assert depths[node] == i
        # insertion order: a node's parent precedes it
        assert all(p < i for i, p in enumerate(parents))
        # commit aliasing argument: node_ids[j] < depth implies node_ids[j] == j
        for nodes in routes:
            for j, nid in enumerate(nodes):
                if nid < 4:
                    assert nid == j


# ---------------------------------------------------------------- a3 mask
def test_ancestor_mask_closed_form():
    _, parents, _, _ = ref.dedup_tree([(10, 20, 30, 40), (10, 20, 31, 41), (11, 21, 32, 42)])
    m = ref.ancestor_mask(parents, 5)
    assert m.shape == (10, 15)
    assert m[:, :5].all()
    tree = m[:, 5:]
    # node 5 (41) sees 0, 1, 4, 5; node 6 (11) sees only itself
    assert np.flatnonzero(tree[5]).tolist() == [0, 1, 4, 5]
    assert np.flatnonzero(tree[6]).tolist() == [6]
    # reflexive, and transitive: a visible column's own visible set is a subset
    for i in range(10):
        assert tree[i, i]
        for j in np.flatnonzero(tree[i]):
            assert (tree[j] <= tree[i]).all()


def test_packbits_matches_numpy_orders():
    rng = np.random.default_rng(1)
    x = rng.random(77) > 0.5
    assert ref.packbits(x).tolist() == np.packbits(x).tolist()
    little = ref.packbits(x, "little")
    assert np.unpackbits(little, bitorder="little")[:77].astype(bool).tolist() == x.tolist()


# ---------------------------------------------------------------- a4 attention
def _sdpa_reference(q, k, v, mask, scale):
    qt = torch.from_numpy(q).permute(1, 0, 2)  # [H, n, D]
    kt = torch.from_numpy(k).permute(1, 0, 2)
    vt = torch.from_numpy(v).permute(1, 0, 2)
    out = torch.nn.functional.scaled_dot_product_attention(
        qt, kt, vt, attn_mask=torch.from_numpy(mask)[None], scale=scale
    )
    return out.permute(1, 0, 2).numpy()


def test_attention_matches_torch_sdpa_and_is_page_permutation_invariant():
    rng = np.random.default_rng(2)
    hq, hkv, d, ps = 8, 2, 32, 4
    prefix = 13
    _, parents, _, _ = ref.dedup_tree([(1, 2, 3), (1, 4, 5)])
    n = len(parents)
    kv_len = prefix + n
    pages = math.ceil(kv_len / ps)
    kv = rng.standard_normal((pages + 3, 2, ps, hkv, d))
    q = rng.standard_normal((n, hq, d))
    mask = ref.ancestor_mask(parents, prefix)
    last = kv_len - (pages - 1) * ps
    perm = list(rng.permutation(pages + 3)[:pages])
    o1, l1 = oatt.masked_attention(q, kv, [0, n], [0, pages], perm, [last], masks=[mask])
    # contiguous copy of the same pages
    kv2 = kv[perm]
    o2, l2 = oatt.masked_attention(q, kv2, [0, n], [0, pages], list(range(pages)), [last], masks=[mask])
    np.testing.assert_allclose(o1, o2, atol=1e-12)
    np.testing.assert_allclose(l1, l2, atol=1e-12)
    k = kv2[:, 0].reshape(-1, hkv, d)[:kv_len].repeat(hq // hkv, axis=1)
    v = kv2[:, 1].reshape(-1, hkv, d)[:kv_len].repeat(hq // hkv, axis=1)
    # the GQA repeat must map q head h to kv head h // group
    k = np.concatenate([np.repeat(kv2[:, 0].reshape(-1, hkv, d)[:kv_len, h : h + 1], hq // hkv, axis=1)
                        for h in range(hkv)], axis=1)
    v = np.concatenate([np.repeat(kv2[:, 1].reshape(-1, hkv, d)[:kv_len, h : h + 1], hq // hkv, axis=1)
                        for h in range(hkv)], axis=1)
    sd = _sdpa_reference(q, k, v, mask, 1 / math.sqrt(d))
    np.testing.assert_allclose(o1, sd, atol=1e-10)
    # lse closed form
    s = np.einsum("nhd,khd->nhk", q, k) / math.sqrt(d)
    s = np.where(mask[:, None, :], s, -np.inf)
    np.testing.assert_allclose(l1, np.log(np.exp(s).sum(-1)), atol=1e-10)


def test_attention_special_cases():
    rng = np.random.default_rng(3)
    hq, hkv, d, ps = 4, 4, 16, 8
    kv = rng.standard_normal((5, 2, ps, hkv, d))
    # uniform V rows -> output equals that row regardless of scores
    kv[:, 1] = rng.standard_normal((hkv, d))[None, None]
    q = rng.standard_normal((3, hq, d))
    o, _ = oatt.masked_attention(q, kv, [0, 3], [0, 5], [0, 1, 2, 3, 4], [8])
    np.testing.assert_allclose(o, np.broadcast_to(kv[0, 1, 0][None], o.shape), atol=1e-12)
    # one visible key -> output is that key's V, lse is its score
    mask = np.zeros((1, 40), dtype=bool)
    mask[0, 17] = True
    kv = rng.standard_normal((5, 2, ps, hkv, d))
    q1 = rng.standard_normal((1, hq, d))
    o, l = oatt.masked_attention(q1, kv, [0, 1], [0, 5], [0, 1, 2, 3, 4], [8], masks=[mask])
    np.testing.assert_allclose(o[0], kv[2, 1, 1], atol=1e-12)
    np.testing.assert_allclose(l[0], (q1[0] * kv[2, 0, 1]).sum(-1) / 4.0, atol=1e-12)
    # fully masked row
    o, l = oatt.masked_attention(q1, kv, [0, 1], [0, 5], [0, 1, 2, 3, 4], [8], masks=[np.zeros((1, 40), bool)])
    assert (o == 0).all() and np.isneginf(l).all()
    # causal: last query sees everything, first sees kv_len - qo_len + 1 keys
    qc = rng.standard_normal((2, hq, d))
    oc, _ = oatt.masked_attention(qc, kv, [0, 2], [0, 5], [0, 1, 2, 3, 4], [8], causal=True)
    om, _ = oatt.masked_attention(qc, kv, [0, 2], [0, 5], [0, 1, 2, 3, 4], [8])
    np.testing.assert_allclose(oc[1], om[1], atol=1e-12)
    m0 = np.zeros((2, 40), bool)
    m0[0, :39] = True
    m0[1] = True
    o0, _ = oatt.masked_attention(qc, kv, [0, 2], [0, 5], [0, 1, 2, 3, 4], [8], masks=[m0])
    np.testing.assert_allclose(oc, o0, atol=1e-12)


# ---------------------------------------------------------------- a5/a6/a7
def _commit_cache():
    # tests/test_target_kv_commit.py:13-25
    cache = np.zeros((2, 2, 4, 1, 1), dtype=np.float32)
    for pos in range(8):
        page, off = divmod(pos, 4)
        cache[page, 0, off, 0, 0] = 100 + pos
        cache[page, 1, off, 0, 0] = 200 + pos
    return cache


def test_commit_reference_literals():
    # tests/test_target_kv_commit.py:28-45
    cache = _commit_cache()
    ref.commit([cache], 3, (0, 2))
    assert cache[0, 0, 3, 0, 0] == 103 and cache[1, 0, 0, 0, 0] == 105
    assert cache[0, 1, 3, 0, 0] == 203 and cache[1, 1, 0, 0, 0] == 205


def test_commit_clone_semantics_brute_force():
    rng = np.random.default_rng(4)
    for _ in range(20):
        cache = rng.standard_normal((6, 2, 4, 1, 2))
        nodes = sorted(rng.choice(10, size=3, replace=False).tolist())
        before = cache.copy()
        ref.commit([cache], 5, nodes)
        for i, nid in enumerate(nodes):
            s, d_ = 5 + nid, 5 + i
            np.testing.assert_array_equal(cache[d_ // 4, :, d_ % 4], before[s // 4, :, s % 4])


def test_capacity_growth_literal():
    # tests/test_target_kv_commit.py:48-55
    cache = _commit_cache()
    (grown,) = ref.grow_capacity([cache], 4)
    assert grown.shape[0] == 4 and np.array_equal(grown[:2], cache) and not grown[2:].any()


def test_prefix_to_paged_literal():
    # tests/test_target_kv_commit.py:58-73
    key = np.arange(5, dtype=np.float32).reshape(1, 1, 5, 1)
    value = (100 + np.arange(5, dtype=np.float32)).reshape(1, 1, 5, 1)
    cache = ref.prefix_to_paged(key, value, 5, 2, 4)
    assert [cache[p // 4, 0, p % 4, 0, 0] for p in range(5)] == [0, 1, 2, 3, 4]
    assert [cache[p // 4, 1, p % 4, 0, 0] for p in range(5)] == [100, 101, 102, 103, 104]


# ---------------------------------------------------------------- a9 / a13
def test_move_kv_reference_fake_semantics():
    # tests/test_tail_page_cow.py:9-16, :77-79
    values = [np.arange(512, dtype=np.float32)]
    ref.move_kv(values, [np.zeros(512)], [40, 41, 42], [0, 1, 2])
    assert values[0][40:43].tolist() == [0.0, 1.0, 2.0]


def test_prune_reference_literals():
    # tests/test_tail_page_cow.py:241-277: prefix [0, 1, 40] after promotion,
    # retained route 2 [0, 1, 40, 41], owned {0, 10, 11} -> free [11] (slot 44).
    released, owned = ref.prune({0, 10, 11}, [0, 1, 40], [[0, 1, 40, 41]], 4)
    assert released == [11] and owned == {0, 10}
    assert [p * 4 for p in released] == [44]
    # tests/test_tail_page_cow.py:280-293
    released, owned = ref.prune({0, 10, 11}, [0, 1], [[0, 1, 40]], 4)
    assert released == [11] and owned == {0, 10}
    assert ref.prune(owned, [0, 1], [[0, 1, 40]], 4)[0] == []


def test_prune_brute_force_sorted_difference():
    rng = np.random.default_rng(5)
    for _ in range(30):
        ps = int(rng.choice([1, 4, 16]))
        owned = set(rng.choice(200, size=60, replace=False).tolist())
        paths = []
        for _ in range(3):
            pages = rng.choice(200, size=4, replace=False)
            length = int(rng.integers(1, 4 * ps + 1))
            paths.append([int(pages[i // ps]) * ps + i % ps for i in range(length)])
        released, left = ref.prune(owned, None, paths, ps)
        live = {s // ps for p in paths for s in p}
        assert released == sorted(owned - live) and left == owned & live


def test_allocator_policy_brute_force():
    ps = 4
    a = ref.PagedAllocator(num_pages=20, page_size=ps)
    assert a.alloc(8) == [4, 5, 6, 7, 8, 9, 10, 11]
    a.free([9, 5, 40])
    assert a.free_pages[:3] == [1, 2, 10]
    # decode: request 0 continues slot 41 (seq 7 -> pre 6 not a boundary),
    # request 1 opens a page (seq 5 -> pre 4 boundary)
    out = a.alloc_decode([7, 5], [41, 99])
    assert out == [42, 4]
    # extend: prefix 6 -> 11 with last 45: slots 46, 47, then new pages
    a2 = ref.PagedAllocator(num_pages=20, page_size=ps)
    out = a2.alloc_extend([6, 0], [11, 3], [45, -1])
    assert out == [46, 47, 4, 5, 6, 8, 9, 10]
    # brute force: every extended slot sits at offset t % ps of its page
    a3 = ref.PagedAllocator(num_pages=100, page_size=ps)
    pre, seq = [3, 9, 0, 12], [10, 10, 5, 30]
    last = [2 * ps + 2, 5 * ps + 0, -1, 7 * ps + 3]
    slots = a3.alloc_extend(pre, seq, last)
    k = 0
    for p, s in zip(pre, seq):
        for t in range(p, s):
            assert slots[k] % ps == t % ps
            k += 1


# ---------------------------------------------------------------- a8 scoring
def test_scoring_reference_literal():
    # tests/test_target_kv_commit.py:76-103
    prefix = np.array([0.0, 3.0, 0.0, 0.0])
    verify = np.array([[0.0, 0.0, 4.0, 2.0], [0, 0, 0, 0], [0, 0, 0, 0]])
    lps = osc.route_token_logprobs([(1, 2), (1, 3)], [[0, 1], [0, 2]], prefix, verify)
    plp = float(torch.log_softmax(torch.tensor(prefix), -1)[1])
    vlp = torch.log_softmax(torch.tensor(verify[0]), -1)
    assert abs(sum(lps[0]) - (plp + float(vlp[2]))) < 1e-9
    assert abs(sum(lps[1]) - (plp + float(vlp[3]))) < 1e-9


def test_selection_literals():
    # target_best tie-break, tests/test_target_kv_commit.py:128-147, :311-331
    a = dict(route_id=9, selection_score=-1.0, draft_path_logprob=-2.0, token_ids=(11,))
    b = dict(route_id=4, selection_score=-1.0, draft_path_logprob=-1.0, token_ids=(12,))
    assert osc.select_best([a, b])["route_id"] == 4
    c = dict(route_id=1, selection_score=-1.0, draft_path_logprob=-0.3, token_ids=(10, 11))
    d = dict(route_id=2, selection_score=-1.0, draft_path_logprob=-2.0, token_ids=(20, 21))
    assert osc.select_best([d, c])["route_id"] == 1
    # identical scores: lowest route id wins
    e = dict(route_id=3, selection_score=-1.0, draft_path_logprob=-1.0, token_ids=(1,))
    f = dict(route_id=5, selection_score=-1.0, draft_path_logprob=-1.0, token_ids=(2,))
    assert osc.select_best([f, e])["route_id"] == 3


def test_sampling_draw_closed_form_and_order_independence():
    # target_runtime.py:507-511 draw; tests/test_target_kv_commit.py:167-219
    scores = [
        dict(route_id=8, token_ids=(30, 31), selection_score=-1.0, draft_path_logprob=-0.8),
        dict(route_id=2, token_ids=(10, 11), selection_score=-1.4, draft_path_logprob=-0.2),
        dict(route_id=5, token_ids=(20, 21), selection_score=-0.7, draft_path_logprob=-0.5),
    ]
    sa, da = osc.sample_route(scores, 1234, 7)
    sb, db = osc.sample_route(list(reversed(scores)), 1234, 7)
    _, dn = osc.sample_route(scores, 1234, 8)
    assert sa["token_ids"] == sb["token_ids"] and da == db and da != dn
    bits = int.from_bytes(hashlib.sha256(b"atlas0709-target-route-sample-v1:1234:7").digest()[:8], "big")
    assert da == (bits + 0.5) / 2.0**64
    # inverse CDF over the canonical (token-sorted) order
    ordered = sorted(scores, key=lambda s: s["token_ids"])
    w = np.exp(np.array([s["selection_score"] for s in ordered]) - max(s["selection_score"] for s in ordered))
    cdf = np.cumsum(w / w.sum())
    assert ordered[int(np.searchsorted(cdf, da, side="right"))]["route_id"] == sa["route_id"]


def test_truncation_literals():
    # tests/test_target_kv_commit.py:345-367
    assert osc.truncate_path((10, 11, 12, 13), (20, 21, 22, 23), 3, 11) == ((10, 11), (20, 21))
    with pytest.raises(ValueError, match="must be positive"):
        osc.truncate_path((10,), (20,), 0, None)


def test_weights_normalised():
    assert osc.normalise_weights([1.0, 3.0]) == (0.25, 0.75)
    with pytest.raises(ValueError):
        osc.normalise_weights([-1.0])


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_rope_matches_torch_16bit_ops(dtype):
    """The oracle's per-op rounding equals torch's own 16-bit tensor ops (what
    apply_rope_with_cos_sin runs, flashinfer_full_verify.py:324-333) bit for
    bit, and reduces to the identity at angle 0 and to rotate_half at cos 0 /
    sin 1; a plain fp32 rotation stays within one rounding step."""
    from oracle import rope as orope

    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    gen = torch.Generator().manual_seed(5)
    n, h, d = 37, 4, 128
    x = (torch.randn((n, h, d), generator=gen) * 3.0).to(tdt)
    pos = torch.arange(1000, 1000 + n, dtype=torch.float32)
    inv = 1.0 / (500000.0 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    emb = torch.cat((torch.outer(pos, inv),) * 2, dim=-1)
    cos, sin = emb.cos().to(tdt), emb.sin().to(tdt)

    def rot(t):
        return torch.cat((-t[..., d // 2:], t[..., : d // 2]), dim=-1)

    want = (x * cos[:, None, :]) + (rot(x) * sin[:, None, :])
    got = orope.apply_rope(x.float().numpy(), cos.float().numpy(), sin.float().numpy(), dtype)
    assert np.array_equal(got, want.float().numpy())
    # a dropped rounding step would differ somewhere in these inputs
    unrounded = x.float() * cos.float()[:, None, :] + rot(x.float()) * sin.float()[:, None, :]
    assert not np.array_equal(orope.round_to(unrounded.numpy(), dtype), got)
    # a wrong sign or half swap of rotate_half fails the plain-rotation bound
    ulp = 2.0 ** -10 if dtype == "f16" else 2.0 ** -7
    assert float(np.abs(got - unrounded.numpy()).max()) <= 4 * ulp * float(np.abs(unrounded.numpy()).max())
    one, zero = np.ones((n, d), np.float32), np.zeros((n, d), np.float32)
    xs = x.float().numpy()
    assert np.array_equal(orope.apply_rope(xs, one, zero, dtype), xs)
    assert np.array_equal(orope.apply_rope(xs, zero, one, dtype), orope.rotate_half(xs))


def _ofr():
    from oracle import frontier as ofr
    return ofr


def _cols(rows):
    """Candidate columns from (parent, root, token, cumulative, rank, parent_lp) tuples."""
    return {
        "parent_route_ids": np.array([r[0] for r in rows], np.int64),
        "stage1_root_ids": np.array([r[1] for r in rows], np.int64),
        "pending_token_ids": np.array([r[2] for r in rows], np.int64),
        "cumulative_logprobs": np.array([r[3] for r in rows], np.float64),
        "ranks_in_parent": np.array([r[4] for r in rows], np.int64),
        "parent_logprobs": np.array([r[5] if len(r) > 5 else 0.0 for r in rows], np.float64),
    }


def test_frontier_order_reference_literals():
    """test_paged_frontier_selection.py:79-130: complete score ties order by
    parent route, rank, token (global), and by root first (per root)."""
    ofr = _ofr()
    c = _cols([(20, 200, 7, -1.0, 0), (10, 100, 1, -1.0, 1), (10, 100, 9, -1.0, 0), (10, 100, 2, -1.0, 0),
               (5, 500, 0, -1.0, 2), (99, 900, 4, -0.5, 3)])
    sel = ofr.select_global(c, 6)
    assert c["pending_token_ids"][sel].tolist() == [4, 0, 2, 9, 1, 7]
    assert sel.tolist() == ofr.python_order(c)
    c = _cols([(20, 200, 8, -1.0, 0), (20, 200, 3, -1.0, 1), (10, 100, 9, -1.0, 0), (10, 100, 4, -1.0, 1),
               (21, 200, 7, -1.0, 0), (21, 200, 2, -1.0, 1), (11, 100, 6, -1.0, 0), (11, 100, 1, -1.0, 1)])
    sel = ofr.select_per_root(c, 2, [(200, 4), (100, 4)])
    assert c["stage1_root_ids"][sel].tolist() == [100, 100, 200, 200]
    assert c["parent_route_ids"][sel].tolist() == [10, 10, 20, 20]


def test_frontier_stable_order_equals_python_order_brute_force():
    """The successive stable argsorts give the Python-object order
    (utils.py:27-43) on batches dense with exact ties, NaN and -0.0 aside."""
    ofr = _ofr()
    rng = np.random.default_rng(3)
    for _ in range(200):
        n = int(rng.integers(1, 40))
        rows = [(int(rng.integers(0, 4)), int(rng.integers(0, 3)), int(rng.integers(0, 5)),
                 float(rng.integers(-3, 1)) * 0.5, int(rng.integers(0, 3))) for _ in range(n)]
        c = _cols(rows)
        assert ofr.stable_order(c).tolist() == ofr.python_order(c)
        by_root = ofr.stable_order(c, include_stage1_root=True).tolist()
        assert by_root == sorted(range(n), key=lambda i: (rows[i][1], ofr.python_order(c).index(i)))


def test_frontier_topk_matches_torch_log_softmax_topk():
    """parent_token_candidates = torch.topk(torch.log_softmax(rows)) on distinct
    fp32 values (sampling.py:131-134); on 16-bit rows the chosen values are
    torch's (the order of equal values is unspecified there); the Gumbel path
    takes the proposal's top-k and gathers the log-probs (:135-153)."""
    ofr = _ofr()
    gen = torch.Generator().manual_seed(8)
    x = torch.randn((6, 3000), generator=gen) * 4.0
    lp, ids = ofr.parent_token_candidates(x.numpy(), 5, "f32")
    tv, ti = torch.topk(torch.log_softmax(x, dim=-1), k=5, dim=-1)
    assert np.array_equal(ids, ti.numpy())
    assert np.allclose(lp, tv.numpy(), atol=2e-6, rtol=0)
    from oracle import rope as orope
    for tdt, odt, ulp in ((torch.float16, "f16", 2.0 ** -10), (torch.bfloat16, "bf16", 2.0 ** -7)):
        xr = (torch.randn((4, 5000), generator=gen) * 0.5).to(tdt)
        lp, ids = ofr.parent_token_candidates(xr.float().numpy(), 9, odt)
        # torch's device kernel rounds (x - max) - log(sum) once from fp32 (its
        # CPU 16-bit path rounds elsewhere): compare with the fp32 log-softmax
        # rounded once -- equal but for rare rounding-boundary cases
        ref = orope.round_to(torch.log_softmax(xr.float(), dim=-1).numpy(), odt)
        got = np.take_along_axis(ref, ids, axis=-1)
        assert float(np.abs(lp - got).max()) <= ulp * 8 and float(np.mean(lp == got)) > 0.95
        assert np.array_equal(np.sort(ref, axis=-1)[:, ::-1][:, :9], lp)
        # equal values come in ascending token order
        for r in range(4):
            for j in range(8):
                if lp[r, j] == lp[r, j + 1]:
                    assert ids[r, j] < ids[r, j + 1]
    prop = torch.randn((6, 3000), generator=gen)
    lp, ids = ofr.parent_token_candidates(x.numpy(), 4, "f32", proposal=prop.numpy())
    assert np.array_equal(ids, torch.topk(prop, k=4, dim=-1).indices.numpy())
    assert np.allclose(lp, torch.log_softmax(x, dim=-1).gather(-1, torch.from_numpy(ids)).numpy(), atol=2e-6)


def test_frontier_depth_and_records_literals():
    """test_paged_frontier_selection.py:189-275: two equal rows, k=2, four
    candidates, the two selected are those of route 1; 4 x 8 record elements
    (+ 2 rows of node ids); parent log-prob travels in column 6."""
    ofr = _ofr()
    logits = np.array([[0.0, 3.0, 3.0, 0.0, 0.0]] * 2, np.float32)
    lp, ids = ofr.parent_token_candidates(logits, 2, "f32")
    assert ids.tolist() == [[1, 2], [1, 2]]
    c = ofr.build_candidates([1, 2], [1, 2], [0.0, 0.0], lp, ids)
    sel = ofr.select_global(c, 2)
    assert c["parent_route_ids"][sel].tolist() == [1, 1] and c["pending_token_ids"][sel].tolist() == [1, 2]
    rec = ofr.pack_records(c, sel)
    assert rec.size == 4 * 8 and rec[:, 7].tolist() == [0, 1, -1, -1]
    rec = ofr.pack_records(c, sel, node_ids=[101, 102])
    assert rec.size == (4 + 2) * 8 and rec[4:, :2].tolist() == [[1, 101], [1, 102]]
    one = _cols([(7, 3, 11, -4.5, 2, -3.25)])
    rec = ofr.pack_records(one, np.array([0]))
    assert rec[0, 6] == np.float64(-3.25).view(np.int64) and rec[0, 5] == np.float64(-4.5).view(np.int64)


# ---------------------------------------------------------------- torch CPU path (baseline legs)
def test_torch_path_commit_and_append_equal_numpy_restatement():
    """The torch restatement of the reference's commit (target_runtime.py:886-912)
    and write_suffix_kv (flashinfer_full_verify.py:1027-1042) equal the numpy
    oracle, pinned by the reference literals above, bit for bit; and the
    commit literal holds for it directly."""
    from oracle import torch_path as tp

    cache = torch.from_numpy(_commit_cache().copy())
    tp.commit_torch([cache], 3, (0, 2), 4)
    assert cache[0, 0, 3, 0, 0] == 103 and cache[1, 0, 0, 0, 0] == 105
    rng = np.random.default_rng(9)
    for _ in range(10):
        layers = [rng.standard_normal((8, 2, 4, 2, 3)).astype(np.float32) for _ in range(3)]
        nodes = sorted(rng.choice(9, size=4, replace=False).tolist())
        mine = [torch.from_numpy(x.copy()) for x in layers]
        tp.commit_torch(mine, 11, nodes, 4)
        ref.commit(layers, 11, nodes)
        for a, b in zip(mine, layers):
            assert np.array_equal(a.numpy(), b)
        key = rng.standard_normal((5, 2, 3)).astype(np.float32)
        val = rng.standard_normal((5, 2, 3)).astype(np.float32)
        cache = rng.standard_normal((8, 2, 4, 2, 3)).astype(np.float32)
        mine = torch.from_numpy(cache.copy())
        tp.write_suffix_kv_torch(mine, torch.from_numpy(key), torch.from_numpy(val), 13, 4)
        ref.write_suffix(cache, key, val, 13)
        assert np.array_equal(mine.numpy(), cache)


def test_torch_path_cow_and_prune_equal_numpy_restatement():
    """Per-page move_kv_cache copies equal the oracle's move (FakeKVCache
    semantics, tests/test_tail_page_cow.py:14-16); the torch prune equals
    sorted(owned - live) with the reference's sampled live pages and the
    reference literals (tests/test_tail_page_cow.py:241-293)."""
    from oracle import torch_path as tp

    rng = np.random.default_rng(10)
    k = [rng.standard_normal((64, 2, 3)).astype(np.float32) for _ in range(2)]
    v = [rng.standard_normal((64, 2, 3)).astype(np.float32) for _ in range(2)]
    tk, tv = [torch.from_numpy(x.copy()) for x in k], [torch.from_numpy(x.copy()) for x in v]
    copies = [(torch.tensor([40, 41, 42]), torch.tensor([8, 9, 10])), (torch.tensor([44, 45]), torch.tensor([8, 9]))]
    tp.cow_copy_torch(tk, tv, copies)
    ref.move_kv(k, v, [40, 41, 42, 44, 45], [8, 9, 10, 8, 9])
    for a, b in zip(tk + tv, k + v):
        assert np.array_equal(a.numpy(), b)
    assert tp.prune_torch({0, 10, 11}, torch.tensor([0, 1, 40]), [torch.tensor([0, 1, 40, 41])], 4) == [11]
    assert tp.prune_torch({0, 10, 11}, torch.tensor([0, 1]), [torch.tensor([0, 1, 40])], 4) == [11]
    for _ in range(20):
        ps = int(rng.choice([1, 4, 16]))
        owned = set(rng.choice(200, size=60, replace=False).tolist())
        paths = []
        for _ in range(3):
            pages = rng.choice(200, size=4, replace=False)
            length = int(rng.integers(1, 4 * ps + 1))
            paths.append([int(pages[i // ps]) * ps + i % ps for i in range(length)])
        prefix = paths[0][: ps * 2]
        expect, _ = ref.prune(owned, prefix, paths, ps)
        got = tp.prune_torch(owned, torch.tensor(prefix), [torch.tensor(p) for p in paths], ps)
        assert got == expect
