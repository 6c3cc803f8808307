"""The verify-attention plan's work decomposition, on the host.

For random request mixes (query and KV lengths, head counts, head dims, page
sizes, workspace sizes, split targets) the work items must cover every
(request, KV head, query row, key) exactly once, the merge items must name
exactly the split items' partial rows, every item must fit the kernels'
limits (row tiles per item, splits per row, workspace rows), and the int32
metadata the kernels read must hold the same lists.  A decomposition that
drops or repeats a key range, or points two splits at one partial row,
fails here without a GPU."""

import math
from collections import defaultdict

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from helpers import pkg

ta = pkg("tree_attention")

HEADS = [(32, 8), (8, 8), (16, 2), (4, 1), (32, 4), (64, 8)]


def _decompose(qo_lens, kv_lens, hq, hkv, d, ps, ws_rows_cap, split_target=None, max_rows=None):
    w = ta.BatchPrefillWithPagedKVCacheWrapper(torch.empty(16, dtype=torch.uint8))
    w.split_target_items = split_target
    w.max_rows_per_item = max_rows
    qo = [0]
    for n in qo_lens:
        qo.append(qo[-1] + n)
    kvp = [0]
    for n in kv_lens:
        kvp.append(kvp[-1] + math.ceil(n / ps))
    cols = [k - q for q, k in zip(qo_lens, kv_lens)]  # the tree's columns start after the prefix
    dec = w._decompose(batch=len(qo_lens), qo=qo, kvp=kvp, qo_lens=list(qo_lens), kv_lens=list(kv_lens), cols=cols,
                       hq=hq, hkv=hkv, d=d, ps=ps, ws_rows_cap=ws_rows_cap)
    return dec, qo, kvp, cols


def _check(dec, qo, kvp, cols, qo_lens, kv_lens, hq, hkv, d, ps, ws_rows_cap):
    group = hq // hkv
    batch = len(qo_lens)
    direct = d == 128 and ps >= 16 and (ps & (ps - 1)) == 0
    row_cap = ta.MAX_ROWS_PER_ITEM if direct else ta.MAX_ROWS_PER_ITEM_OTHER
    work = dec["work"]
    assert all(len(it) == 16 for it in work)

    # the metadata array the kernels read holds the same lists
    meta = dec["meta"]
    assert meta.dtype == np.int32
    n = len(work)
    assert dec["merge_off"] == 16 * n
    assert (meta[: 16 * n].reshape(n, 16) == np.asarray(work, dtype=np.int64)).all()
    nm = dec["num_merge"]
    merges = meta[dec["merge_off"]: dec["merge_off"] + 8 * nm].reshape(nm, 8).tolist()
    assert dec["kvlen_off"] == dec["merge_off"] + 8 * nm
    assert meta[dec["kvlen_off"]: dec["kvlen_off"] + batch].tolist() == list(kv_lens)
    assert meta[dec["col_off"]: dec["col_off"] + batch].tolist() == cols
    assert meta[dec["qo_off"]: dec["qo_off"] + batch + 1].tolist() == qo
    assert meta[dec["kvp_off"]: dec["kvp_off"] + batch + 1].tolist() == kvp
    assert len(meta) == dec["kvp_off"] + batch + 1

    blocks = defaultdict(list)  # (b, h, r0, nr) -> [(k0, k1, base)]
    for it in work:
        b, h, r0, nr, k0, k1, base = it[:7]
        assert 0 <= b < batch and 0 <= h < hkv
        # the request values every item repeats, then padding
        assert tuple(it[7:12]) == (qo[b], qo_lens[b], kv_lens[b], cols[b], kvp[b])
        assert tuple(it[12:]) == (0, 0, 0, 0)
        assert 0 <= nr <= row_cap and math.ceil(nr / 16) <= 16
        blocks[(b, h, r0, nr)].append((k0, k1, base))

    # row blocks: for each (request, KV head), they tile [0, rows) in order
    for b in range(batch):
        rows = qo_lens[b] * group
        for h in range(hkv):
            mine = sorted((r0, nr) for (bb, hh, r0, nr) in blocks if bb == b and hh == h)
            if rows == 0:
                assert mine == [(0, 0)]
                continue
            at = 0
            for r0, nr in mine:
                assert r0 == at and nr > 0
                at += nr
            assert at == rows

    # key ranges: for each row block, the splits tile [0, kv_len) in whole
    # tiles, balanced to within one tile; partial rows only when split
    used = []  # (start, end) partial-row regions
    merge_keys = {}
    for m in merges:
        b, h, r0, nr, base, splits = m[:6]
        assert tuple(m[6:]) == (0, 0)
        assert (b, h, r0, nr) not in merge_keys
        merge_keys[(b, h, r0, nr)] = (base, splits)
    for (b, h, r0, nr), ranges in blocks.items():
        kv = kv_lens[b]
        ranges.sort()
        splits = len(ranges)
        assert 1 <= splits <= ta.MAX_SPLITS
        at = 0
        for k0, k1, _ in ranges:
            assert k0 == at and k0 % ta.TILE_KEYS == 0
            assert k1 > k0 or kv == 0
            at = k1
        assert at == kv
        tiles = [math.ceil((k1 - k0) / ta.TILE_KEYS) for k0, k1, _ in ranges]
        assert max(tiles) - min(tiles) <= 1
        assert tiles[-1] <= tiles[0]  # the split with the masked tail tile is not the longest
        if splits == 1:
            assert ranges[0][2] == -1 and (b, h, r0, nr) not in merge_keys
            continue
        base, msplits = merge_keys.pop((b, h, r0, nr))
        assert msplits == splits
        assert [r[2] for r in ranges] == [base + s * nr for s in range(splits)]
        used.append((base, base + splits * nr))
    assert not merge_keys, "merge items without split items"
    used.sort()
    for (a0, a1), (b0, _) in zip(used, used[1:]):
        assert a1 <= b0, "two merge items share partial rows"
    assert dec["partial_rows"] == sum(e - s for s, e in used)
    assert dec["partial_rows"] <= ws_rows_cap

    # dispatch order: longest items first
    lens = [it[5] - it[4] for it in work]
    assert lens == sorted(lens, reverse=True)
    assert dec["tiles_per_split"] == max((math.ceil(x / ta.TILE_KEYS) for x in lens), default=0)
    assert dec["max_rows"] == max(nr for (_, _, _, nr) in blocks)
    assert dec["direct"] == direct
    assert dec["fused_append"] == (direct and all(r0 == 0 for (_, _, r0, _) in blocks))


@st.composite
def request_mix(draw):
    hq, hkv = draw(st.sampled_from(HEADS))
    d = draw(st.sampled_from([64, 128]))
    ps = draw(st.sampled_from([1, 16, 64]))
    batch = draw(st.integers(1, 6))
    qo_lens = draw(st.lists(st.integers(0, 48), min_size=batch, max_size=batch))
    kv_lens = [q + draw(st.integers(0, 20000)) for q in qo_lens]
    ws_rows_cap = draw(st.sampled_from([0, 64, 1000, 20000, 1 << 22]))
    split_target = draw(st.sampled_from([None, 1, 37, 240, 512]))
    max_rows = draw(st.sampled_from([None, None, 16, 48, 256]))
    return qo_lens, kv_lens, hq, hkv, d, ps, ws_rows_cap, split_target, max_rows


@settings(max_examples=300, deadline=None, derandomize=True, suppress_health_check=[HealthCheck.too_slow])
@given(request_mix())
def test_random_request_mixes_are_covered_exactly_once(mix):
    qo_lens, kv_lens, hq, hkv, d, ps, ws_rows_cap, split_target, max_rows = mix
    dec, qo, kvp, cols = _decompose(qo_lens, kv_lens, hq, hkv, d, ps, ws_rows_cap, split_target, max_rows)
    _check(dec, qo, kvp, cols, qo_lens, kv_lens, hq, hkv, d, ps, ws_rows_cap)


@pytest.mark.parametrize("nodes,kv_len,splits", [(34, 16418, 30), (12, 16396, 30), (12, 4108, 30)])
def test_single_request_fills_240_items(nodes, kv_len, splits):
    """One head_dim-128 request with a large workspace: one row block per KV
    head (fused append allowed) and 8 x 30 = 240 items, each KV head's splits
    within one tile of each other."""
    dec, qo, kvp, cols = _decompose([nodes], [kv_len], 32, 8, 128, 16, 1 << 22)
    _check(dec, qo, kvp, cols, [nodes], [kv_len], 32, 8, 128, 16, 1 << 22)
    assert len(dec["work"]) == 8 * splits and dec["num_merge"] == 8 and dec["fused_append"]


def test_small_workspace_coarsens_the_splits():
    """A workspace too small for the finest split doubles the tiles per split
    until the partial rows fit; with no workspace every row block is one item."""
    big, *_ = _decompose([34], [16418], 32, 8, 128, 16, 1 << 22)
    small, qo, kvp, cols = _decompose([34], [16418], 32, 8, 128, 16, 136 * 8 * 10)
    none, *_ = _decompose([34], [16418], 32, 8, 128, 16, 0)
    _check(small, qo, kvp, cols, [34], [16418], 32, 8, 128, 16, 136 * 8 * 10)
    assert big["partial_rows"] > 136 * 8 * 10 >= small["partial_rows"] > 0
    assert len(none["work"]) == 8 and none["num_merge"] == 0 and none["partial_rows"] == 0
