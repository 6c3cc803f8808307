"""Drafter frontier on the gfx950 kernels against the oracle (oracle/frontier.py)
and against torch's own device log_softmax + topk: per-parent top-k, the
candidate records, the stable order and both selection policies, the packed
materialisation and the frontier depth flows of the reference's tests
(test_paged_frontier_selection.py)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import pkg
from oracle import frontier as ofr

pytestmark = pytest.mark.gpu

DT = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}


def _logits(gen, rows, vocab, dtype, scale):
    return (torch.randn((rows, vocab), generator=gen) * scale).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,vocab,k,scale", [(1, 5, 2, 1.0), (3, 1000, 3, 2.0), (9, 128256, 3, 3.0),
                                                (72, 128256, 3, 1.0), (5, 32001, 17, 0.05), (2, 4096, 32, 0.5)])
def test_topk_matches_oracle(dev, dtype, rows, vocab, k, scale):
    """batch_parent_token_candidates (greedy): ids and log-probs equal the
    oracle's, equal log-probs in ascending token order (scale 0.05 in 16-bit
    makes many equal values; vocab 32001 leaves rows unaligned)."""
    sampling = pkg("flashinfer_paged.sampling")
    gen = torch.Generator().manual_seed(rows * 1000 + vocab + k)
    x = _logits(gen, rows, vocab, dtype, scale)
    lp, ids = sampling.batch_parent_token_candidates(x.to(dev), k=k, sampling=None,
                                                     relative_parent_paths=[()] * rows)
    torch.cuda.synchronize()
    olp, oids = ofr.parent_token_candidates(x.float().numpy(), k, DT[dtype])
    assert lp.dtype == dtype and tuple(ids.shape) == (rows, min(k, vocab))
    assert np.array_equal(ids.cpu().numpy(), oids)
    _assert_logprobs(lp, olp, dtype)


def _assert_logprobs(lp, olp, dtype):
    """16-bit log-probs are rounded once from fp32 and must be equal; fp32
    log-probs keep the last bits of the log-sum-exp, whose summation order
    differs from the oracle's: within 1e-5."""
    got = lp.float().cpu().numpy()
    if dtype == torch.float32:
        assert float(np.abs(got - olp).max()) <= 1e-5
    else:
        assert np.array_equal(got, olp)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_topk_matches_torch_device_ops(dev, dtype):
    """The reference's own ops on the device, torch.topk(torch.log_softmax(x))
    (sampling.py:131-134): the same log-prob values, and the same tokens
    wherever a value is not tied (torch leaves the order of ties open)."""
    sampling = pkg("flashinfer_paged.sampling")
    gen = torch.Generator().manual_seed(21)
    x = _logits(gen, 9, 128256, dtype, 2.0).to(dev)
    lp, ids = sampling.batch_parent_token_candidates(x, k=8, sampling=None, relative_parent_paths=[()] * 9)
    tv, ti = torch.topk(torch.log_softmax(x, dim=-1), k=9, dim=-1)
    torch.cuda.synchronize()
    _assert_logprobs(lp, tv[:, :8].float().cpu().numpy(), dtype)
    tvf, tif = tv.float().cpu(), ti.cpu()
    for r in range(9):
        for j in range(8):
            v = tvf[r, j]
            if (tvf[r] == v).sum() == 1:
                assert int(ids[r, j]) == int(tif[r, j])


def _routes(types, n, roots=None):
    return [types.RouteState(route_id=10 + i, stage1_root_id=(roots[i] if roots else 10 + i), parent_route_id=None,
                             materialized_leaf_node_id=None, pending_token_id=0,
                             cumulative_logprob=float(-0.25 * (i % 3)), stage1_depth=0, stage2_depth=0,
                             kv_view=types.PrefixKVView(committed_length=1).fork())
            for i in range(n)]


def _oracle_cands(routes, olp, oids):
    return ofr.build_candidates([r.route_id for r in routes], [r.stage1_root_id for r in routes],
                                [r.cumulative_logprob for r in routes], olp, oids)


@pytest.mark.parametrize("policy", ["global", "per_root"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fused_depth_records_match_oracle(dev, policy, dtype):
    """One fused launch pair: the packed records (every column, float64 bits
    of the cumulative and parent log-probs, the selection order) and the
    candidate batch equal the oracle's candidates + order + selection."""
    fr = pkg("flashinfer_paged.frontier")
    types = pkg("flashinfer_paged.types")
    lib = pkg("_lib")
    gen = torch.Generator().manual_seed(7)
    rows, vocab, k = 12, 50000, 3
    roots = [1, 1, 2, 2, 2, 3, 1, 3, 2, 1, 3, 3] if policy == "per_root" else None
    routes = _routes(types, rows, roots)
    x = _logits(gen, rows, vocab, dtype, 0.3)
    sel_policy = fr.GlobalTopKSelection() if policy == "global" else fr.PerStage1RootTopKSelection()
    if policy == "global":
        mode, num, _ = sel_policy.device_selection(k=5, active_routes=routes)
        total = 5
    else:
        mode, num, total = sel_policy.device_selection(k=2, active_routes=routes, candidates_per_parent=k)
    batch, records, selected = fr._fused(routes, x.to(dev), k=k, sampling=None, relative_parent_paths=None,
                                         select_mode=mode, num_selected=num)
    torch.cuda.synchronize()
    olp, oids = ofr.parent_token_candidates(x.float().numpy(), k, DT[dtype])
    c = _oracle_cands(routes, olp, oids)
    if policy == "global":
        osel = ofr.select_global(c, 5)
    else:
        osel = ofr.select_per_root(c, 2, [(r, 3 * roots.count(r)) for r in set(roots)])
    rec, orec = records.cpu().numpy(), ofr.pack_records(c, osel)
    if dtype == torch.float32:  # cumulative log-probs to 1e-5 (see _assert_logprobs)
        assert np.abs(rec[:, 5].view(np.float64) - orec[:, 5].view(np.float64)).max() <= 1e-5
        rec, orec = np.delete(rec, 5, axis=1), np.delete(orec, 5, axis=1)
    assert np.array_equal(rec, orec)
    assert selected[:total].cpu().tolist() == osel.tolist()
    assert batch.candidate_count == rows * k and batch.candidates_per_parent == k
    assert np.abs(batch.cumulative_logprobs.cpu().numpy() - c["cumulative_logprobs"]).max() <= 1e-5
    assert np.array_equal(batch.parent_row_indices.cpu().numpy(), c["parent_row_indices"])
    assert mode in (lib.FRONTIER_SELECT_GLOBAL, lib.FRONTIER_SELECT_PER_ROOT)


def _device_batch(types, c, dev, strided=False):
    def col(a, dt):
        t = torch.as_tensor(a, dtype=dt)
        if strided:  # every other element of a longer buffer
            buf = torch.zeros(2 * len(a), dtype=dt)
            buf[::2] = t
            return buf.to(dev)[::2]
        return t.to(dev)
    return types.PendingCandidateBatch(
        parent_route_ids=col(c["parent_route_ids"], torch.long), stage1_root_ids=col(c["stage1_root_ids"], torch.long),
        parent_row_indices=col(np.arange(len(c["pending_token_ids"])), torch.long),
        pending_token_ids=col(c["pending_token_ids"], torch.long),
        cumulative_logprobs=col(c["cumulative_logprobs"], torch.float64),
        parent_logprobs=col(c["parent_logprobs"], torch.float64), ranks_in_parent=col(c["ranks_in_parent"], torch.long),
        candidates_per_parent=1)


@pytest.mark.parametrize("n,strided", [(1, False), (37, True), (700, False), (4096, False)])
def test_candidate_order_and_selection_match_oracle(dev, n, strided):
    """atlas_candidate_select on batches dense with exact ties (plus NaN and
    -0.0 scores): the full order (global and by root), both selections and the
    packing of a given selection equal the oracle's stable argsorts."""
    utils = pkg("flashinfer_paged.utils")
    types = pkg("flashinfer_paged.types")
    fr = pkg("flashinfer_paged.frontier")
    rng = np.random.default_rng(n)
    cum = rng.integers(-4, 1, n).astype(np.float64) * 0.5
    if n > 10:
        cum[rng.integers(0, n, 3)] = np.nan
        cum[rng.integers(0, n, 3)] = -0.0
    c = {"parent_route_ids": rng.integers(0, 6, n), "stage1_root_ids": rng.integers(0, 4, n),
         "pending_token_ids": rng.integers(0, 9, n), "ranks_in_parent": rng.integers(0, 3, n),
         "cumulative_logprobs": cum, "parent_logprobs": rng.normal(size=n)}
    c = {key: np.asarray(v) for key, v in c.items()}
    batch = _device_batch(types, c, dev, strided)
    order = utils.stable_candidate_order(batch)
    order_root = utils.stable_candidate_order(batch, include_stage1_root=True)
    top = utils.global_topk_candidate_indices(batch, num_selected=min(n, 5))
    roots, counts = np.unique(c["stage1_root_ids"], return_counts=True)
    root_counts = list(zip(roots.tolist(), counts.tolist()))
    per_root = utils.per_root_topk_candidate_indices(batch, num_selected=3, root_candidate_counts=root_counts)
    torch.cuda.synchronize()
    assert order.cpu().tolist() == ofr.stable_order(c).tolist()
    assert order_root.cpu().tolist() == ofr.stable_order(c, include_stage1_root=True).tolist()
    assert top.cpu().tolist() == ofr.select_global(c, min(n, 5)).tolist()
    assert per_root.cpu().tolist() == ofr.select_per_root(c, 3, root_counts).tolist()
    # pack a given selection, with node ids appended
    pick = torch.tensor(ofr.select_global(c, min(n, 4)), dtype=torch.long, device=dev)
    nodes = torch.tensor([5, 6, 7], dtype=torch.long, device=dev)
    _, _, recs = fr.candidate_select(batch, pkg("_lib").FRONTIER_PACK, selected_in=pick, node_ids=nodes, records=True)
    torch.cuda.synchronize()
    assert np.array_equal(recs.cpu().numpy(), ofr.pack_records(c, pick.cpu().numpy(), node_ids=[5, 6, 7]))


def _pc(types, *args, **kw):
    return types.PendingCandidate(*args, **kw)


def test_reference_selection_literals_on_device(dev):
    """test_paged_frontier_selection.py:79-130 with device tensors."""
    fr = pkg("flashinfer_paged.frontier")
    types = pkg("flashinfer_paged.types")
    cands = [_pc(types, 20, 200, 7, -1.0, rank_in_parent=0), _pc(types, 10, 100, 1, -1.0, rank_in_parent=1),
             _pc(types, 10, 100, 9, -1.0, rank_in_parent=0), _pc(types, 10, 100, 2, -1.0, rank_in_parent=0),
             _pc(types, 5, 500, 0, -1.0, rank_in_parent=2), _pc(types, 99, 900, 4, -0.5, rank_in_parent=3)]

    def batch(cs, per_parent):
        return types.PendingCandidateBatch(
            parent_route_ids=torch.tensor([x.parent_route_id for x in cs], device=dev),
            stage1_root_ids=torch.tensor([x.stage1_root_id for x in cs], device=dev),
            parent_row_indices=torch.arange(len(cs), device=dev),
            pending_token_ids=torch.tensor([x.pending_token_id for x in cs], device=dev),
            cumulative_logprobs=torch.tensor([x.cumulative_logprob for x in cs], dtype=torch.float64, device=dev),
            parent_logprobs=torch.tensor([x.parent_logprob for x in cs], dtype=torch.float64, device=dev),
            ranks_in_parent=torch.tensor([x.rank_in_parent for x in cs], device=dev),
            candidates_per_parent=per_parent)

    pol = fr.GlobalTopKSelection()
    idx = pol.select_indices(batch(cands, 1), k=len(cands), active_routes=[])
    actual = [cands[i] for i in idx.tolist()]
    assert actual == fr.global_topk_candidates(cands, num_selected=len(cands))
    assert [x.pending_token_id for x in actual] == [4, 0, 2, 9, 1, 7]
    cands = [_pc(types, 20, 200, 8, -1.0, rank_in_parent=0), _pc(types, 20, 200, 3, -1.0, rank_in_parent=1),
             _pc(types, 10, 100, 9, -1.0, rank_in_parent=0), _pc(types, 10, 100, 4, -1.0, rank_in_parent=1),
             _pc(types, 21, 200, 7, -1.0, rank_in_parent=0), _pc(types, 21, 200, 2, -1.0, rank_in_parent=1),
             _pc(types, 11, 100, 6, -1.0, rank_in_parent=0), _pc(types, 11, 100, 1, -1.0, rank_in_parent=1)]
    routes = [types.RouteState(route_id=r, stage1_root_id=root, parent_route_id=None, materialized_leaf_node_id=None,
                               pending_token_id=0, cumulative_logprob=0.0, stage1_depth=0, stage2_depth=0,
                               kv_view=types.PrefixKVView(committed_length=1).fork())
              for r, root in ((20, 200), (10, 100), (21, 200), (11, 100))]
    pol = fr.PerStage1RootTopKSelection()
    idx = pol.select_indices(batch(cands, 2), k=2, active_routes=routes)
    actual = [cands[i] for i in idx.tolist()]
    assert actual == pol.select(cands, k=2, active_routes=routes)
    assert [x.stage1_root_id for x in actual] == [100, 100, 200, 200]
    assert [x.parent_route_id for x in actual] == [10, 10, 20, 20]
    # materialisation keeps the parent log-prob (:258-275)
    one = _pc(types, 7, 3, 11, -4.5, rank_in_parent=2, parent_logprob=-3.25)
    mat, sel, _, stats = fr.materialize_pending_candidate_batch(batch([one], 1), torch.tensor([0], device=dev))
    assert mat == [one] and sel == [one] and stats.host_materialization_batches == 1


class _ReservingBackend:
    def __init__(self, store, logits):
        self.store, self.logits = store, logits

    def decode_frontier_one_token(self, active_routes, attention_backend=None):
        types = pkg("flashinfer_paged.types")
        ids = self.store.reserve_node_ids(len(active_routes))
        return types.FrontierDecodeOutput(route_ids=torch.tensor([r.route_id for r in active_routes]),
                                          next_token_logits=self.logits.clone(),
                                          new_node_ids=torch.tensor(ids, dtype=torch.long))


class _TensorOnlyNodeBackend:
    def __init__(self, logits):
        self.logits = logits

    def decode_frontier_one_token(self, active_routes, attention_backend=None):
        types = pkg("flashinfer_paged.types")
        return types.FrontierDecodeOutput(route_ids=torch.tensor([r.route_id for r in active_routes]),
                                          next_token_logits=self.logits.clone(),
                                          new_node_ids=torch.tensor([101, 102], dtype=torch.long))


def _registered_routes(store, types):
    out = []
    for token in (3, 4):
        rid = store.allocate_route_id()
        out.append(store.register_route(types.RouteState(
            route_id=rid, stage1_root_id=rid, parent_route_id=None, materialized_leaf_node_id=None,
            pending_token_id=token, cumulative_logprob=0.0, stage1_depth=0, stage2_depth=0,
            kv_view=types.PrefixKVView(committed_length=1).fork())))
    return out


def test_frontier_depth_flows(dev):
    """test_paged_frontier_selection.py:189-255 on the device: one packed
    materialisation per depth, node ids from the store counter or from the
    packed transfer, the selection equal to the host-object selection."""
    fr = pkg("flashinfer_paged.frontier")
    kv = pkg("flashinfer_paged.kv")
    types = pkg("flashinfer_paged.types")
    store = kv.KVTreeStore()
    active = _registered_routes(store, types)
    logits = torch.tensor([[0.0, 3.0, 3.0, 0.0, 0.0], [0.0, 3.0, 3.0, 0.0, 0.0]], device=dev)
    step = fr.advance_frontier_one_token(active, k=2, route_store=store,
                                         model_backend=_ReservingBackend(store, logits),
                                         selection_policy=fr.GlobalTopKSelection(phase=types.DecodePhase.STAGE1))
    assert len(step.candidates) == 4 and len(step.selected_candidates) == 2
    assert step.selected_candidates == fr.global_topk_candidates(step.candidates, num_selected=2)
    assert sorted(store.nodes) == [1, 2]
    st = step.selection_stats
    assert (st.candidate_count, st.selected_count, st.host_materialization_batches) == (4, 2, 1)
    assert st.host_materialization_elements == 4 * 8 and st.host_transfer_batches == 1
    assert st.new_node_ids_source == "route_store_counter"
    assert [r.pending_token_id for r in step.next_routes] == [1, 2]
    assert all(r.parent_route_id == active[0].route_id for r in step.next_routes)

    store = kv.KVTreeStore()
    active = _registered_routes(store, types)
    logits = torch.tensor([[0.0, 2.0, 1.0], [0.0, 2.0, 1.0]], device=dev)
    step = fr.advance_frontier_one_token(active, k=2, route_store=store, model_backend=_TensorOnlyNodeBackend(logits),
                                         selection_policy=fr.GlobalTopKSelection())
    assert sorted(store.nodes) == [101, 102]
    assert step.selection_stats.host_materialization_elements == (4 + 2) * 8
    assert step.selection_stats.new_node_ids_source == "packed_transfer"


def test_frontier_depth_per_root_and_custom_policy(dev):
    """A stage-2 depth with PerStage1RootTopKSelection (fused selection) and the
    same depth through a policy object the launch does not know (batch, its
    select_indices, then the packing launch): the same routes come out."""
    fr = pkg("flashinfer_paged.frontier")
    kv = pkg("flashinfer_paged.kv")
    types = pkg("flashinfer_paged.types")
    gen = torch.Generator().manual_seed(5)
    logits = (torch.randn((4, 3000), generator=gen) * 2).to(torch.bfloat16).to(dev)

    class Wrapped:
        phase = types.DecodePhase.STAGE2

        def __init__(self):
            self.inner = fr.PerStage1RootTopKSelection()

        def select(self, *a, **kw):
            return self.inner.select(*a, **kw)

        def select_indices(self, *a, **kw):
            return self.inner.select_indices(*a, **kw)

    outs = []
    for policy in (fr.PerStage1RootTopKSelection(), Wrapped()):
        store = kv.KVTreeStore()
        active = []
        for i, root in enumerate((1, 2, 1, 2)):
            rid = store.allocate_route_id()
            active.append(store.register_route(types.RouteState(
                route_id=rid, stage1_root_id=root, parent_route_id=None, materialized_leaf_node_id=None,
                pending_token_id=5 + i, cumulative_logprob=-0.5 * i, stage1_depth=1, stage2_depth=0,
                kv_view=types.PrefixKVView(committed_length=3).fork())))
        step = fr.advance_frontier_one_token(active, k=3, route_store=store,
                                             model_backend=_ReservingBackend(store, logits), selection_policy=policy)
        assert step.selected_candidates == policy.select(step.candidates, k=3, active_routes=active)
        outs.append([(r.stage1_root_id, r.pending_token_id, r.cumulative_logprob) for r in step.next_routes])
    assert outs[0] == outs[1] and len(outs[0]) == 6


def test_sampling_path_matches_oracle(dev):
    """do_sample: the Gumbel proposal drawn per parent exactly as the
    reference draws it; the kernels take its top-k and gather the model
    log-probs -- equal to the oracle on the same proposal; the draw depends
    on the parent's semantic path only (sampling.py:51-86)."""
    sampling = pkg("flashinfer_paged.sampling")
    gen = torch.Generator().manual_seed(9)
    x = _logits(gen, 3, 20000, torch.bfloat16, 1.0).to(dev)
    ctx = sampling.DrafterSamplingContext(sampling.DrafterSamplingConfig(do_sample=True, seed=4, temperature=0.7),
                                          committed_token_ids=(1, 2, 3))
    paths = [(5,), (6, 7), ()]
    lp, ids = sampling.batch_parent_token_candidates(x, k=4, sampling=ctx, relative_parent_paths=paths)
    prop = sampling.gumbel_proposal(x, ctx, paths)
    torch.cuda.synchronize()
    olp, oids = ofr.parent_token_candidates(x.float().cpu().numpy(), 4, "bf16", proposal=prop.cpu().numpy())
    assert np.array_equal(ids.cpu().numpy(), oids)
    assert np.array_equal(lp.float().cpu().numpy(), olp)
    # same path, other batch position -> same draw
    lp2, ids2 = sampling.batch_parent_token_candidates(x[[1]], k=4, sampling=ctx, relative_parent_paths=[(6, 7)])
    assert torch.equal(ids2[0], ids[1])


def test_frontier_refusals(dev):
    """Errors of the frontier entry points: CPU tensors, k above 32, more
    than 4096 candidates with selection, mismatched batch sizes."""
    sampling = pkg("flashinfer_paged.sampling")
    fr = pkg("flashinfer_paged.frontier")
    types = pkg("flashinfer_paged.types")
    x = torch.randn((2, 100))
    with pytest.raises(RuntimeError):
        sampling.batch_parent_token_candidates(x, k=2, sampling=None, relative_parent_paths=[(), ()])
    with pytest.raises(NotImplementedError):
        sampling.batch_parent_token_candidates(x.to(dev), k=33, sampling=None, relative_parent_paths=[(), ()])
    with pytest.raises(ValueError):
        sampling.batch_parent_token_candidates(x.to(dev), k=0, sampling=None, relative_parent_paths=[(), ()])
    big = torch.randn((200, 64), device=dev)
    with pytest.raises(NotImplementedError):
        fr.build_pending_candidate_batch(_routes(types, 200), big, k=32)
    with pytest.raises(ValueError):
        fr.build_pending_candidate_batch(_routes(types, 3), x.to(dev), k=2)


def test_frontier_edge_shapes(dev):
    """Edge shapes of one depth: a single parent, vocab below the chunk size
    and equal to k, rows with a stride wider than the vocabulary (a slice of
    a bigger tensor, 16-byte aligned and not), a row of equal logits (ties
    everywhere), -inf logits, records without a selection (order column -1)
    with node ids appended."""
    sampling = pkg("flashinfer_paged.sampling")
    fr = pkg("flashinfer_paged.frontier")
    types = pkg("flashinfer_paged.types")
    gen = torch.Generator().manual_seed(3)

    def check(x, k, dt="f32"):
        lp, ids = sampling.batch_parent_token_candidates(x.to(dev) if x.device.type == "cpu" else x, k=k,
                                                         sampling=None, relative_parent_paths=[()] * x.shape[0])
        olp, oids = ofr.parent_token_candidates(x.float().cpu().numpy(), k, dt)
        assert np.array_equal(ids.cpu().numpy(), oids)
        got = lp.float().cpu().numpy()
        if dt == "f32":
            assert np.allclose(got, olp, atol=1e-5, rtol=0, equal_nan=True)
        else:
            assert np.array_equal(got, olp)

    check(torch.randn((1, 3), generator=gen), 3)
    check(torch.randn((2, 7), generator=gen), 5)
    big = (torch.randn((4, 1000), generator=gen) * 2).half().to(dev)
    check(big[:, :640], 4, "f16")       # stride 1000 elements: rows 16-byte aligned
    check(big[:, 3:650], 4, "f16")      # rows start 6 bytes in: element loads
    flat = torch.zeros((3, 5000), dtype=torch.bfloat16)
    check(flat, 6, "bf16")              # all equal: tokens 0..5
    ninf = torch.randn((2, 300), generator=gen)
    ninf[:, ::2] = float("-inf")
    check(ninf, 3)
    routes = [types.RouteState(route_id=5 + i, stage1_root_id=1, parent_route_id=None, materialized_leaf_node_id=None,
                               pending_token_id=0, cumulative_logprob=0.5 * i, stage1_depth=0, stage2_depth=0,
                               kv_view=types.PrefixKVView(committed_length=1).fork()) for i in range(3)]
    x = torch.randn((3, 900), generator=gen).to(dev)
    batch, records, _ = fr._fused(routes, x, k=2, sampling=None, relative_parent_paths=None,
                                  node_ids=torch.tensor([41, 42, 43]))
    torch.cuda.synchronize()
    rec = records.cpu().numpy()
    assert rec.shape == (6 + 3, 8) and (rec[:6, 7] == -1).all()
    assert rec[6:, :2].tolist() == [[1, 41], [1, 42], [1, 43]] and (rec[6:, 2:] == 0).all()
    assert rec[:6, 1].tolist() == [5, 5, 6, 6, 7, 7] and rec[:6, 4].tolist() == [0, 1] * 3
