"""Route scoring kernel vs the oracle, Target commit/scoring drop-in methods,
and HIP-graph replays of the verify forward vs its eager result."""

import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import bits16, pkg
from oracle import paged_kv as ref
from oracle import scoring as osc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_gather_logprobs_matches_oracle(dev, dtype):
    tr = pkg("target_runtime")
    gen = torch.Generator().manual_seed(0)
    logits = (torch.randn((36, 128256), generator=gen) * 3).to(dtype)
    rows = [int(x) for x in torch.randint(0, 36, (40,), generator=gen)]
    toks = [int(x) for x in torch.randint(0, 128256, (40,), generator=gen)]
    out = tr.gather_token_logprobs(logits.to(dev), rows, toks).cpu().numpy()
    lp = osc.log_softmax(logits.double().numpy())
    exp = np.array([lp[r, t] for r, t in zip(rows, toks)])
    assert np.abs(out - exp).max() <= 2e-4  # fp32 accumulation over 128256 logits


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape,offset", [((7, 1003), 0), ((5, 1001), 1), ((3, 9), 1)])
def test_gather_logprobs_unaligned_and_ragged_rows(dev, dtype, shape, offset):
    """Row starts that are not 16-byte aligned (scalar path) and vocabularies
    that are not a multiple of the vector width (vector path tail)."""
    tr = pkg("target_runtime")
    gen = torch.Generator().manual_seed(shape[1] + offset)
    full = (torch.randn((shape[0], shape[1] + offset), generator=gen) * 4).to(dtype)
    logits = full[:, offset:]
    rows = [r % shape[0] for r in range(11)]
    toks = [int(x) for x in torch.randint(0, shape[1], (11,), generator=gen)]
    out = tr.gather_token_logprobs(logits.to(dev) if offset == 0 else full.to(dev)[:, offset:], rows, toks)
    lp = osc.log_softmax(logits.double().numpy())
    exp = np.array([lp[r, t] for r, t in zip(rows, toks)])
    assert np.abs(out.cpu().numpy() - exp).max() <= 2e-5


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gather_logprobs_two_logits_tensors_in_one_launch(dev, dtype):
    """Rows of a second logits tensor (the prefix logits) follow the first
    tensor's rows in one launch; repeated calls reuse the workspace (left
    zero by each call) and give the same values bit for bit; out-of-range
    tokens give NaN."""
    tr = pkg("target_runtime")
    gen = torch.Generator().manual_seed(3)
    verify = (torch.randn((34, 128256), generator=gen) * 3).to(dtype)
    prefix = (torch.randn((128256,), generator=gen) * 3).to(dtype)
    rows = [34] * 9 + [int(x) for x in torch.randint(0, 34, (27,), generator=gen)] + [5]
    toks = [int(x) for x in torch.randint(0, 128256, (36,), generator=gen)] + [128256]
    first = tr.gather_token_logprobs(verify.to(dev), rows, toks, extra_logits=prefix.to(dev)).cpu()
    again = tr.gather_token_logprobs(verify.to(dev), rows, toks, extra_logits=prefix.to(dev)).cpu()
    assert torch.equal(first.view(torch.int32), again.view(torch.int32))
    lp = osc.log_softmax(torch.cat((verify, prefix[None])).double().numpy())
    exp = np.array([lp[r, t] for r, t in zip(rows[:-1], toks[:-1])])
    assert np.abs(first[:-1].numpy() - exp).max() <= 2e-4
    assert math.isnan(float(first[-1]))


def _backend(tr, **attrs):
    b = object.__new__(tr.DirectFlashInferMaskedTreeVerifyBackend)
    b.score_weights = None
    b.route_selection_policy = "target_best"
    b.route_sampling_temperature = 1.0
    b.match_logits_dtype_rounding = True
    for k, v in attrs.items():
        setattr(b, k, v)
    return b


def test_score_routes_reference_literal(dev):
    # tests/test_target_kv_commit.py:76-103 (float32 logits)
    tr = pkg("target_runtime")
    b = _backend(tr)
    prefix = torch.tensor([0.0, 3.0, 0.0, 0.0], device=dev)
    verify = torch.tensor([[0.0, 0.0, 4.0, 2.0], [0, 0, 0, 0], [0, 0, 0, 0]], device=dev)
    routes = [tr.VerifyRoutePayload(1, (1, 2), -1.0), tr.VerifyRoutePayload(2, (1, 3), -2.0)]
    scores = b._score_routes(routes=routes, paths=[r.token_ids for r in routes], prefix_logits=prefix,
                             verify_logits=verify, route_to_node_paths=[[0, 1], [0, 2]])
    plp = torch.log_softmax(prefix.cpu(), -1)[1].item()
    vlp = torch.log_softmax(verify[0].cpu(), -1)
    assert abs(scores[0].target_logprob - (plp + vlp[2].item())) < 1e-6
    assert abs(scores[1].target_logprob - (plp + vlp[3].item())) < 1e-6
    assert b._select_route(scores).route_id == 1


def test_score_routes_forest_matches_oracle_and_selection(dev):
    tr = pkg("target_runtime")
    wl = pkg("workloads")
    b = _backend(tr)
    routes = wl.forest_routes(3)
    _, _, _, nodes = ref.dedup_tree(routes)
    n = max(max(x) for x in nodes) + 1
    gen = torch.Generator().manual_seed(1)
    verify = (torch.randn((n, 128256), generator=gen) * 2).half()
    prefix = (torch.randn((128256,), generator=gen) * 2).half()
    # plant the scored tokens so the routes differ clearly
    payloads = [tr.VerifyRoutePayload(i, r, -float(i)) for i, r in enumerate(routes)]
    scores = b._score_routes(routes=payloads, paths=routes, prefix_logits=prefix.to(dev), verify_logits=verify.to(dev),
                             route_to_node_paths=nodes)
    # the reference reads fp16 log_softmax outputs: compare to the oracle rounded the same way
    lps = osc.route_token_logprobs(routes, nodes, prefix.double().numpy(), verify.double().numpy())
    for s, exact in zip(scores, lps):
        rounded = np.array(exact, dtype=np.float16).astype(np.float64)
        assert np.abs(np.array(s.token_logprobs) - rounded).max() <= 2e-3
        assert np.abs(np.array(s.token_logprobs) - np.array(exact)).max() <= 2e-3 + 2 ** -7
    best = osc.select_best([dict(route_id=s.route_id, selection_score=s.selection_score,
                                 draft_path_logprob=s.draft_path_logprob, token_ids=s.token_ids) for s in scores])
    assert b._select_route(scores).route_id == best["route_id"]


@pytest.mark.parametrize("layout", ["NHD", "HND"])
def test_commit_selected_path_reference_literal(dev, layout):
    # tests/test_target_kv_commit.py:13-45 on fp16 rows (D = 8 for 16-byte
    # rows, two KV heads), in the reference's NHD pages and in HND pages
    tr = pkg("target_runtime")
    b = _backend(tr, kv_layout=layout)
    b.config = SimpleNamespace(page_size=4)
    b.prefix_token_ids = (1, 2, 3)
    b._prefix_logits = torch.zeros((1, 8), device=dev)
    b._committed_verify_rounds = 0
    cache = torch.zeros((2, 2, 4, 2, 8), dtype=torch.float16)
    for pos in range(8):
        page, off = divmod(pos, 4)
        cache[page, 0, off] = 100 + pos + torch.tensor([[0.0], [0.5]])
        cache[page, 1, off] = 200 + pos + torch.tensor([[0.0], [0.5]])
    as_layout = (lambda t: t) if layout == "NHD" else (lambda t: t.permute(0, 1, 3, 2, 4))
    b._paged_prefix_kv = [as_layout(cache).contiguous().to(dev)]
    logits = torch.arange(32, dtype=torch.float32, device=dev).reshape(4, 8)
    b._commit_selected_path(token_ids=(9, 10), node_ids=(0, 2), verify_logits=logits)
    c = as_layout(b._paged_prefix_kv[0].cpu())  # back to NHD indexing
    for h, add in ((0, 0.0), (1, 0.5)):
        assert c[0, 0, 3, h, 0].item() == 103 + add and c[1, 0, 0, h, 0].item() == 105 + add
        assert c[0, 1, 3, h, 0].item() == 203 + add and c[1, 1, 0, h, 0].item() == 205 + add
    assert b.prefix_token_ids == (1, 2, 3, 9, 10)
    assert torch.equal(b._prefix_logits, logits[2].unsqueeze(0))
    assert b._committed_verify_rounds == 1
    b._ensure_page_capacity(4)
    assert b._paged_prefix_kv[0].shape[0] == 4 and torch.equal(as_layout(b._paged_prefix_kv[0][:2].cpu()), c)
    with pytest.raises(ValueError):
        b._commit_selected_path(token_ids=(1,), node_ids=(), verify_logits=logits)


def test_graph_replays_match_eager_forward(dev):
    """Capture append + attention over 4 layers, replay it several times with
    eager work and synchronisations in between; every replay equals eager."""
    ffv = pkg("flashinfer_full_verify")
    kv_ops = pkg("kv_ops")
    wl = pkg("workloads")
    geom = wl.Geometry(4, 32, 8, 128)
    routes = wl.forest_routes(1)
    prefix_len, ps = 3000, 16
    spec, _ = ffv.build_deduplicated_tree_spec_from_paths(paths=routes, prefix_len=prefix_len, page_size=ps, device=dev)
    n = spec.node_count
    kv = wl.make_paged_target_kv(geom, kv_len=prefix_len + n, page_size=ps, dtype=torch.float16, device=dev,
                                 seed=3, spare_pages=9)
    layers = kv.layers
    q = wl.random_queries(geom, n, dtype=torch.float16, device=dev, seed=4)
    g = torch.Generator(device=dev).manual_seed(5)
    kn = [(torch.randn((n, 8, 128), generator=g, device=dev) * 0.1).half() for _ in range(4)]
    vn = [(torch.randn((n, 8, 128), generator=g, device=dev) * 0.1).half() for _ in range(4)]
    pages = math.ceil((prefix_len + n) / ps)
    idx = kv.kv_indices.cpu().long()
    pos = torch.arange(prefix_len, prefix_len + n)
    slots = (idx[pos // ps] * ps + pos % ps).to(dev)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    w = ffv.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")

    def plan():
        w.plan(spec.qo_indptr, torch.tensor([0, pages], dtype=torch.int32, device=dev), kv.kv_indices,
               torch.tensor([prefix_len + n - (pages - 1) * ps], dtype=torch.int32, device=dev), 32, 8, 128, ps,
               custom_mask=spec.bool_mask, q_data_type=torch.float16)

    outs = [torch.empty_like(x) for x in q]

    def forward():
        for l in range(4):
            kv_ops.append_paged([layers[l]], [kn[l]], [vn[l]], dst_slots=slots)
            w.run(q[l], layers[l], out=outs[l])

    plan()
    forward()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    eager_kv = kv.pool.clone()
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
        plan()  # re-plan into the persistent buffers between replays
        scratch = torch.randn(1 << 20, device=dev).sum()  # unrelated eager work
        graph.replay()
        torch.cuda.synchronize()
        assert float(scratch) == float(scratch)
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {rep} differs from eager"
        assert torch.equal(kv.pool, eager_kv)


def test_gather_logprobs_graph_replays(dev):
    """The scoring launch through the C ABI, twice in one HIP graph over
    device index buffers and one shared workspace, replayed with new logits
    copied in between: every replay equals an eager launch on the same logits
    bit for bit (so each launch leaves the workspace zero for the next), and
    the values are within 2e-3 of the oracle."""
    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    vocab, rows1 = 128256, 34
    gen = torch.Generator().manual_seed(21)
    verify = torch.empty((rows1, vocab), dtype=torch.bfloat16, device=dev)
    prefix = torch.empty((1, vocab), dtype=torch.bfloat16, device=dev)
    row_list = [rows1] * 9 + [int(x) for x in torch.randint(0, rows1, (27,), generator=gen)]
    tok_list = [int(x) for x in torch.randint(0, vocab, (36,), generator=gen)]
    rows = torch.tensor(row_list, dtype=torch.int32, device=dev)
    toks = torch.tensor(tok_list, dtype=torch.int64, device=dev)
    n = len(row_list)
    need = int(lib.atlas_gather_logprobs_workspace_bytes(rows1 + 1, vocab))
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    outs = [torch.empty(n, dtype=torch.float32, device=dev) for _ in range(3)]

    def launch(out):
        rc = lib.atlas_gather_logprobs(lib_mod.ptr(verify), vocab, rows1, lib_mod.ptr(prefix), vocab, 1, vocab,
                                       lib_mod.dtype_code(torch.bfloat16), lib_mod.ptr(rows), lib_mod.ptr(toks), n,
                                       None, lib_mod.ptr(out), lib_mod.ptr(ws), need, lib_mod.stream_of(dev))
        lib_mod.check(rc, "atlas_gather_logprobs")

    def fill(seed):
        g = torch.Generator().manual_seed(seed)
        verify.copy_((torch.randn((rows1, vocab), generator=g) * 3).to(torch.bfloat16))
        prefix.copy_((torch.randn((1, vocab), generator=g) * 3).to(torch.bfloat16))

    fill(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch(outs[0])
        launch(outs[1])
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch(outs[0])
        launch(outs[1])
    for rep in range(4):
        fill(100 + rep)
        launch(outs[2])  # eager, same logits
        torch.cuda.synchronize()
        eager = outs[2].clone()
        outs[0].zero_()
        outs[1].zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(outs[0], eager) and torch.equal(outs[1], eager), f"replay {rep} differs from eager"
        assert int(ws.sum()) == 0
        if rep == 0:
            lp_v = osc.log_softmax(verify.float().cpu().double().numpy())
            lp_p = osc.log_softmax(prefix.float().cpu().double().numpy())
            exp = np.array([lp_p[0, t] if r == rows1 else lp_v[r, t] for r, t in zip(row_list, tok_list)])
            assert np.abs(eager.cpu().numpy() - exp).max() <= 2e-3
