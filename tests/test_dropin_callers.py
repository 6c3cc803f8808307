"""The reference runtime's own call sequences into this package's drop-ins,
replayed by stand-in callers (``standin_callers.py``; the reference is not
imported).

Target (``src/atlas_0709/rpc.py:66-160``): health -> prefill -> verify ->
the ``target_verify_result_to_dict`` fields, through JSON.  The keys and the
static values of ``runtime_metadata()`` are pinned against the health
metadata the reference itself recorded (``tests/golden/target_health_metadata.json``,
from ``atlas_0709_e2e_smoke.json``) and the key list of
``target_runtime.py:322-359``; the verify metadata's keys against
``target_runtime.py:235-320``.  The CPU suite has no GPU, so the device steps
(the prefill's paged layout; a verify's wrapper plan, masked tree forward,
log-prob gather and KV commit) are replaced here by CPU stand-ins: a row copy
into pages, a dense causal forward of the same model per tree node,
``log_softmax`` and a gather-then-scatter of the paged rows.
``tests/test_gpu_target_model.py`` runs the same sequence on the device with
nothing replaced.

Drafter (``src/atlas_0709/distributed_system.py:639-660``, ``:707-735``):
``from_runner`` on a runner holding host pools, prompt prefill, a frontier
step, then the fallback handoff (``retain_route_rows([])``, prune,
``reset_speculative``, ``append_known_tokens_as_prefix``); and the path a
runner-backed executor takes (the reference's ``SGLangFlashInferPagedDecodeBackend``
has no ``forward_extend``): the EXTEND ``ForwardBatch`` fields of
``sglang_runtime.py:1211-1235``, through stand-in reference helpers.
"""

import json
import math
import sys
from pathlib import Path
from types import ModuleType, SimpleNamespace

import pytest
import torch

from helpers import pkg
from oracle.route_pool import OracleAllocator, OracleReqPool
from standin_callers import (
    RUNTIME_METADATA_KEYS, VERIFY_COMMON_KEYS, VERIFY_FALLBACK_KEYS, VERIFY_SELECT_KEYS, TargetRpcStandIn,
    edge_decision_metadata, edge_fallback_handoff, edge_prepare_prefix,
)

GOLDEN = Path(__file__).resolve().parent / "golden" / "target_health_metadata.json"
VOCAB = 97


def _tiny_llama(seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(seed)
    cfg = LlamaConfig(vocab_size=VOCAB, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=16, max_position_embeddings=256,
                      attn_implementation="eager")
    return LlamaForCausalLM(cfg).float().eval()


class _Tok:
    bos_token_id, eos_token_id, pad_token_id = 1, 2, None

    def __len__(self):
        return VOCAB


def _dense_node_logits(model, prefix, tree):
    """Logits after each tree node: a dense causal forward of the prefix and
    the node's ancestor path."""
    toks = tree.flat_token_ids.tolist()
    rows = []
    for i in range(tree.node_count):
        path, j = [], i
        while j >= 0:
            path.append(int(toks[j]))
            j = tree.parent_indices[j]
        ids = torch.tensor([list(prefix) + path[::-1]])
        rows.append(model(input_ids=ids).logits[0, -1])
    return torch.stack(rows)


@pytest.fixture
def cpu_target(monkeypatch):
    """A Target backend on a CPU model with the device steps of a verify
    replaced by CPU stand-ins (see the module docstring)."""
    tr = pkg("target_runtime")
    model = _tiny_llama()
    state = {}

    def run_full_verify(*, model, wrapper, state: SimpleNamespace, prefix_len, page_size, fused=None):
        return _dense_node_logits(model, backend.prefix_token_ids, state.tree)

    def gather(logits, rows, tokens, extra_logits=None):
        lg = torch.cat([logits.reshape(-1, logits.shape[-1]), extra_logits.reshape(-1, logits.shape[-1])])
        lp = torch.log_softmax(lg.float(), dim=-1)
        return lp[torch.tensor(rows), torch.tensor(tokens)]

    def layout(*, key, value, prefix_len, node_count, page_size, kv_layout="NHD"):
        assert kv_layout == "NHD"  # the configuration below asks for the reference's pages
        pages = math.ceil((prefix_len + node_count) / page_size)
        out = torch.zeros((pages, 2, page_size, key.shape[1], key.shape[3]), dtype=key.dtype)
        for pos in range(prefix_len):
            out[pos // page_size, 0, pos % page_size] = key[0, :, pos]
            out[pos // page_size, 1, pos % page_size] = value[0, :, pos]
        return out

    def commit(layers, src, dst, kv_layout="NHD"):
        assert kv_layout == "NHD"
        for kv in layers:
            ps = kv.shape[2]
            rows = [kv[s // ps, :, s % ps].clone() for s in src]
            for d, r in zip(dst, rows):
                kv[d // ps, :, d % ps] = r

    monkeypatch.setattr(tr, "prefix_layer_to_paged_kv", layout)
    monkeypatch.setattr(tr, "make_prefill_wrapper", lambda **kw: SimpleNamespace())
    monkeypatch.setattr(tr, "plan_prefill_wrapper", lambda *a, **kw: None)
    monkeypatch.setattr(tr, "run_full_verify", run_full_verify)
    monkeypatch.setattr(tr, "gather_token_logprobs", gather)
    monkeypatch.setattr(tr.kv_ops, "commit_paged", commit)
    cfg = SimpleNamespace(k=3, d=3, page_size=4, device="cpu", dtype="float32", workspace_mb=1,
                          flashinfer_backend="auto", use_packed_custom_mask=False, kv_layout="NHD")

    def make(**kw):
        nonlocal backend
        backend = tr.DirectFlashInferMaskedTreeVerifyBackend(model_path="/models/tiny-llama", config=cfg, model=model,
                                                             tokenizer=_Tok(), **kw)
        return backend

    backend = None
    state["make"] = make
    state["tr"] = tr
    state["model"] = model
    return SimpleNamespace(**state)


def test_runtime_metadata_matches_the_reference_health_record(cpu_target):
    golden = json.loads(GOLDEN.read_text())["target_health"]["metadata"]
    backend = cpu_target.make()
    app = TargetRpcStandIn(backend, cpu_target.tr.verify_payload_from_mapping)
    health = app.health()
    meta = health["metadata"]
    assert health["ok"] is True
    assert tuple(meta) == RUNTIME_METADATA_KEYS
    assert set(golden) <= set(meta)
    for key in ("backend", "custom_mask", "deduplicated_tree_nodes", "logits_aligned", "packed_custom_mask",
                "paged_kv", "persistent_target_paged_kv", "rope_applied", "runtime_alignment_checked",
                "semantic_correctness_required", "committed_prefix_length", "committed_verify_rounds", "page_size"):
        if key == "page_size":
            continue
        assert meta[key] == golden[key], key
    # configuration-derived values follow the configuration
    assert meta["page_size"] == 4 and meta["dtype"] == "float32" and meta["device"] == "cpu"
    assert meta["model"] == "/models/tiny-llama" and meta["model_vocab_size"] == VOCAB
    assert meta["tokenizer_vocab_size"] == VOCAB and meta["tokenizer_eos_token_id"] == 2
    assert meta["selection_policy"] == "best_of_n_target_path_logprob"
    assert meta["route_selection_policy"] == "target_best"
    assert meta["score_weights"] is None and meta["fallback_ar_sampling"] == "greedy_argmax"
    assert isinstance(meta["flashinfer_version"], str)
    weighted = cpu_target.make(score_weights=[2.0, 1.0, 1.0], route_selection_policy="target_sample")
    wm = weighted.runtime_metadata()
    assert wm["score_weights"] == [0.5, 0.25, 0.25]
    assert wm["selection_policy"] == "sample_weighted_target_route_score_distribution"
    assert wm["route_selection_policy"] == "target_sample"


def test_rpc_sequence_prefill_verify_commit(cpu_target):
    backend = cpu_target.make()
    app = TargetRpcStandIn(backend, cpu_target.tr.verify_payload_from_mapping)
    prompt = [5, 9, 14, 3, 7, 11]
    pre = app.prefill({"prompt_token_ids": prompt})
    assert pre == {"ok": True, "prompt_len": 6, "metadata": pre["metadata"]}
    assert tuple(pre["metadata"]) == RUNTIME_METADATA_KEYS
    assert pre["metadata"]["committed_prefix_length"] == 6 and pre["metadata"]["committed_verify_rounds"] == 0
    # the prefix logits are the model's own last-token logits
    dense = cpu_target.model(input_ids=torch.tensor([prompt])).logits[0, -1]
    assert torch.allclose(backend._prefix_logits[0], dense, atol=1e-5)
    assert len(backend._paged_prefix_kv) == 2 and backend._paged_prefix_kv[0].shape[1:] == (2, 4, 2, 16)

    routes = [{"route_id": 10, "token_ids": [20, 21, 22], "draft_logprob": -1.0,
               "draft_token_logprobs": [-0.2, -0.3, -0.5]},
              {"route_id": 11, "token_ids": [20, 21, 30], "draft_logprob": -0.5,
               "draft_token_logprobs": [-0.1, -0.1, -0.3]},
              {"route_id": 12, "token_ids": [40, 41, 42], "draft_logprob": -2.0}]
    out = app.verify({"prefix_token_ids": prompt, "routes": routes})
    assert out["ok"] is True and out["decision"] == "select"
    meta = out["metadata"]
    for key in RUNTIME_METADATA_KEYS + VERIFY_COMMON_KEYS + VERIFY_SELECT_KEYS:
        assert key in meta, key
    assert meta["node_count"] == 7 and meta["unmerged_path_node_count"] == 9 and meta["prefix_len_before"] == 6
    assert meta["selection_score_name"] == "target_logprob"
    # the scores are the dense model's log-probs of each route token
    lp = {}
    for r in routes:
        ids = prompt + r["token_ids"]
        logits = cpu_target.model(input_ids=torch.tensor([ids])).logits[0]
        lps = torch.log_softmax(logits.float(), -1)
        lp[r["route_id"]] = [float(lps[len(prompt) - 1 + t, ids[len(prompt) + t]].detach()) for t in range(3)]
    by_id = {s["route_id"]: s for s in out["scores"]}
    for rid, want in lp.items():
        assert by_id[rid]["token_logprobs"] == pytest.approx(want, abs=1e-4)
    best = max(out["scores"], key=lambda s: (s["target_logprob"], s["draft_path_logprob"], -s["route_id"]))
    assert out["selected_route_id"] == best["route_id"] == meta["best_route_id"] == meta["selected_route_id"]
    assert out["selected_score"] == best
    assert meta["best_selection_score"] == pytest.approx(best["target_logprob"])
    assert meta["selected_selection_score"] == meta["best_selection_score"]
    assert meta["route0_route_id"] == 10 and meta["draft_top_route_id"] == 11
    assert meta["prefix_len_after"] == 9 and meta["target_kv_commit"] == "selected_tree_path_in_place"
    assert meta["committed_prefix_length"] == 6  # the runtime metadata taken before the commit
    decision = edge_decision_metadata(meta)
    assert decision["route_intervention"]["selected"]["route_id"] == best["route_id"]
    # the commit left the prefix grown by the route and its logits as the next prefix logits
    assert backend.prefix_token_ids == tuple(prompt + best["token_ids"])
    assert app.health()["metadata"]["committed_verify_rounds"] == 1
    assert app.health()["metadata"]["committed_prefix_length"] == 9
    # a second verify from the grown prefix: the prefix mismatch refusal, then a good request
    with pytest.raises(RuntimeError, match="target committed prefix mismatch"):
        app.verify({"prefix_token_ids": prompt, "routes": routes})
    out2 = app.verify({"prefix_token_ids": list(backend.prefix_token_ids), "routes": routes,
                       "selected_path_max_tokens": 2})
    assert out2["metadata"]["selected_path_committed_tokens"] == 2
    assert out2["metadata"]["selected_path_was_truncated"] is True
    assert out2["metadata"]["prefix_len_after"] == 11


def test_rpc_fallback_metadata_keys(cpu_target, monkeypatch):
    backend = cpu_target.make(fallback_threshold=0.0)  # every route scores below 0: fallback
    monkeypatch.setattr(backend, "_generate_fallback_ar", lambda *, max_tokens, eos_token_id: [3, 4][:max_tokens])
    app = TargetRpcStandIn(backend, cpu_target.tr.verify_payload_from_mapping)
    prompt = [5, 9, 14, 3]
    app.prefill({"prompt_token_ids": prompt})
    routes = [{"route_id": i, "token_ids": [20 + i, 21, 22]} for i in range(3)]
    out = app.verify({"prefix_token_ids": prompt, "routes": routes, "fallback_max_tokens": 2})
    assert out["decision"] == "fallback_ar" and out["selected_route_id"] is None
    assert out["fallback_token_ids"] == [3, 4] and out["fallback_reason"] == "path_score_below_threshold"
    meta = out["metadata"]
    for key in RUNTIME_METADATA_KEYS + VERIFY_COMMON_KEYS + VERIFY_FALLBACK_KEYS:
        assert key in meta, key
    assert meta["fallback_threshold"] == 0.0 and meta["fallback_token_count"] == 2
    assert meta["route_intervention"]["draft_token_logprobs_available"] is False


def test_route_intervention_metadata_reference_cases():
    """The two cases of the reference's tests/test_target_kv_commit.py:243-306."""
    tr = pkg("target_runtime")
    TRS = pkg("types").TargetRouteScore
    backend = object.__new__(tr.DirectFlashInferMaskedTreeVerifyBackend)
    route0 = TRS(route_id=10, token_ids=(100, 101), target_logprob=-5.0, draft_logprob=-0.1,
                 first_token_logprob=-2.0, selection_score=-5.0, draft_token_logprobs=(-0.05, -0.05))
    selected = TRS(route_id=20, token_ids=(200, 201), target_logprob=-1.0, draft_logprob=-2.0,
                   first_token_logprob=-0.2, selection_score=-1.0, draft_token_logprobs=(-1.0, -1.0))
    meta = backend._route_intervention_metadata([route0, selected], selected)
    iv = meta["route_intervention"]
    assert meta["selected_draft_rank"] == 2 and meta["route0_route_id"] == 10 and meta["draft_top_route_id"] == 10
    assert meta["selected_route_changed_from_route0"] is True
    assert meta["selected_first_token_changed_from_route0"] is True
    assert abs(meta["selected_minus_route0_draft_first_token_logprob"] + 0.95) < 1e-8
    assert abs(meta["selected_minus_route0_draft_logprob"] + 1.9) < 1e-8
    assert abs(meta["selected_minus_route0_target_selection_score"] - 4.0) < 1e-8
    assert iv["draft_token_logprobs_available"] is True
    assert iv["selected_vs_draft_top"]["first_token_changed"] is True

    top = TRS(route_id=1, token_ids=(10, 11), target_logprob=-3.0, draft_logprob=-102.0,
              draft_token_logprobs=(-0.8, -1.2))
    sel = TRS(route_id=2, token_ids=(20, 21), target_logprob=-1.0, draft_logprob=-13.0,
              draft_token_logprobs=(-1.0, -2.0))
    meta = backend._route_intervention_metadata([top, sel], sel)
    assert meta["draft_top_route_id"] == 1 and meta["selected_draft_rank"] == 2
    assert meta["selected_minus_route0_draft_logprob"] == -1.0
    assert meta["route_intervention"]["selected_vs_route0"]["legacy_cumulative_draft_logprob_delta"] == 89.0
    # ties in the draft order go to the earlier payload route; None deltas stay None
    a = TRS(route_id=7, token_ids=(1, 2), target_logprob=-1.0, draft_logprob=-1.0)
    b = TRS(route_id=3, token_ids=(1, 5), target_logprob=-0.5, draft_logprob=-1.0)
    meta = backend._route_intervention_metadata([a, b], b)
    assert meta["draft_top_route_id"] == 7 and meta["selected_draft_rank"] == 2
    assert meta["selected_minus_route0_draft_first_token_logprob"] is None
    assert meta["selected_first_token_changed_from_route0"] is False
    with pytest.raises(ValueError, match="non-empty scores"):
        backend._route_intervention_metadata([], a)


# ------------------------------------------------------------------ Drafter
def _runner(page_size=4, num_pages=64):
    alloc = OracleAllocator(num_pages=num_pages, page_size=page_size)
    rows = OracleReqPool(size=16, max_context_len=512)
    return SimpleNamespace(req_to_token_pool=rows, token_to_kv_pool_allocator=alloc, atlas_pool_page_size=page_size,
                           atlas_max_context_len=512, atlas_use_page_attention_metadata=False), alloc


class _ValueExecutor:
    """Writes the next value id into each new token's slot; zero logits."""

    def __init__(self, alloc):
        self.alloc = alloc
        self.next = 1

    def _write(self, slots):
        n = int(slots.numel())
        self.alloc.kv.write(slots.numpy(), torch.arange(self.next, self.next + n).numpy())
        self.next += n
        return torch.zeros((n, 8))

    def forward_frontier(self, *, input_ids, route_kv_metadata):
        return self._write(route_kv_metadata.out_cache_loc)

    def forward_extend(self, *, input_ids, out_cache_loc, positions, req_pool_indices, seq_lens_cpu):
        return self._write(out_cache_loc)


def _mods():
    sr = pkg("flashinfer_paged.sglang_runtime")
    kv = pkg("flashinfer_paged.kv")
    return SimpleNamespace(KVTreeStore=kv.KVTreeStore, SGLangFlashInferFrontierModelBackend=sr.SGLangFlashInferFrontierModelBackend)


def test_edge_prepare_prefix_decode_and_fallback_handoff():
    mods = _mods()
    runner, alloc = _runner()
    ex = _ValueExecutor(alloc)
    prompt = list(range(3, 13))  # 10 tokens: the tail page (size 4) holds 2
    ctx = edge_prepare_prefix(mods, runner=runner, page_size=4, prompt=prompt, executor=ex)
    assert ctx.prefix.committed_length == 10 and ctx.backend.route_pool.prefix_slot_count == 10
    # three stage-1 roots, one frontier step (the roots share the partial tail: copy-on-write)
    roots = [ctx.store.new_root_route(30 + i, ctx.store.prefix_view()) for i in range(3)]
    out = ctx.backend.decode_frontier_one_token(roots)
    active = ctx.store.mark_routes_materialized(roots, out.new_node_ids)
    assert out.metadata["cow_pages_copied_total"] == 2 and out.metadata["branch_safe_page_size"] is True
    assert len(ctx.store.routes) == 3 and len(ctx.store.nodes) == 3
    free_before = len(alloc.free_pages)
    res = edge_fallback_handoff(ctx, [50, 51, 52])
    assert res["released_route_rows"] == 3
    # the two copied tails; the first route wrote into the prefix's own tail page
    assert res["released_kv_pages"] == 2
    assert len(alloc.free_pages) == free_before + 2 - 1  # the extend opened one new page
    assert ctx.store.routes == {} and ctx.store.nodes == {}
    assert ctx.store.committed_token_ids == prompt + [50, 51, 52]
    assert res["prefix_token_ids"] == tuple(prompt + [50, 51, 52])
    assert res["prefix_view"].committed_length == 13
    slots = ctx.backend.route_pool.prefix_slot_ids
    assert slots.numel() == 13
    # the prompt's values, then the three extended tokens' values
    vals = alloc.kv.values[slots.numpy()].tolist()
    assert vals[:10] == list(range(1, 11)) and vals[10:] == [14, 15, 16]
    # the ids keep counting after the reset
    r = ctx.store.new_root_route(60, ctx.store.prefix_view())
    assert r.route_id == 4 and ctx.store.allocate_node_id() == 4


def test_from_runner_without_executor_or_reference_refuses():
    mods = _mods()
    runner, _ = _runner()
    with pytest.raises(RuntimeError, match="needs the Drafter model executor"):
        mods.SGLangFlashInferFrontierModelBackend.from_runner(route_store=mods.KVTreeStore(), model_runner=runner,
                                                              page_size=4, device="cpu")
    with pytest.raises(RuntimeError, match="does not match the physical SGLang KV pool"):
        mods.SGLangFlashInferFrontierModelBackend.from_runner(route_store=mods.KVTreeStore(), model_runner=runner,
                                                              page_size=8, device="cpu", executor=object())


class _Recorder:
    """Keyword arguments of one constructor call."""

    def __init__(self, **kw):
        self.kw = kw


def _standin_reference_runtime(calls, alloc):
    """Stand-ins for the reference route-pool module's SGLang helpers (the
    names its own backend calls), recording what they receive."""
    mod = ModuleType("atlas_0709.flashinfer_paged.sglang_runtime")
    mode = SimpleNamespace(EXTEND="extend-mode", DECODE="decode-mode")

    class RunnerExecutor:
        def __init__(self, *, model_runner, page_size):
            self.model_runner = model_runner
            self.page_size = page_size
            calls.append(("executor", page_size))
            self.inner = _ValueExecutor(alloc)

        def forward_frontier(self, *, input_ids, route_kv_metadata):
            return self.inner.forward_frontier(input_ids=input_ids, route_kv_metadata=route_kv_metadata)

        def runtime_metadata(self, *, cascade_level, verify_backend):
            return {"model_runner_class": "Fake", "cascade_level": cascade_level, "verify_backend": verify_backend}

    def forward(batch):
        calls.append(("forward", batch.kw))
        n = int(batch.kw["out_cache_loc"].numel())
        alloc.kv.write(batch.kw["out_cache_loc"].numpy(), torch.arange(900, 900 + n).numpy())
        return SimpleNamespace(next_token_logits=torch.full((1, 8), 7.0))

    mod.ensure_sglang_runner_runtime_defaults = lambda r: calls.append(("defaults",))
    mod.ensure_sglang_eager_runner = lambda r: calls.append(("eager",))
    mod.assert_sglang_flashinfer_active = lambda r: calls.append(("assert",))
    mod.SGLangFlashInferPagedDecodeBackend = RunnerExecutor
    mod._sglang_forward_batch_classes = lambda: (_Recorder, mode)
    mod._forward_mode = lambda cls, names: getattr(cls, names[0])
    mod._capture_hidden_mode_null = lambda: "null-capture"
    mod._extract_next_token_logits = lambda out: out.next_token_logits
    return mod, forward


def test_from_runner_builds_the_reference_executor_and_extends_on_its_runner(monkeypatch):
    mods = _mods()
    runner, alloc = _runner()
    calls = []
    ref, forward = _standin_reference_runtime(calls, alloc)
    runner.forward = forward
    monkeypatch.setitem(sys.modules, "atlas_0709.flashinfer_paged.sglang_runtime", ref)
    store = mods.KVTreeStore()
    backend = mods.SGLangFlashInferFrontierModelBackend.from_runner(route_store=store, model_runner=runner,
                                                                    page_size=4, device="cpu")
    assert calls[:3] == [("defaults",), ("assert",), ("executor", 4)]
    assert backend.executor.model_runner is runner
    # prompt prefill (value ids from the executor's own writer), then a frontier step
    pool = backend.route_pool
    handle = SimpleNamespace(rid="p", req_pool_idx=None)
    row = int(torch.as_tensor(pool.req_to_token_pool.alloc([handle])).reshape(-1)[0])
    slots = pool.allocate_extend_slots(prefix_lens=[0], seq_lens=[6], last_locs=torch.full((1,), -1))
    pool._write_req_token_row(row, slots)
    alloc.kv.write(slots.numpy(), torch.arange(1, 7).numpy())
    pool.req_to_token_pool.free(handle)
    backend.attach_prefilled_prefix(prompt_token_ids=list(range(6)), prefix_slot_ids=slots,
                                    next_token_logits=torch.zeros(8))
    del calls[:]
    root = store.new_root_route(40, store.prefix_view())
    out = backend.decode_frontier_one_token([root])
    assert calls == [("defaults",), ("eager",)]
    assert out.metadata["cascade_level"] == 0 and out.metadata["verify_backend"] == "none"
    assert out.metadata["model_runner_class"] == "Fake"
    # fallback EXTEND on the runner: one EXTEND ForwardBatch with the reference's fields
    del calls[:]
    pool.retain_route_rows([])
    pool.release_unreferenced_node_slots([])
    store.reset_speculative()
    logits = backend.append_known_tokens_as_prefix([70, 71, 72])
    assert [c[0] for c in calls] == ["defaults", "eager", "forward"]
    kw = calls[2][1]
    assert list(kw) == ["forward_mode", "batch_size", "input_ids", "req_pool_indices", "seq_lens", "out_cache_loc",
                        "seq_lens_sum", "orig_seq_lens", "positions", "seq_lens_cpu", "capture_hidden_mode",
                        "is_extend_in_batch", "all_extend_in_batch", "extend_num_tokens", "extend_seq_lens",
                        "extend_prefix_lens", "extend_start_loc", "extend_seq_lens_cpu", "extend_prefix_lens_cpu",
                        "extend_logprob_start_lens_cpu"]
    assert kw["forward_mode"] == "extend-mode" and kw["batch_size"] == 1
    assert kw["input_ids"].tolist() == [70, 71, 72] and kw["positions"].tolist() == [6, 7, 8]
    assert kw["seq_lens"].tolist() == [9] and kw["seq_lens_cpu"].tolist() == [9] and kw["seq_lens_sum"] == 9
    assert kw["extend_num_tokens"] == 3 and kw["extend_seq_lens"].tolist() == [3]
    assert kw["extend_prefix_lens"].tolist() == [6] and kw["extend_start_loc"].tolist() == [0]
    assert kw["extend_seq_lens_cpu"] == [3] and kw["extend_prefix_lens_cpu"] == [6]
    assert kw["extend_logprob_start_lens_cpu"] == [2] and kw["capture_hidden_mode"] == "null-capture"
    assert kw["is_extend_in_batch"] is True and kw["all_extend_in_batch"] is True
    assert torch.equal(logits, torch.full((8,), 7.0))
    assert alloc.kv.values[pool.prefix_slot_ids.numpy()].tolist()[-3:] == [900, 901, 902]
    assert math.isclose(float(logits[0]), 7.0)
