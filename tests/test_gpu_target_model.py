"""The Target drop-in on a small Llama-layout model built here from torch.nn
(random weights, nothing downloaded): 2 layers, hidden 1024, 8 query heads,
2 KV heads, head_dim 128, fp16, page 16.

* The verify forward with RoPE, append and attention fused into one launch per
  layer returns the logits, scores, selected route and committed KV cache of
  the separate ops (torch RoPE, write_suffix_kv, attention) bit for bit
  (src/atlas_0709/flashinfer_full_verify.py:1207-1223).
* The fallback AR (src/atlas_0709/target_runtime.py:767-851) starts from the
  argmax of the prefix logits, appends every generated token's K/V to the
  prefix pages, and each step's logits match a dense float32 recomputation of
  that step from the same weights and cache within 2e-2 (fp16 activations
  through two layers), with the same greedy tokens wherever the dense top-2
  margin exceeds that tolerance.
"""

import math
from types import SimpleNamespace

import pytest
import torch
from torch import nn

from helpers import pkg

pytestmark = pytest.mark.gpu

HIDDEN, HQ, HKV, D, LAYERS, VOCAB, PS = 1024, 8, 2, 128, 2, 1000, 16


class RMSNorm(nn.Module):
    def __init__(self, n, eps=1e-5):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(n))
        self.eps = eps

    def forward(self, x):
        y = x.float()
        y = y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + self.eps)
        return (y * self.weight.float()).to(x.dtype)


class MLP(nn.Module):
    def __init__(self):
        super().__init__()
        self.gate_proj = nn.Linear(HIDDEN, 2 * HIDDEN, bias=False)
        self.up_proj = nn.Linear(HIDDEN, 2 * HIDDEN, bias=False)
        self.down_proj = nn.Linear(2 * HIDDEN, HIDDEN, bias=False)

    def forward(self, x):
        return self.down_proj(nn.functional.silu(self.gate_proj(x)) * self.up_proj(x))


class Layer(nn.Module):
    def __init__(self):
        super().__init__()
        self.input_layernorm = RMSNorm(HIDDEN)
        self.post_attention_layernorm = RMSNorm(HIDDEN)
        self.self_attn = nn.Module()
        self.self_attn.q_proj = nn.Linear(HIDDEN, HQ * D, bias=False)
        self.self_attn.k_proj = nn.Linear(HIDDEN, HKV * D, bias=False)
        self.self_attn.v_proj = nn.Linear(HIDDEN, HKV * D, bias=False)
        self.self_attn.o_proj = nn.Linear(HQ * D, HIDDEN, bias=False)
        self.mlp = MLP()


class TinyLlama(nn.Module):
    def __init__(self):
        super().__init__()
        self.model = nn.Module()
        self.model.embed_tokens = nn.Embedding(VOCAB, HIDDEN)
        self.model.layers = nn.ModuleList([Layer() for _ in range(LAYERS)])
        self.model.norm = RMSNorm(HIDDEN)
        self.lm_head = nn.Linear(HIDDEN, VOCAB, bias=False)
        self.config = SimpleNamespace(hidden_size=HIDDEN, num_attention_heads=HQ, num_key_value_heads=HKV,
                                      head_dim=D, rope_theta=500000.0, vocab_size=VOCAB)


def _model(dev, seed):
    torch.manual_seed(seed)
    m = TinyLlama()
    with torch.no_grad():
        m.model.embed_tokens.weight.normal_(0.0, 1.0)
    return m.half().to(dev).eval()


def _nhd(cache, layout):
    """A paged layer as NHD pages [pages, 2, PS, HKV, D]."""
    return cache if layout == "NHD" else cache.permute(0, 1, 3, 2, 4)


def _backend(dev, model, *, prefix_len, seed, kv_layout=None, **kw):
    """The runtime over a random prefix cache; ``kv_layout`` None takes the
    runtime's default (HND pages), the same values either way."""
    tr = pkg("target_runtime")
    cfg = SimpleNamespace(k=3, d=4, page_size=PS, device=str(dev), workspace_mb=64, flashinfer_backend="auto",
                          use_packed_custom_mask=False, kv_layout=kv_layout)
    b = tr.DirectFlashInferMaskedTreeVerifyBackend(config=cfg, model=model, **kw)
    g = torch.Generator(device=dev).manual_seed(seed)
    pages = math.ceil(prefix_len / PS)
    nhd = [(torch.randn((pages, 2, PS, HKV, D), generator=g, device=dev) * 0.5).half() for _ in range(LAYERS)]
    b._paged_prefix_kv = nhd if b.kv_layout == "NHD" else [x.permute(0, 1, 3, 2, 4).contiguous() for x in nhd]
    b.prefix_token_ids = tuple(int(x) for x in torch.randint(0, VOCAB, (prefix_len,), generator=g, device=dev))
    b._prefix_logits = (torch.randn((1, VOCAB), generator=g, device=dev) * 3).half()
    return b


def _routes(seed):
    tr = pkg("target_runtime")
    g = torch.Generator().manual_seed(seed)
    return [tr.VerifyRoutePayload(route_id=10 + i, token_ids=tuple(int(x) for x in torch.randint(0, VOCAB, (4,), generator=g)),
                                  draft_logprob=-0.5 * i) for i in range(3)]


def test_fused_verify_forward_equals_separate_ops(dev):
    model = _model(dev, 1)
    results = []
    for fused in (True, False):
        b = _backend(dev, model, prefix_len=300, seed=2)
        b.fused_verify_step = fused
        routes = _routes(3)
        res = b.verify_payloads(prefix_token_ids=b.prefix_token_ids, routes=routes)
        torch.cuda.synchronize()
        assert b._wrapper.current_plan.fused_append
        results.append((res, [x.clone() for x in b._paged_prefix_kv], b.prefix_token_ids, b._prefix_logits.clone()))
    (ra, kva, pa, la), (rb, kvb, pb, lb) = results
    assert ra.selected_route_id == rb.selected_route_id and pa == pb
    assert [s.token_logprobs for s in ra.scores] == [s.token_logprobs for s in rb.scores]
    assert torch.equal(la.view(torch.int16), lb.view(torch.int16))
    for x, y in zip(kva, kvb):
        assert torch.equal(x.view(torch.int16), y.view(torch.int16))


def test_three_verify_rounds_fused_equals_separate(dev):
    """Three verify rounds in a row, each committing its selected route into
    the prefix (300 tokens grow past the page boundary at 304, so the paged
    prefix grows): the fused and the separate forward agree at every round
    on the selection, committed tokens, per-token log-probs and prefix
    logits, and end with bit-equal KV pages."""
    model = _model(dev, 7)
    runs = []
    for fused in (True, False):
        b = _backend(dev, model, prefix_len=300, seed=8)
        b.fused_verify_step = fused
        rounds = []
        for r in range(3):
            res = b.verify_payloads(prefix_token_ids=b.prefix_token_ids, routes=_routes(20 + r))
            torch.cuda.synchronize()
            rounds.append((res.selected_route_id, b.prefix_token_ids, [sc.token_logprobs for sc in res.scores],
                           b._prefix_logits.clone().view(torch.int16)))
        runs.append((rounds, [x.clone() for x in b._paged_prefix_kv]))
    (ra, kva), (rb, kvb) = runs
    assert len(ra[-1][1]) > 304  # the committed prefix crossed a page boundary
    for (sa, pa, la, xa), (sb, pb, lb, xb) in zip(ra, rb):
        assert sa == sb and pa == pb and la == lb and torch.equal(xa, xb)
    assert len(kva) == len(kvb)
    for x, y in zip(kva, kvb):
        assert x.shape == y.shape and torch.equal(x.view(torch.int16), y.view(torch.int16))


def test_hnd_and_nhd_prefix_pages_give_the_same_rounds(dev):
    """The runtime's HND prefix pages and the reference's NHD pages holding
    the same values: three verify rounds (fused forward, commits growing the
    prefix past a page boundary) and a fallback AR give the same selections,
    per-token log-probs, prefix logits and, read as NHD, the same KV bits."""
    model = _model(dev, 9)
    runs = []
    for layout in ("NHD", "HND"):
        b = _backend(dev, model, prefix_len=300, seed=10, kv_layout=layout, fallback_ar_tokens=3)
        assert b.kv_layout == layout and b._wrapper.kv_layout == layout
        rounds = []
        for r in range(3):
            res = b.verify_payloads(prefix_token_ids=b.prefix_token_ids, routes=_routes(30 + r))
            torch.cuda.synchronize()
            rounds.append((res.selected_route_id, b.prefix_token_ids, [sc.token_logprobs for sc in res.scores],
                           b._prefix_logits.clone().view(torch.int16)))
        b.fallback_threshold = 1e9
        res = b.verify_payloads(prefix_token_ids=b.prefix_token_ids, routes=_routes(40))
        torch.cuda.synchronize()
        rounds.append((tuple(res.fallback_token_ids), b.prefix_token_ids, None,
                       b._prefix_logits.clone().view(torch.int16)))
        runs.append((rounds, [_nhd(x, layout).contiguous() for x in b._paged_prefix_kv]))
    (ra, kva), (rb, kvb) = runs
    assert len(ra[2][1]) > 304
    for (sa, pa, la, xa), (sb, pb, lb, xb) in zip(ra, rb):
        assert sa == sb and pa == pb and la == lb and torch.equal(xa, xb)
    for x, y in zip(kva, kvb):
        assert x.shape == y.shape and torch.equal(x.view(torch.int16), y.view(torch.int16))


def _dense_step_logits(model, cache, seq_len, token, pos):
    """One decode step of the tiny model in float32 over the first seq_len
    rows of the paged cache (whose row pos already holds this token's K/V,
    written by the step under test; it is recomputed here and checked)."""
    tr = pkg("target_runtime")
    base = model.model
    h = base.embed_tokens(torch.tensor([token], device=cache[0].device))
    cos, sin = tr.rope_cos_sin(model, torch.tensor([pos], device=h.device), D, h.dtype, h.device)
    cos, sin = cos[:, None, :], sin[:, None, :]
    for li, layer in enumerate(base.layers):
        x = layer.input_layernorm(h)
        q = layer.self_attn.q_proj(x).reshape(1, HQ, D)
        k = layer.self_attn.k_proj(x).reshape(1, HKV, D)
        q = q * cos + tr.rotate_half(q) * sin
        k = k * cos + tr.rotate_half(k) * sin
        kv = cache[li]
        keys = kv[:, 0].reshape(-1, HKV, D)[:seq_len].float()
        vals = kv[:, 1].reshape(-1, HKV, D)[:seq_len].float()
        if li == 0:  # the first layer's K row depends on the token alone: written bit for bit
            assert torch.equal(kv[pos // PS, 0, pos % PS].view(torch.int16), k[0].view(torch.int16))
        out = []
        for hh in range(HQ):
            kh = keys[:, hh // (HQ // HKV)]
            s = (kh @ q[0, hh].float()) / math.sqrt(D)
            p = torch.softmax(s, dim=0)
            out.append(p @ vals[:, hh // (HQ // HKV)])
        attn = torch.stack(out).reshape(1, HQ * D).half()
        h = h + layer.self_attn.o_proj(attn)
        h = h + layer.mlp(layer.post_attention_layernorm(h))
    return model.lm_head(base.norm(h)).float()


def test_fallback_ar_decodes_on_the_prefix_pages(dev):
    model = _model(dev, 4)
    b = _backend(dev, model, prefix_len=203, seed=5, fallback_threshold=1e9, fallback_ar_tokens=4)
    prefix_len = len(b.prefix_token_ids)
    first = int(torch.argmax(b._prefix_logits, dim=-1))
    res = b.verify_payloads(prefix_token_ids=b.prefix_token_ids, routes=_routes(6))
    torch.cuda.synchronize()
    assert res.decision == "fallback_ar" and res.selected_route_id is None
    toks = list(res.fallback_token_ids)
    assert len(toks) == 4 and toks[0] == first
    assert b.prefix_token_ids[prefix_len:] == tuple(toks) and res.metadata["prefix_len_after"] == prefix_len + 4
    # replay the steps densely: step i consumed token i at position prefix_len + i
    for i, tok in enumerate(toks):
        with torch.no_grad():
            dense = _dense_step_logits(model, [_nhd(x, b.kv_layout) for x in b._paged_prefix_kv],
                                       prefix_len + i + 1, tok, prefix_len + i)
        if i + 1 < len(toks):
            top2 = torch.topk(dense[0], 2).values
            if float(top2[0] - top2[1]) > 2e-2:
                assert int(torch.argmax(dense)) == toks[i + 1], f"step {i}: greedy token differs"
    assert float((b._prefix_logits.float() - dense).abs().max()) <= 2e-2


def _hf_llama(dev, seed):
    """A transformers Llama of the tiny geometry above (random weights)."""
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(seed)
    cfg = LlamaConfig(vocab_size=VOCAB, hidden_size=HIDDEN, intermediate_size=2 * HIDDEN, num_hidden_layers=LAYERS,
                      num_attention_heads=HQ, num_key_value_heads=HKV, head_dim=D, max_position_embeddings=1024,
                      rope_theta=500000.0, attn_implementation="sdpa")
    m = LlamaForCausalLM(cfg)
    with torch.no_grad():
        m.model.embed_tokens.weight.normal_(0.0, 1.0)
    return m.half().to(dev).eval()


def test_rpc_sequence_from_prefill_on_a_transformers_llama(dev):
    """The reference server's sequence (rpc.py:66-128) from a real prefill:
    health, prefill of a 300-token prompt through the model's own forward and
    KV cache, then two verifies with commits.  Each selected route's per-token
    log-probs match the model's own dense forward over the committed prefix
    and the route (fp16 activations through two layers: 3e-2), the metadata
    carries the reference's keys, and the prefix grows by the committed
    routes."""
    from standin_callers import (RUNTIME_METADATA_KEYS, VERIFY_COMMON_KEYS, VERIFY_SELECT_KEYS,
                                 TargetRpcStandIn)

    tr = pkg("target_runtime")
    model = _hf_llama(dev, 11)
    cfg = SimpleNamespace(k=3, d=4, page_size=PS, device=str(dev), dtype="float16", workspace_mb=64,
                          flashinfer_backend="auto", use_packed_custom_mask=False)
    backend = tr.DirectFlashInferMaskedTreeVerifyBackend(model_path="tiny-llama", config=cfg, model=model)
    app = TargetRpcStandIn(backend, tr.verify_payload_from_mapping)
    health = app.health()
    assert tuple(health["metadata"]) == RUNTIME_METADATA_KEYS and health["metadata"]["committed_prefix_length"] == 0
    g = torch.Generator().manual_seed(12)
    prompt = [int(x) for x in torch.randint(0, VOCAB, (300,), generator=g)]
    pre = app.prefill({"prompt_token_ids": prompt})
    assert pre["prompt_len"] == 300 and pre["metadata"]["committed_prefix_length"] == 300
    assert backend.kv_layout == "HND"  # the runtime's default pages: [pages, 2, Hkv, page_size, D]
    assert len(backend._paged_prefix_kv) == LAYERS and backend._paged_prefix_kv[0].shape[1:] == (2, HKV, PS, D)
    prefix = list(prompt)
    for rnd in range(2):
        routes = [{"route_id": 10 * rnd + i, "token_ids": [int(x) for x in torch.randint(0, VOCAB, (4,), generator=g)],
                   "draft_logprob": -0.5 * i} for i in range(3)]
        routes[1]["token_ids"][:2] = routes[0]["token_ids"][:2]  # a shared prefix: 10 unique nodes
        out = app.verify({"prefix_token_ids": prefix, "routes": routes})
        torch.cuda.synchronize()
        meta = out["metadata"]
        for key in RUNTIME_METADATA_KEYS + VERIFY_COMMON_KEYS + VERIFY_SELECT_KEYS:
            assert key in meta, key
        assert meta["node_count"] == 10 and meta["prefix_len_before"] == len(prefix)
        with torch.no_grad():
            for s in out["scores"]:
                ids = torch.tensor([prefix + s["token_ids"]], device=dev)
                lps = torch.log_softmax(model(input_ids=ids).logits[0].float(), dim=-1)
                want = [float(lps[len(prefix) - 1 + t, s["token_ids"][t]]) for t in range(4)]
                assert s["token_logprobs"] == pytest.approx(want, abs=3e-2), (rnd, s["route_id"])
        sel = out["selected_score"]
        prefix = prefix + sel["token_ids"]
        assert list(backend.prefix_token_ids) == prefix and meta["prefix_len_after"] == len(prefix)
    assert app.health()["metadata"]["committed_verify_rounds"] == 2
    # the next prefix logits are the model's own after the committed prefix
    with torch.no_grad():
        dense = model(input_ids=torch.tensor([prefix], device=dev)).logits[0, -1].float()
    assert float((backend._prefix_logits[0].float() - dense).abs().max()) <= 5e-2


@pytest.mark.parametrize("variant", ["best", "truncate_eos", "thresholds", "weights", "first_route"])
def test_device_route_selection_equals_host_path(dev, variant):
    """verify_payloads with the selection and commit queued on the device
    and with both on the host: the same result records (selection, scores,
    metadata, fallback tokens), prefix tokens, prefix logits and KV bits over
    four rounds (the variants truncate at an EOS token and a token limit,
    fall back on thresholds, weight the scores, or take the first route)."""
    model = _model(dev, 11)
    runs = []
    for on_device in (True, False):
        kw = {}
        if variant == "thresholds":
            kw = dict(first_token_threshold=-7.6, fallback_threshold=-40.0, fallback_ar_tokens=2)
        elif variant == "weights":
            kw = dict(score_weights=(1.0, 0.5, 0.25, 0.125))
        elif variant == "first_route":
            kw = dict(route_selection_policy="first_route")
        b = _backend(dev, model, prefix_len=290, seed=12, **kw)
        b.device_route_selection = on_device
        rounds = []
        for r in range(4):
            routes = _routes(50 + r)
            call = {}
            if variant == "truncate_eos":
                call = dict(selected_path_max_tokens=3 if r % 2 else None,
                            eos_token_id=routes[r % 3].token_ids[1 + r % 2])
            res = b.verify_payloads(prefix_token_ids=b.prefix_token_ids, routes=routes, **call)
            torch.cuda.synchronize()
            meta = {key: v for key, v in res.metadata.items() if key != "fallback_ar_profile"}
            rounds.append((res.selected_route_id, res.decision, res.fallback_token_ids, res.scores, meta,
                           b.prefix_token_ids, b._prefix_logits.clone().view(torch.int16)))
        runs.append((rounds, [x.clone() for x in b._paged_prefix_kv]))
    (ra, kva), (rb, kvb) = runs
    for a, bb in zip(ra, rb):
        assert a[:3] == bb[:3] and a[3] == bb[3] and a[4] == bb[4] and a[5] == bb[5] and torch.equal(a[6], bb[6])
    decisions = {x[1] for x in ra}
    if variant == "thresholds":
        assert decisions == {"select", "fallback_ar"}
    for x, y in zip(kva, kvb):
        assert x.shape == y.shape and torch.equal(x.view(torch.int16), y.view(torch.int16))
