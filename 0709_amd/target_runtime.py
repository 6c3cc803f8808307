"""Target-side persistent tree verifier (drop-in for the reference's
``atlas_0709.target_runtime``).

``DirectFlashInferMaskedTreeVerifyBackend`` keeps the reference's method
names, arguments, metadata and exceptions (``target_runtime.py:41-920``).  The
work that touches KV or logits runs on the gfx950 kernels:

* ``_commit_selected_path`` -- one all-layer commit launch whose positions
  travel in the kernel arguments (the reference issues gather + clone +
  index_put per layer, ``:885-912``);
* ``_score_routes`` -- one log-sum-exp + gather launch per logits tensor and a
  single device-to-host copy of the k*d log-probs (the reference converts each
  token's log-prob with ``.cpu()``, ``:742``);
* the masked verify forward uses ``write_suffix_kv`` and the tree attention
  wrapper of this package.

Model compute (embedding, projections, MLP, lm_head) stays in the caller's
torch model; ``run_full_verify`` drives a Hugging Face Llama-layout module the
way ``flashinfer_full_verify.run_flashinfer_full_verify`` does (``:1182-1231``).
"""

from __future__ import annotations

import ctypes
import hashlib
import json
import math
import time
from dataclasses import dataclass
from typing import Sequence

import numpy as np
import torch

from . import _lib, kv_ops
from .decode_attention import make_decode_wrapper, plan_decode_wrapper
from .flashinfer_full_verify import (
    FullVerifyState,
    build_deduplicated_tree_spec_from_paths,
    ceil_div,
    first_tensor,
    make_prefill_wrapper,
    plan_prefill_wrapper,
    prefix_layer_to_paged_kv,
    write_suffix_kv,
)
from .types import PrefixState, TargetRouteScore, TargetVerifyResult

ROUTE_POLICIES = ("target_best", "target_sample", "first_route")
# what runs the verify attention, reported where the reference reports its
# FlashInfer version
ATTENTION_LIBRARY = "atlas0709-hip-gfx950"


@dataclass(frozen=True)
class VerifyRoutePayload:
    route_id: int
    token_ids: tuple[int, ...]
    draft_logprob: float
    draft_token_logprobs: tuple[float, ...] = ()


def verify_payload_from_mapping(item: dict) -> VerifyRoutePayload:
    """``target_runtime.py:922-935``."""
    raw = item.get("draft_token_logprobs")
    if raw is None:
        draft_token_logprobs: tuple[float, ...] = ()
    elif isinstance(raw, (list, tuple)):
        draft_token_logprobs = tuple(float(v) for v in raw)
    else:
        raise ValueError("draft_token_logprobs must be a list of numbers when provided")
    return VerifyRoutePayload(
        route_id=int(item["route_id"]),
        token_ids=tuple(int(t) for t in item["token_ids"]),
        draft_logprob=float(item.get("draft_logprob", 0.0)),
        draft_token_logprobs=draft_token_logprobs,
    )


def gather_token_logprobs(logits: torch.Tensor, rows: Sequence[int], tokens: Sequence[int],
                          extra_logits: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 ``log_softmax(logits[row])[token]`` for each (row, token) pair,
    computed on the device in one launch.  ``logits``: [rows, vocab] or [vocab].
    With ``extra_logits`` ([rows2, vocab] or [vocab], same dtype and vocab),
    row indices ``rows .. rows + rows2 - 1`` name its rows, in the same launch.
    ``out``: a contiguous fp32 device tensor of len(rows) values to write."""
    device = _lib.require_device(logits, what="route scoring")
    lg = logits.reshape(1, -1) if logits.ndim == 1 else logits
    if lg.ndim != 2 or lg.stride(-1) != 1:
        raise ValueError("logits must be [rows, vocab] with contiguous rows")
    lg2 = None
    if extra_logits is not None:
        _lib.require_device(logits, extra_logits, what="route scoring")
        lg2 = extra_logits.reshape(1, -1) if extra_logits.ndim == 1 else extra_logits
        if lg2.ndim != 2 or lg2.stride(-1) != 1 or int(lg2.shape[1]) != int(lg.shape[1]) or lg2.dtype != lg.dtype:
            raise ValueError("extra_logits must be [rows, vocab] rows of the same vocabulary and dtype")
    n = len(rows)
    if out is None:
        out = torch.empty(n, dtype=torch.float32, device=device)
    elif out.dtype != torch.float32 or out.device != device or not out.is_contiguous() or int(out.numel()) != n:
        raise ValueError(f"out must be a contiguous float32 tensor of {n} values on {device}")
    if n == 0:
        return out
    if len(tokens) != n:
        raise ValueError("rows and tokens must have equal length")
    # tokens (int64) and rows (int32) in one upload from pinned memory, queued
    # without waiting for the work ahead on the stream (the logits' producer)
    host = np.concatenate((np.asarray(tokens, dtype=np.int64).view(np.uint8),
                           np.asarray(rows, dtype=np.int32).view(np.uint8)))
    idx = _lib.staging().upload(host, device)
    tok = idx[: 8 * n].view(torch.int64)
    row = idx[8 * n:].view(torch.int32)
    lib = _lib.load()
    rows2 = 0 if lg2 is None else int(lg2.shape[0])
    need = int(lib.atlas_gather_logprobs_workspace_bytes(int(lg.shape[0]) + rows2, int(lg.shape[1])))
    if need < 0:
        raise ValueError(f"bad logits shape {tuple(lg.shape)}")
    ws = _scoring_workspace(device, need)
    rc = lib.atlas_gather_logprobs(
        _lib.ptr(lg), lg.stride(0), int(lg.shape[0]), _lib.ptr(lg2), lg2.stride(0) if lg2 is not None else 0, rows2,
        int(lg.shape[1]), _lib.dtype_code(lg.dtype), _lib.ptr(row), _lib.ptr(tok), n, None, _lib.ptr(out),
        _lib.ptr(ws), int(ws.numel()), _lib.stream_of(device),
    )
    _lib.check(rc, "atlas_gather_logprobs")
    return out


_SCORING_WS: dict = {}


def _scoring_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """The scoring launch's chunk statistics: zero-filled once per device (and
    when it grows); every launch leaves them zero."""
    key = (device.type, device.index)
    ws = _SCORING_WS.get(key)
    if ws is None or int(ws.numel()) < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
        _SCORING_WS[key] = ws
    return ws


def rotate_half(hidden_states: torch.Tensor) -> torch.Tensor:
    first, second = hidden_states.chunk(2, dim=-1)
    return torch.cat((-second, first), dim=-1)


def rope_cos_sin(model, positions: torch.Tensor, head_dim: int, dtype: torch.dtype, device) -> tuple:
    """cos/sin at the given positions from the model's rotary module, else the
    default theta schedule (``flashinfer_full_verify.py:231-297``)."""
    positions = positions.to(device=device, dtype=torch.long).reshape(-1)
    rotary = getattr(getattr(model, "model", None), "rotary_emb", None)
    if rotary is not None:
        hidden = int(getattr(model.config, "hidden_size", head_dim))
        dummy = torch.empty((1, int(positions.numel()), hidden), dtype=dtype, device=device)
        cos, sin = rotary(dummy, positions.reshape(1, -1))
        return cos.to(dtype).reshape(-1, head_dim), sin.to(dtype).reshape(-1, head_dim)
    theta = float(getattr(model.config, "rope_theta", 10000.0))
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim))
    emb = torch.outer(positions.float(), inv)
    emb = torch.cat((emb, emb), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


@torch.inference_mode()
def run_full_verify(*, model, wrapper, state: FullVerifyState, prefix_len: int, page_size: int,
                    fused: bool | None = None) -> torch.Tensor:
    """Masked tree forward of a Llama-layout model: per layer RMSNorm, QKV,
    RoPE at prefix_len + depth, ``write_suffix_kv`` then tree attention
    (append before attention, as ``flashinfer_full_verify.py:1207-1223``).

    When the plan allows it (head_dim 128, power-of-two pages of >= 16
    tokens, one row block per (request, KV head): ``current_plan.fused_append``)
    the rotary embedding, the append and the attention are one launch per
    layer (``wrapper.run(q, kv, append_key_states=k, append_value_states=v,
    rope_cos_sin=(cos, sin))`` on the projections before RoPE), which writes
    the cache and returns the output of the separate ops bit for bit.
    ``fused=False`` runs the separate ops; ``fused=True`` requires the fused
    launch."""
    cfg = model.config
    base = model.model
    head_dim = getattr(cfg, "head_dim", None) or int(cfg.hidden_size) // int(cfg.num_attention_heads)
    hq, hkv = int(cfg.num_attention_heads), int(cfg.num_key_value_heads)
    n = state.tree.node_count
    hidden = base.embed_tokens(state.tree.flat_token_ids)
    positions = int(prefix_len) + state.tree.depths.to(device=hidden.device, dtype=torch.long)
    cos, sin = rope_cos_sin(model, positions, head_dim, hidden.dtype, hidden.device)
    plan = getattr(wrapper, "current_plan", None)
    can_fuse = plan is not None and bool(getattr(plan, "fused_append", False))
    if fused and not can_fuse:
        raise NotImplementedError("the plan does not allow the fused verify step (see current_plan.fused_append)")
    use_fused = can_fuse if fused is None else bool(fused)
    cos3, sin3 = cos[:, None, :], sin[:, None, :]
    for layer_idx, layer in enumerate(base.layers):
        residual = hidden
        normed = layer.input_layernorm(hidden)
        q = layer.self_attn.q_proj(normed).reshape(n, hq, head_dim)
        k = layer.self_attn.k_proj(normed).reshape(n, hkv, head_dim)
        v = layer.self_attn.v_proj(normed).reshape(n, hkv, head_dim).contiguous()
        kv_cache = state.paged_prefix_kv[layer_idx]
        if use_fused:
            out = wrapper.run(q.contiguous(), kv_cache, append_key_states=k.contiguous(), append_value_states=v,
                              rope_cos_sin=(cos, sin))
        else:
            q = (q * cos3 + rotate_half(q) * sin3).contiguous()
            k = (k * cos3 + rotate_half(k) * sin3).contiguous()
            write_suffix_kv(kv_cache, key_states=k, value_states=v, prefix_len=prefix_len, page_size=page_size,
                            kv_layout=getattr(wrapper, "kv_layout", "NHD"))
            out = wrapper.run(q, kv_cache)
        attn = first_tensor(out).reshape(n, hq * head_dim)
        hidden = residual + layer.self_attn.o_proj(attn)
        residual = hidden
        hidden = residual + layer.mlp(layer.post_attention_layernorm(hidden))
    return model.lm_head(base.norm(hidden))


def next_argmax_inputs(logits: torch.Tensor) -> torch.Tensor:
    """Greedy next token (``flashinfer_full_verify.py:444-445``)."""
    return torch.argmax(logits, dim=-1).to(dtype=torch.long)


@dataclass
class FullDecodeState:
    input_ids: torch.Tensor
    paged_prefix_kv: list


@torch.inference_mode()
def run_full_ar_decode(*, model, wrappers, state: FullDecodeState, prefix_len: int, page_size: int) -> torch.Tensor:
    """Greedy autoregressive decode steps of a Llama-layout model on the paged
    prefix KV, one planned decode wrapper per step
    (``flashinfer_full_verify.py:1066-1122``): per layer RMSNorm, QKV, RoPE at
    the step's position, ``write_suffix_kv`` of the new token, then paged
    decode attention over the prefix and the new token."""
    cfg = model.config
    base = model.model
    head_dim = getattr(cfg, "head_dim", None) or int(cfg.hidden_size) // int(cfg.num_attention_heads)
    hq, hkv = int(cfg.num_attention_heads), int(cfg.num_key_value_heads)
    input_ids = state.input_ids
    logits = None
    for step_idx, wrapper in enumerate(wrappers):
        hidden = base.embed_tokens(input_ids.reshape(-1))
        pos = int(prefix_len) + int(step_idx)
        cos, sin = rope_cos_sin(model, torch.tensor([pos], device=hidden.device), head_dim, hidden.dtype,
                                hidden.device)
        cos, sin = cos[:, None, :], sin[:, None, :]
        for layer_idx, layer in enumerate(base.layers):
            residual = hidden
            normed = layer.input_layernorm(hidden)
            q = layer.self_attn.q_proj(normed).reshape(1, hq, head_dim)
            k = layer.self_attn.k_proj(normed).reshape(1, hkv, head_dim)
            v = layer.self_attn.v_proj(normed).reshape(1, hkv, head_dim).contiguous()
            q = (q * cos + rotate_half(q) * sin).contiguous()
            k = (k * cos + rotate_half(k) * sin).contiguous()
            kv_cache = state.paged_prefix_kv[layer_idx]
            write_suffix_kv(kv_cache, key_states=k, value_states=v, prefix_len=prefix_len, page_size=page_size,
                            start_pos=pos, kv_layout=getattr(wrapper, "kv_layout", "NHD"))
            attn = first_tensor(wrapper.run(q, kv_cache)).reshape(1, hq * head_dim)
            hidden = residual + layer.self_attn.o_proj(attn)
            residual = hidden
            hidden = residual + layer.mlp(layer.post_attention_layernorm(hidden))
        logits = model.lm_head(base.norm(hidden))
        input_ids = next_argmax_inputs(logits)
    if logits is None:
        raise RuntimeError("decode steps must be positive")
    return logits


def _scoring_pairs(paths, route_to_node_paths, n_verify: int) -> tuple[list[int], list[int]]:
    """(row, token) pairs of the route scoring, in the order the selection
    launch reads them: every route's first token (the prefix logits, row
    ``n_verify``), then each route's tokens t > 0 (the verify row of its node
    t - 1)."""
    rows = [n_verify] * len(paths)
    toks = [int(path[0]) for path in paths]
    for path, nodes in zip(paths, route_to_node_paths):
        for off in range(1, len(path)):
            rows.append(int(nodes[off - 1]))
            toks.append(int(path[off]))
    return rows, toks


def _route_score(**fields) -> TargetRouteScore:
    """``TargetRouteScore(**fields)`` for a keyword set naming every field,
    with the fields set through the instance dict instead of the frozen
    dataclass's per-field ``object.__setattr__`` (a verify step waits on the
    loop that builds one per route)."""
    score = object.__new__(TargetRouteScore)
    score.__dict__.update(fields)
    return score


class DirectFlashInferMaskedTreeVerifyBackend:
    """Persistent Target: committed prefix KV, masked tree verify, route
    scoring / selection and in-place commit of the selected path."""

    # Select target_best / first_route routes on the device and queue the
    # commit behind the scoring (the host still selects from the read-back
    # scores and refuses a disagreement); False keeps selection and commit
    # launch on the host.
    device_route_selection: bool = True

    def __init__(
        self,
        *,
        model_path: str | None = None,
        config,
        model=None,
        tokenizer=None,
        score_weights: Sequence[float] | None = None,
        fallback_threshold: float | None = None,
        first_token_threshold: float | None = None,
        fallback_ar_tokens: int = 4,
        profile_fallback_ar: bool = False,
        route_selection_policy: str = "target_best",
        route_sampling_temperature: float = 1.0,
    ) -> None:
        validate = getattr(config, "validate", None)
        if callable(validate):
            validate()
        self.model_path = model_path
        self.config = config
        self.score_weights = self._validate_score_weights(score_weights)
        self.fallback_threshold = None if fallback_threshold is None else float(fallback_threshold)
        self.first_token_threshold = None if first_token_threshold is None else float(first_token_threshold)
        self.fallback_ar_tokens = int(fallback_ar_tokens)
        self.profile_fallback_ar = bool(profile_fallback_ar)
        self.route_selection_policy = self._validate_route_selection_policy(route_selection_policy)
        self.route_sampling_temperature = self._validate_route_sampling_temperature(route_sampling_temperature)
        if self.fallback_ar_tokens <= 0:
            raise ValueError("fallback_ar_tokens must be positive")
        if self.route_selection_policy == "first_route" and (
            self.fallback_threshold is not None or self.first_token_threshold is not None
        ):
            raise ValueError(
                "first_route is a strict diagnostic policy and requires fallback thresholds to be disabled"
            )
        if model is None and model_path is not None:
            from transformers import AutoModelForCausalLM, AutoTokenizer

            dtype = getattr(torch, str(getattr(config, "dtype", "float16")))
            tokenizer = AutoTokenizer.from_pretrained(model_path)
            model = AutoModelForCausalLM.from_pretrained(model_path, torch_dtype=dtype).to(config.device).eval()
        self.model = model
        self.tokenizer = tokenizer
        self.dtype = next(model.parameters()).dtype if model is not None else torch.float16
        # The committed prefix lives in HND pages ([pages, 2, Hkv, page_size, D]):
        # each KV head's keys of a page are one contiguous run, which the
        # attention streams faster than the NHD pages of the reference
        # (``args.kv_layout = "NHD"`` keeps those).
        self.kv_layout = kv_ops.check_kv_layout(getattr(config, "kv_layout", None) or "HND")
        self._wrapper = make_prefill_wrapper(args=config, kv_layout=self.kv_layout) if model is not None else None
        self.prefix_token_ids: tuple[int, ...] = ()
        self._paged_prefix_kv: list[torch.Tensor] | None = None
        self._prefix_logits: torch.Tensor | None = None
        self._committed_verify_rounds = 0
        self._fallback_decode_wrapper = None
        self._last_fallback_ar_profile = None
        self.match_logits_dtype_rounding = True
        # run the verify forward's RoPE + append + attention as one launch per
        # layer when the plan allows it (None: whenever it does)
        self.fused_verify_step: bool | None = None

    # ------------------------------------------------------------ prefill
    @torch.inference_mode()
    def prefill(self, prompt_token_ids: Sequence[int]) -> PrefixState:
        """Prompt forward of the caller's model, its K/V laid out as the
        committed paged prefix (``target_runtime.py:114-142``)."""
        token_ids = tuple(int(t) for t in prompt_token_ids)
        if not token_ids:
            raise ValueError("target prefill requires a non-empty prompt")
        if self.model is None:
            raise RuntimeError("target prefill needs a model")
        ids = torch.tensor([token_ids], dtype=torch.long, device=self.config.device)
        out = self.model(input_ids=ids, use_cache=True)
        past = out.past_key_values
        layers = []
        for layer_idx in range(len(self.model.model.layers)):
            key, value = _legacy_layer_kv(past, layer_idx)
            layers.append(prefix_layer_to_paged_kv(key=key, value=value, prefix_len=len(token_ids), node_count=0,
                                                   page_size=self.config.page_size, kv_layout=self.kv_layout))
        self.prefix_token_ids = token_ids
        self._paged_prefix_kv = layers
        self._prefix_logits = out.logits[:, -1, :].detach()
        self._committed_verify_rounds = 0
        self._last_fallback_ar_profile = None
        return PrefixState(token_ids=token_ids, next_token_logits=self._prefix_logits[0],
                           committed_length=len(token_ids), metadata=self.runtime_metadata())

    def runtime_metadata(self) -> dict[str, object]:
        """The keys of the reference's ``runtime_metadata``
        (``target_runtime.py:322-359``), read by the health call and the edge
        controller's policy checks.  ``backend`` keeps the reference's name so
        callers that key on it still match; ``flashinfer_version`` names the
        kernel library that runs the attention instead (no FlashInfer is
        involved)."""
        cfg = self.config
        tok = self.tokenizer
        model_cfg = getattr(self.model, "config", None)
        vocab = getattr(model_cfg, "vocab_size", None)
        return {
            "backend": "direct_flashinfer_full_llama_masked_verify",
            "model": self.model_path,
            "model_vocab_size": None if vocab is None else int(vocab),
            "tokenizer_vocab_size": None if tok is None else int(len(tok)),
            "tokenizer_bos_token_id": getattr(tok, "bos_token_id", None),
            "tokenizer_eos_token_id": getattr(tok, "eos_token_id", None),
            "tokenizer_pad_token_id": getattr(tok, "pad_token_id", None),
            "paged_kv": True,
            "custom_mask": True,
            "packed_custom_mask": bool(getattr(cfg, "use_packed_custom_mask", False)),
            "rope_applied": True,
            "logits_aligned": None,
            "runtime_alignment_checked": False,
            "semantic_correctness_required": True,
            "page_size": cfg.page_size,
            "dtype": getattr(cfg, "dtype", None),
            "device": getattr(cfg, "device", None),
            "flashinfer_version": ATTENTION_LIBRARY,
            "persistent_target_paged_kv": True,
            "deduplicated_tree_nodes": True,
            "selection_policy": self._selection_policy_name(),
            "route_selection_policy": self.route_selection_policy,
            "route_sampling_scope": "verified_route_level_only",
            "route_sampling_temperature": float(self.route_sampling_temperature),
            "fallback_ar_sampling": "greedy_argmax",
            "score_weights": None if self.score_weights is None else [float(w) for w in self.score_weights],
            "fallback_threshold": self.fallback_threshold,
            "first_token_threshold": self.first_token_threshold,
            "fallback_ar_tokens": int(self.fallback_ar_tokens),
            "fallback_decode_wrapper_reused": True,
            "profile_fallback_ar": self.profile_fallback_ar,
            "committed_verify_rounds": self._committed_verify_rounds,
            "committed_prefix_length": len(self.prefix_token_ids),
        }

    # ------------------------------------------------------------ verify
    @torch.inference_mode()
    def verify_payloads(
        self,
        *,
        prefix_token_ids: Sequence[int],
        routes: Sequence[VerifyRoutePayload],
        fallback_max_tokens: int | None = None,
        selected_path_max_tokens: int | None = None,
        eos_token_id: int | None = None,
        route_sampling_seed: int | None = None,
        route_sampling_round: int | None = None,
    ) -> TargetVerifyResult:
        prefix = tuple(int(t) for t in prefix_token_ids)
        if self._paged_prefix_kv is None or self._prefix_logits is None:
            self.prefill(prefix)
        elif prefix != self.prefix_token_ids:
            raise RuntimeError(
                "target committed prefix mismatch; incremental verify cannot silently rebuild KV: "
                f"request_len={len(prefix)}, target_len={len(self.prefix_token_ids)}"
            )
        if not routes:
            raise ValueError("verify requires at least one route")
        if len(routes) != int(self.config.k):
            raise ValueError(f"verify route count does not match configured k: routes={len(routes)}, k={int(self.config.k)}")
        route_ids = [int(r.route_id) for r in routes]
        if len(set(route_ids)) != len(route_ids):
            raise ValueError("verify route ids must be unique")
        paths = [tuple(int(t) for t in r.token_ids) for r in routes]
        for r, p in zip(routes, paths):
            if r.draft_token_logprobs and len(r.draft_token_logprobs) != len(p):
                raise ValueError(
                    "draft_token_logprobs must be empty or match route depth: "
                    f"route_id={int(r.route_id)}, values={len(r.draft_token_logprobs)}, depth={len(p)}"
                )
        depths = {len(p) for p in paths}
        if len(depths) != 1:
            raise ValueError(f"all verify routes must have the same depth, got {sorted(depths)}")
        depth = next(iter(depths))
        if depth <= 0:
            raise ValueError("verify routes must contain at least one token")
        if int(depth) != int(self.config.d):
            raise ValueError(f"verify route depth does not match configured d: depth={int(depth)}, d={int(self.config.d)}")
        tree, route_nodes = build_deduplicated_tree_spec_from_paths(
            paths=paths, prefix_len=len(prefix), page_size=self.config.page_size, device=self.config.device
        )
        self._ensure_page_capacity(tree.total_pages)
        state = FullVerifyState(tree=tree, paged_prefix_kv=self._paged_prefix_kv)
        plan_prefill_wrapper(self._wrapper, tree, args=self.config, config=self.model.config, dtype=self.dtype)
        logits = run_full_verify(model=self.model, wrapper=self._wrapper, state=state, prefix_len=len(prefix),
                                 page_size=self.config.page_size, fused=self.fused_verify_step)
        device_inputs = self._device_selection_inputs(routes, paths, route_nodes) if logits.is_cuda else None
        if selected_path_max_tokens is not None and int(selected_path_max_tokens) <= 0:
            device_inputs = None  # the host path raises after the fallback decision, as the reference does
        if device_inputs is not None:
            # every route's committed length (truncation), so the device
            # commits the selected one without a host round trip
            commit_lens = [len(self._truncate_selected_path(token_ids=p, node_ids=nd, max_tokens=selected_path_max_tokens,
                                                            eos_token_id=eos_token_id)[0])
                           for p, nd in zip(paths, route_nodes)]
            scores, device_idx, device_count = self._score_select_commit(
                routes=routes, paths=paths, prefix_logits=self._prefix_logits[0], verify_logits=logits,
                route_to_node_paths=route_nodes, inputs=device_inputs, commit_lens=commit_lens,
                prefix_len=len(prefix), layers=self._paged_prefix_kv, kv_layout=self.kv_layout)
        else:
            scores = self._score_routes(routes=routes, paths=paths, prefix_logits=self._prefix_logits[0],
                                        verify_logits=logits, route_to_node_paths=route_nodes)
        best = max(scores, key=lambda s: (self._selection_score(s), s.draft_path_logprob, -s.route_id))
        selected, sampling_meta = self._select_route_with_metadata(
            scores, route_sampling_seed=route_sampling_seed, route_sampling_round=route_sampling_round
        )
        reason = self._fallback_reason(selected)
        if device_inputs is not None:
            host_idx = next(i for i, r in enumerate(routes) if int(r.route_id) == int(selected.route_id))
            host_count = 0 if reason is not None else commit_lens[host_idx]
            if (host_idx, host_count) != (device_idx, device_count):
                raise RuntimeError(
                    "device route selection disagrees with the host selection: device route index "
                    f"{device_idx} ({device_count} tokens), host {host_idx} ({host_count} tokens)")
        # the key order of target_runtime.py:235-252 (later keys override the
        # runtime metadata's)
        common = {
            **self.runtime_metadata(),
            "route_count": len(routes),
            "path_depth": int(depth),
            "node_count": int(tree.node_count),
            "unmerged_path_node_count": int(len(routes) * depth),
            "kv_len": int(tree.kv_len),
            "prefix_len_before": len(self.prefix_token_ids),
            "selection_policy": self._selection_policy_name(),
            "selection_score_name": "weighted_target_logprob" if self.score_weights is not None else "target_logprob",
            "fallback_threshold": self.fallback_threshold,
            "first_token_threshold": self.first_token_threshold,
            "fallback_ar_tokens": int(self.fallback_ar_tokens),
            **sampling_meta,
            **self._route_intervention_metadata(scores, selected),
        }
        best_meta = {
            "best_route_id": int(best.route_id),
            "best_selection_score": float(self._selection_score(best)),
            "best_first_token_logprob": None if best.first_token_logprob is None else float(best.first_token_logprob),
        }
        if reason is not None:
            generated = self._generate_fallback_ar(
                max_tokens=(self.fallback_ar_tokens if fallback_max_tokens is None
                            else min(int(fallback_max_tokens), self.fallback_ar_tokens)),
                eos_token_id=eos_token_id,
            )
            return TargetVerifyResult(
                selected_route_id=None,
                scores=scores,
                decision="fallback_ar",
                fallback_token_ids=tuple(generated),
                fallback_reason=reason,
                metadata={
                    **common,
                    "prefix_len_after": len(self.prefix_token_ids),
                    "target_kv_commit": "fallback_ar_in_place",
                    "target_reprefill_after_verify": False,
                    "fallback_triggered": True,
                    "fallback_reason": reason,
                    "fallback_token_count": len(generated),
                    **best_meta,
                    "fallback_ar_profile": self._last_fallback_ar_profile,
                },
            )
        idx = next(i for i, r in enumerate(routes) if int(r.route_id) == int(selected.route_id))
        path, nodes = self._truncate_selected_path(token_ids=paths[idx], node_ids=route_nodes[idx],
                                                   max_tokens=selected_path_max_tokens, eos_token_id=eos_token_id)
        self._commit_selected_path(token_ids=path, node_ids=nodes, verify_logits=logits,
                                   launch=device_inputs is None)
        return TargetVerifyResult(
            selected_route_id=selected.route_id,
            scores=scores,
            metadata={
                **common,
                "prefix_len_after": len(self.prefix_token_ids),
                "target_kv_commit": "selected_tree_path_in_place",
                "target_reprefill_after_verify": False,
                "fallback_triggered": False,
                **best_meta,
                "selected_route_id": int(selected.route_id),
                "selected_selection_score": float(self._selection_score(selected)),
                "selected_path_committed_tokens": len(path),
                "selected_path_was_truncated": len(path) != len(paths[idx]),
            },
        )

    # ------------------------------------------------------------ policies
    @staticmethod
    def _validate_score_weights(weights: Sequence[float] | None) -> tuple[float, ...] | None:
        if weights is None:
            return None
        values = tuple(float(v) for v in weights)
        if not values:
            return None
        if any(v < 0.0 for v in values):
            raise ValueError("score weights must be non-negative")
        total = sum(values)
        if total <= 0.0:
            raise ValueError("at least one score weight must be positive")
        return tuple(v / total for v in values)

    def _weights_for_depth(self, depth: int) -> tuple[float, ...] | None:
        if self.score_weights is None:
            return None
        if len(self.score_weights) != int(depth):
            raise ValueError(
                f"score weights must match verify route depth: weights={len(self.score_weights)}, depth={int(depth)}"
            )
        return self.score_weights

    def _selection_policy_name(self) -> str:
        if self.route_selection_policy == "first_route":
            return "diagnostic_first_payload_route"
        weighted = self.score_weights is not None
        if self.route_selection_policy == "target_sample":
            return "sample_weighted_target_route_score_distribution" if weighted else "sample_target_route_logprob_distribution"
        return "best_of_n_weighted_target_path_logprob" if weighted else "best_of_n_target_path_logprob"

    @staticmethod
    def _validate_route_selection_policy(policy: str) -> str:
        value = str(policy).strip().lower()
        if value not in ROUTE_POLICIES:
            raise ValueError("route_selection_policy must be one of: target_best, target_sample, first_route")
        return value

    @staticmethod
    def _validate_route_sampling_temperature(temperature: float) -> float:
        value = float(temperature)
        if not math.isfinite(value) or value <= 0.0:
            raise ValueError("route_sampling_temperature must be finite and positive")
        return value

    @staticmethod
    def _selection_score(score: TargetRouteScore) -> float:
        return float(score.target_logprob if score.selection_score is None else score.selection_score)

    def _select_route(self, scores, *, route_sampling_seed=None, route_sampling_round=None) -> TargetRouteScore:
        return self._select_route_with_metadata(
            scores, route_sampling_seed=route_sampling_seed, route_sampling_round=route_sampling_round
        )[0]

    def _select_route_with_metadata(self, scores, *, route_sampling_seed=None, route_sampling_round=None):
        if not scores:
            raise ValueError("cannot select from an empty route score list")
        if self.route_selection_policy == "first_route":
            return scores[0], self._route_sampling_disabled_metadata()
        if self.route_selection_policy == "target_sample":
            return self._sample_target_route(scores, route_sampling_seed=route_sampling_seed,
                                             route_sampling_round=route_sampling_round)
        best = max(scores, key=lambda s: (self._selection_score(s), s.draft_path_logprob, -s.route_id))
        return best, self._route_sampling_disabled_metadata()

    def _route_sampling_disabled_metadata(self) -> dict:
        return {
            "route_sampling_enabled": False,
            "route_sampling_scope": "verified_route_level_only",
            "route_sampling_seed": None,
            "route_sampling_round": None,
            "route_sampling_temperature": float(getattr(self, "route_sampling_temperature", 1.0)),
        }

    @staticmethod
    def _token_path_hash(token_ids: Sequence[int]) -> str:
        return hashlib.sha256(json.dumps([int(t) for t in token_ids], separators=(",", ":")).encode("utf-8")).hexdigest()

    def _route_intervention_metadata(self, scores: Sequence[TargetRouteScore],
                                     selected: TargetRouteScore) -> dict[str, object]:
        """Audit of the Target's choice against the first payload route
        ("route0") and the Drafter's own top route (highest current-path draft
        log-prob, earliest on ties), with the aggregated fields repeated at
        the top level (``target_runtime.py:567-660``)."""
        if not scores:
            raise ValueError("route intervention metadata requires non-empty scores")
        route0 = scores[0]
        by_draft = sorted(range(len(scores)), key=lambda i: (-float(scores[i].draft_path_logprob), i))
        rank = {int(scores[i].route_id): r for r, i in enumerate(by_draft, start=1)}
        draft_top = scores[by_draft[0]]
        sel_score = self._selection_score

        def summary(s: TargetRouteScore) -> dict[str, object]:
            return {
                "route_id": int(s.route_id),
                "token_path_hash": self._token_path_hash(s.token_ids),
                "first_token_id": int(s.token_ids[0]),
                "draft_rank": int(rank[int(s.route_id)]),
                "draft_first_token_logprob": s.draft_first_token_logprob,
                "draft_path_logprob": float(s.draft_path_logprob),
                "legacy_cumulative_draft_logprob": float(s.draft_logprob),
                "target_first_token_logprob": None if s.first_token_logprob is None else float(s.first_token_logprob),
                "target_logprob": float(s.target_logprob),
                "target_selection_score": float(sel_score(s)),
            }

        def delta(a, b):
            return None if a is None or b is None else float(a) - float(b)

        def versus(base: TargetRouteScore) -> dict[str, object]:
            return {
                "route_changed": tuple(selected.token_ids) != tuple(base.token_ids),
                "first_token_changed": int(selected.token_ids[0]) != int(base.token_ids[0]),
                "draft_first_token_logprob_delta": delta(selected.draft_first_token_logprob,
                                                         base.draft_first_token_logprob),
                "draft_path_logprob_delta": float(selected.draft_path_logprob) - float(base.draft_path_logprob),
                "legacy_cumulative_draft_logprob_delta": float(selected.draft_logprob) - float(base.draft_logprob),
                "target_first_token_logprob_delta": delta(selected.first_token_logprob, base.first_token_logprob),
                "target_path_logprob_delta": float(selected.target_logprob) - float(base.target_logprob),
                "target_selection_score_delta": sel_score(selected) - sel_score(base),
            }

        vs0, vs_top = versus(route0), versus(draft_top)
        return {
            "route_intervention": {
                "baseline": "route0",
                "draft_token_logprobs_available": bool(all(s.draft_token_logprobs for s in scores)),
                "route0_is_draft_top": int(route0.route_id) == int(draft_top.route_id),
                "route0": summary(route0),
                "draft_top": summary(draft_top),
                "selected": summary(selected),
                "selected_vs_route0": vs0,
                "selected_vs_draft_top": vs_top,
            },
            "selected_draft_rank": int(rank[int(selected.route_id)]),
            "route0_route_id": int(route0.route_id),
            "draft_top_route_id": int(draft_top.route_id),
            "selected_route_changed_from_route0": bool(vs0["route_changed"]),
            "selected_first_token_changed_from_route0": bool(vs0["first_token_changed"]),
            "selected_minus_route0_draft_first_token_logprob": vs0["draft_first_token_logprob_delta"],
            "selected_minus_route0_draft_logprob": float(vs0["draft_path_logprob_delta"]),
            "selected_minus_route0_target_selection_score": float(vs0["target_selection_score_delta"]),
        }

    def _sample_target_route(self, scores, *, route_sampling_seed, route_sampling_round):
        """Seeded route draw (``target_runtime.py:454-546``): canonical
        semantic order, softmax of score / temperature, SHA-256 uniform,
        inverse CDF."""
        if route_sampling_seed is None or route_sampling_round is None:
            raise ValueError(
                "target_sample requires explicit route_sampling_seed and route_sampling_round on every verify request"
            )
        rnd = int(route_sampling_round)
        if rnd < 0:
            raise ValueError("route_sampling_round must be non-negative")
        seed = int(route_sampling_seed)
        ordered = sorted(
            scores,
            key=lambda s: (tuple(int(t) for t in s.token_ids), float(s.draft_path_logprob), self._selection_score(s),
                           int(s.route_id)),
        )
        temp = float(getattr(self, "route_sampling_temperature", 1.0))
        logits = [self._selection_score(s) / temp for s in ordered]
        if any(math.isnan(v) for v in logits):
            raise ValueError("cannot sample a route from NaN target scores")
        pos_inf = [math.isinf(v) and v > 0.0 for v in logits]
        if any(pos_inf):
            probs = [1.0 / sum(pos_inf) if f else 0.0 for f in pos_inf]
        else:
            finite = [v for v in logits if math.isfinite(v)]
            if not finite:
                probs = [1.0 / len(ordered)] * len(ordered)
            else:
                top = max(finite)
                w = [0.0 if v == -math.inf else math.exp(v - top) for v in logits]
                probs = [x / sum(w) for x in w]
        material = f"atlas0709-target-route-sample-v1:{seed}:{rnd}".encode("utf-8")
        draw = (int.from_bytes(hashlib.sha256(material).digest()[:8], "big") + 0.5) / float(1 << 64)
        last = len(ordered) - 1
        idx, lo, hi, cum = last, 0.0, 1.0, 0.0
        for i, p in enumerate(probs):
            nxt = cum + p
            if draw < nxt or i == last:
                idx, lo, hi = i, cum, (nxt if i < last else 1.0)
                break
            cum = nxt
        chosen = ordered[idx]
        return chosen, {
            "route_sampling_enabled": True,
            "route_sampling_scope": "verified_route_level_only",
            "route_sampling_seed": seed,
            "route_sampling_round": rnd,
            "route_sampling_temperature": temp,
            "route_sampling_uniform": float(draw),
            "route_sampling_selected_probability": float(probs[idx]),
            "route_sampling_selected_cdf_low": float(lo),
            "route_sampling_selected_cdf_high": float(hi),
            "route_sampling_boundary_margin": float(min(draw - lo, hi - draw)),
            "route_sampling_ordered_candidates": [
                {"route_id": int(s.route_id), "token_path_hash": self._token_path_hash(s.token_ids),
                 "probability": float(p)}
                for s, p in zip(ordered, probs)
            ],
        }

    @staticmethod
    def _truncate_selected_path(*, token_ids, node_ids, max_tokens, eos_token_id):
        if len(token_ids) != len(node_ids) or not token_ids:
            raise ValueError("selected path tokens and node ids must have equal non-zero length")
        limit = len(token_ids) if max_tokens is None else min(len(token_ids), int(max_tokens))
        if limit <= 0:
            raise ValueError("selected_path_max_tokens must be positive")
        toks = [int(t) for t in token_ids[:limit]]
        if eos_token_id is not None and int(eos_token_id) in toks:
            toks = toks[: toks.index(int(eos_token_id)) + 1]
        return tuple(toks), tuple(int(n) for n in node_ids[: len(toks)])

    def _fallback_reason(self, selected: TargetRouteScore) -> str | None:
        if (self.first_token_threshold is not None and selected.first_token_logprob is not None
                and float(selected.first_token_logprob) < float(self.first_token_threshold)):
            return "first_token_below_threshold"
        if self.fallback_threshold is not None and self._selection_score(selected) < float(self.fallback_threshold):
            return "path_score_below_threshold"
        return None

    # ------------------------------------------------------------ scoring
    def _score_routes(self, *, routes, paths, prefix_logits, verify_logits, route_to_node_paths):
        """Per-token target log-probs: token 0 of a route reads the prefix
        logits, token t > 0 the verify row of the route's node t - 1
        (``target_runtime.py:722-765``).  One device launch per logits tensor
        and one device-to-host copy for all routes."""
        # One launch for both logits tensors: the verify rows, then the
        # prefix logits as row n_verify.
        vl = verify_logits.reshape(1, -1) if verify_logits.ndim == 1 else verify_logits
        rows, toks = _scoring_pairs(paths, route_to_node_paths, int(vl.shape[0]))
        values = gather_token_logprobs(vl, rows, toks, extra_logits=prefix_logits).cpu().numpy()
        return self._route_scores_from_values(routes, paths, values, verify_logits.dtype)

    def _rounding_code(self, dtype: torch.dtype) -> int:
        if self.match_logits_dtype_rounding and dtype == torch.float16:
            return _lib.ROUND_F16
        if self.match_logits_dtype_rounding and dtype == torch.bfloat16:
            return _lib.ROUND_BF16
        return _lib.ROUND_NONE

    def _route_score_parts(self, routes, paths) -> list[tuple[int, tuple | None, dict]]:
        """The parts of each route's TargetRouteScore that do not depend on the
        scores: (depth, weights or None, the fixed fields)."""
        parts = []
        weights_of: dict[int, tuple[float, ...] | None] = {}
        for route, path in zip(routes, paths):
            d = len(path)
            if d not in weights_of:
                weights_of[d] = self._weights_for_depth(d)
            weights = weights_of[d]
            parts.append((d, weights, dict(
                route_id=int(route.route_id), token_ids=tuple(map(int, path)),
                draft_logprob=float(route.draft_logprob), score_weights=() if weights is None else tuple(weights),
                draft_token_logprobs=tuple(map(float, route.draft_token_logprobs)))))
        return parts

    def _route_scores_from_values(self, routes, paths, values: np.ndarray, dtype: torch.dtype, *,
                                  parts=None, rounded: bool = False):
        """The routes' TargetRouteScores from the scoring launch's fp32 values
        (every route's first token, then each route's other tokens).
        ``rounded``: the values are already rounded to the logits dtype;
        ``parts``: ``_route_score_parts(routes, paths)``, when built ahead."""
        if not rounded:
            rounding = self._rounding_code(dtype)
            if rounding == _lib.ROUND_F16:
                # The reference reads log_softmax outputs in the logits dtype.
                values = values.astype(np.float16).astype(np.float32)
            elif rounding == _lib.ROUND_BF16:
                values = torch.from_numpy(values).to(torch.bfloat16).float().numpy()
        vals = values.tolist()
        if parts is None:
            parts = self._route_score_parts(routes, paths)
        scores, k = [], len(paths)
        for i, (d, weights, fixed) in enumerate(parts):
            rest = max(d - 1, 0)
            lps = (vals[i], *vals[k : k + rest])
            k += rest
            target = sum(lps)
            sel = target if weights is None else sum(w * v for w, v in zip(weights, lps))
            scores.append(_route_score(target_logprob=target, token_logprobs=lps, first_token_logprob=lps[0],
                                       selection_score=sel, **fixed))
        return scores

    # ------------------------------------------------------------ device selection
    def _device_selection_inputs(self, routes, paths, route_to_node_paths):
        """The host inputs of the device selection (policy, weights, draft
        path log-probs, route ids, node table), or None when this verify's
        selection stays on the host: target_sample, routes or depth beyond
        the selection launch's limits, or a NaN draft log-prob (Python's
        tuple comparison treats one NaN object as equal to itself)."""
        if not self.device_route_selection:
            return None
        policy = {"target_best": _lib.SELECT_TARGET_BEST, "first_route": _lib.SELECT_FIRST_ROUTE}.get(
            self.route_selection_policy)
        k, d = len(paths), len(paths[0])
        if policy is None or k > _lib.SELECT_MAX_ROUTES or d > _lib.SELECT_MAX_DEPTH or \
                k * d > _lib.SELECT_MAX_ENTRIES:
            return None
        weights = self._weights_for_depth(d)
        if weights is not None and len(weights) != d:
            return None
        nodes = [int(x) for path_nodes in route_to_node_paths for x in path_nodes]
        if len(nodes) != k * d or max(nodes) > 32767:
            return None
        draft = [float(sum(map(float, r.draft_token_logprobs))) if r.draft_token_logprobs else float(r.draft_logprob)
                 for r in routes]
        if any(math.isnan(x) for x in draft):
            return None
        return policy, weights, draft, [int(r.route_id) for r in routes], nodes

    def _score_select_commit(self, *, routes, paths, prefix_logits, verify_logits, route_to_node_paths, inputs,
                             commit_lens, prefix_len, layers, kv_indptr=None, kv_indices=None, kv_layout="NHD",
                             before_commit=None, then=None):
        """Scoring, route selection and the commit, queued in stream order:
        the scoring launch, the selection launch (``atlas_route_select``: the
        selected route and its commit positions, or none on a fallback; it
        also writes the values, rounded to the logits dtype, and the selection
        to mapped host memory), the
        commit of the selected route (``commit_lens[r]`` tokens of route r;
        rows past the count copy onto themselves) and ``then()``; then the
        host waits for the selection launch alone.  ``before_commit`` and
        ``then`` (optional) queue the caller's own work around the commit
        launch.  Returns the routes' scores and the device's (route index,
        committed count)."""
        policy, weights, draft, route_ids, nodes = inputs
        vl = verify_logits.reshape(1, -1) if verify_logits.ndim == 1 else verify_logits
        device = vl.device
        k, d = len(paths), len(paths[0])
        rows, toks = _scoring_pairs(paths, route_to_node_paths, int(vl.shape[0]))
        n = len(rows)
        # values, then the selection result (two int32)
        buf = torch.empty(n + 2, dtype=torch.float32, device=device)
        gather_token_logprobs(vl, rows, toks, extra_logits=prefix_logits, out=buf[:n])
        pos = torch.empty(2 * d, dtype=torch.int64, device=device)
        c_double, c_i64, c_i32 = ctypes.c_double, ctypes.c_int64, ctypes.c_int32
        thr_p, thr_f = self.fallback_threshold, self.first_token_threshold
        readback = self._readback_buffer()
        rc = _lib.load().atlas_route_select(
            _lib.ptr(buf), k, d, policy, self._rounding_code(verify_logits.dtype),
            (c_double * d)(*weights) if weights is not None else None, 0 if weights is None else d,
            (c_double * k)(*draft), (c_i64 * k)(*route_ids), (c_i32 * k)(*commit_lens), (c_i32 * (k * d))(*nodes),
            int(thr_p is not None), float(thr_p or 0.0), int(thr_f is not None), float(thr_f or 0.0), int(prefix_len),
            _lib.ptr(pos), _lib.ptr(pos[d:]), _lib.ptr(buf[n:]), readback.device_ptr, _lib.stream_of(device))
        _lib.check(rc, "atlas_route_select")
        done = self._readback_event()
        done.record()
        # the commit hazards of every route's committed rows, decided on the host
        staging = any(
            kv_ops.commit_positions_need_staging([prefix_len + x for x in route_to_node_paths[r][:commit_lens[r]]],
                                                 range(prefix_len, prefix_len + commit_lens[r]))
            for r in range(k))
        if before_commit is not None:
            before_commit()
        kv_ops.commit_paged(layers, pos[:d], pos[d:], kv_indptr=kv_indptr, kv_indices=kv_indices,
                            needs_staging=staging, kv_layout=kv_layout)
        if then is not None:
            then()
        parts = self._route_score_parts(routes, paths)
        done.synchronize()
        host_np = readback.np
        chosen, count = host_np[n:n + 2].view(np.int32).tolist()
        # the launch wrote the values rounded to the logits dtype
        scores = self._route_scores_from_values(routes, paths, host_np[:n], verify_logits.dtype, parts=parts,
                                                rounded=True)
        return scores, chosen, count

    def _readback_buffer(self) -> "_lib.MappedReadback":
        """The mapped read-back buffer: room for the largest selection the
        launch accepts (its values and the two result words)."""
        buf = getattr(self, "_readback", None)
        if buf is None:
            buf = self._readback = _lib.MappedReadback(_lib.SELECT_MAX_ENTRIES + 2)
        return buf

    def _readback_event(self) -> torch.cuda.Event:
        ev = getattr(self, "_readback_done", None)
        if ev is None:
            ev = self._readback_done = torch.cuda.Event()
        return ev

    # ------------------------------------------------------------ fallback AR
    def _generate_fallback_ar(self, *, max_tokens: int, eos_token_id: int | None) -> list[int]:
        """Greedy decode of up to ``max_tokens`` tokens on the committed prefix
        in place (``target_runtime.py:767-851``): the first token is the
        argmax of the prefix logits; each step plans the paged decode wrapper
        for the grown sequence, runs one decode forward (its K/V appended to
        the prefix pages) and keeps its logits as the next prefix logits.
        Stops after an EOS token."""
        if self._paged_prefix_kv is None or self._prefix_logits is None:
            raise RuntimeError("target fallback AR requires initialized prefix KV")
        max_tokens = int(max_tokens)
        if max_tokens <= 0:
            return []
        prefix_len = len(self.prefix_token_ids)
        self._ensure_page_capacity(math.ceil((prefix_len + max_tokens) / int(self.config.page_size)))
        generated: list[int] = []
        input_ids = next_argmax_inputs(self._prefix_logits)
        was_cached = self._fallback_decode_wrapper is not None
        profile = self.profile_fallback_ar
        setup_s = plan_s = model_s = 0.0
        t0 = self._profile_clock() if profile else 0.0
        if self._fallback_decode_wrapper is None:
            self._fallback_decode_wrapper = make_decode_wrapper(args=self.config, kv_layout=self.kv_layout)
        if profile:
            setup_s = self._profile_clock() - t0
        wrapper = self._fallback_decode_wrapper
        for step_idx in range(max_tokens):
            token_id = int(input_ids.reshape(-1)[0].detach().cpu())
            generated.append(token_id)
            t0 = self._profile_clock() if profile else 0.0
            plan_decode_wrapper(wrapper, seq_len=prefix_len + step_idx + 1, args=self.config,
                                config=self.model.config, dtype=self.dtype)
            if profile:
                t1 = self._profile_clock()
                plan_s += t1 - t0
            logits = run_full_ar_decode(model=self.model, wrappers=[wrapper],
                                        state=FullDecodeState(input_ids=input_ids,
                                                              paged_prefix_kv=self._paged_prefix_kv),
                                        prefix_len=prefix_len + step_idx, page_size=self.config.page_size)
            if profile:
                model_s += self._profile_clock() - t1
            self._prefix_logits = logits.detach()
            if eos_token_id is not None and token_id == int(eos_token_id):
                break
            input_ids = next_argmax_inputs(logits)
        self.prefix_token_ids = (*self.prefix_token_ids, *generated)
        self._committed_verify_rounds += 1
        self._last_fallback_ar_profile = (
            {"enabled": True, "wrapper_was_cached": was_cached, "wrapper_setup_seconds": setup_s,
             "decode_plan_seconds": plan_s, "model_forward_seconds": model_s, "token_count": len(generated)}
            if profile else None
        )
        return generated

    def _profile_clock(self) -> float:
        device = torch.device(self.config.device)
        if device.type == "cuda" and torch.cuda.is_available():
            torch.cuda.synchronize(device)
        return time.perf_counter()

    # ------------------------------------------------------------ KV state
    def _ensure_page_capacity(self, required_pages: int) -> None:
        """Grow every layer to ``required_pages`` pages, keeping the existing
        pages (``target_runtime.py:858-871``)."""
        if self._paged_prefix_kv is None:
            raise RuntimeError("target prefill must initialize paged prefix KV")
        required_pages = int(required_pages)
        grown = []
        for layer_kv in self._paged_prefix_kv:
            if int(layer_kv.shape[0]) >= required_pages:
                grown.append(layer_kv)
                continue
            expanded = torch.zeros((required_pages, *layer_kv.shape[1:]), dtype=layer_kv.dtype, device=layer_kv.device)
            expanded[: int(layer_kv.shape[0])].copy_(layer_kv)
            grown.append(expanded)
        self._paged_prefix_kv = grown

    def _commit_selected_path(self, *, token_ids, node_ids, verify_logits, launch: bool = True) -> None:
        """Compact the selected nodes' KV into the committed prefix (every
        layer, one launch), extend the prefix and keep the last node's logits
        as the next prefix logits (``target_runtime.py:873-920``).
        ``launch=False``: the device selection already queued the copy."""
        if self._paged_prefix_kv is None:
            raise RuntimeError("target paged prefix KV is not initialized")
        if len(token_ids) != len(node_ids) or not node_ids:
            raise ValueError("selected path tokens and node ids must have equal non-zero length")
        if launch:
            prefix_len = len(self.prefix_token_ids)
            src = [prefix_len + int(n) for n in node_ids]
            dst = list(range(prefix_len, prefix_len + len(node_ids)))
            kv_ops.commit_paged(self._paged_prefix_kv, src, dst, kv_layout=self.kv_layout)
        self.prefix_token_ids = (*self.prefix_token_ids, *(int(t) for t in token_ids))
        self._prefix_logits = verify_logits[int(node_ids[-1])].detach().unsqueeze(0)
        self._committed_verify_rounds += 1


def _legacy_layer_kv(past, layer_idx: int):
    if hasattr(past, "layers"):
        layer = past.layers[layer_idx]
        for kn, vn in (("keys", "values"), ("key_cache", "value_cache")):
            if hasattr(layer, kn):
                return getattr(layer, kn), getattr(layer, vn)
    if hasattr(past, "key_cache"):
        return past.key_cache[layer_idx], past.value_cache[layer_idx]
    if hasattr(past, "to_legacy_cache"):
        legacy = past.to_legacy_cache()
        return legacy[layer_idx][0], legacy[layer_idx][1]
    return past[layer_idx][0], past[layer_idx][1]
