"""Install this package under the reference's import names.

The reference runtime imports its hot-path pieces as ``atlas_0709.<module>``
names (and FlashInfer's wrapper through ``flashinfer``).  Two ways to drop
this package in:

* the reference package is importable: ``install_atlas_0709_alias()``
  replaces, inside the reference's own modules, exactly the hot-path names
  listed in ``HOT_PATH`` with this package's versions; every other name of
  those modules (model runners, RPC, configs) stays the reference's;
* it is not: the same call registers this package's modules under the
  reference's module names in ``sys.modules``.

The reference's wrapper factories (``make_prefill_wrapper``,
``plan_prefill_wrapper``, ``make_decode_wrapper``, ``plan_decode_wrapper``,
``flashinfer_full_verify.py:877-927``) are always replaced, so the verify and
fallback-decode attention run on the gfx950 kernels whether or not some
``flashinfer`` is importable: this package's factories ignore the
``flashinfer`` module they are handed.

``flashinfer=True`` also registers a ``flashinfer`` module exposing
``BatchPrefillWithPagedKVCacheWrapper``, ``BatchDecodeWithPagedKVCacheWrapper``
and ``packbits`` backed by the gfx950 kernels, when no ``flashinfer`` is
importable, for code that constructs the wrappers by name (the reference's
``import flashinfer`` in ``target_runtime.py:99`` and
``flashinfer_full_verify.py:502-507``).  An importable ``flashinfer`` is left
in place; what constructs its wrappers directly (SGLang's own attention
backend inside the Drafter's model forward) then still runs it.
"""

from __future__ import annotations

import importlib
import sys
import types as _types

_PKG = __name__.rsplit(".", 1)[0]

# reference module -> (this package's module, names on the hot path)
HOT_PATH: dict[str, tuple[str, tuple[str, ...]]] = {
    "atlas_0709.flashinfer_paged.paged_metadata": (
        "flashinfer_paged.paged_metadata", ("FlashInferPagedKVMetadata", "build_flashinfer_paged_kv_metadata")),
    "atlas_0709.flashinfer_paged.types": (
        "flashinfer_paged.types", ("DecodePhase", "PrefixKVView", "RouteKVView", "RouteState", "DraftPrefixState",
                                   "FrontierDecodeOutput", "PendingCandidate", "PendingCandidateBatch",
                                   "FrontierSelectionStats", "FrontierStepOutput")),
    "atlas_0709.flashinfer_paged.kv": ("flashinfer_paged.kv", ("KVTreeNode", "KVTreeStore")),
    "atlas_0709.flashinfer_paged.sampling": (
        "flashinfer_paged.sampling", ("DrafterSamplingConfig", "DrafterSamplingContext", "batch_parent_token_candidates",
                                      "single_parent_token_candidates")),
    "atlas_0709.flashinfer_paged.utils": (
        "flashinfer_paged.utils", ("topk_logprobs", "global_topk_candidates", "stable_candidate_order",
                                   "global_topk_candidate_indices", "per_root_topk_candidate_indices",
                                   "group_candidates_by_stage1_root", "topk_pairs_to_python", "logprob_of_token")),
    "atlas_0709.flashinfer_paged.frontier": (
        "flashinfer_paged.frontier", ("GlobalTopKSelection", "PerStage1RootTopKSelection",
                                      "build_pending_candidate_batch", "materialize_pending_candidate_batch",
                                      "collect_pending_candidates", "advance_frontier_one_token")),
    "atlas_0709.flashinfer_paged.sglang_runtime": (
        "flashinfer_paged.sglang_runtime", ("SGLangRoutePoolBridge", "SGLangRouteRow", "SGLangFlashInferFrontierModelBackend")),
    "atlas_0709.flashinfer_full_verify": (
        "flashinfer_full_verify", ("TreeSpec", "build_path_tree_tokens_from_paths", "build_deduplicated_path_tree_tokens",
                                   "ancestors_inclusive", "build_tree_spec_from_paths",
                                   "build_deduplicated_tree_spec_from_paths", "prefix_layer_to_paged_kv",
                                   "write_suffix_kv", "first_tensor", "packbits", "make_prefill_wrapper",
                                   "plan_prefill_wrapper", "make_decode_wrapper", "plan_decode_wrapper")),
    "atlas_0709.target_runtime": (
        "target_runtime", ("VerifyRoutePayload", "verify_payload_from_mapping",
                           "DirectFlashInferMaskedTreeVerifyBackend")),
    "atlas_0709.types": ("types", ("PrefixState", "TargetRouteScore", "TargetVerifyResult")),
}


def _ours(rel: str):
    return importlib.import_module(f"{_PKG}.{rel}")


def install_atlas_0709_alias(*, flashinfer: bool = False) -> dict[str, str]:
    """Returns {reference module name: "patched" | "registered"}, plus
    ``"flashinfer"``: ``"registered"`` or ``"present"`` when
    ``flashinfer=True``.  Call it before the reference's entry modules
    (``target_server``, ``rpc``, ``distributed_system``) are imported: they
    bind the hot-path names at import time."""
    done: dict[str, str] = {}
    for ref_name, (rel, names) in HOT_PATH.items():
        ours = _ours(rel)
        try:
            ref_mod = importlib.import_module(ref_name)
        except ImportError:
            ref_mod = None
        if ref_mod is not None and ref_mod is not ours:
            for name in names:
                setattr(ref_mod, name, getattr(ours, name))
            done[ref_name] = "patched"
        else:
            sys.modules[ref_name] = ours
            parent, _, leaf = ref_name.rpartition(".")
            _ensure_package(parent)
            setattr(sys.modules[parent], leaf, ours)
            done[ref_name] = "registered"
    if flashinfer:
        try:
            importlib.import_module("flashinfer")
        except ImportError:
            shim = _types.ModuleType("flashinfer")
            shim.BatchPrefillWithPagedKVCacheWrapper = _ours("tree_attention").BatchPrefillWithPagedKVCacheWrapper
            shim.BatchDecodeWithPagedKVCacheWrapper = _ours("decode_attention").BatchDecodeWithPagedKVCacheWrapper
            shim.packbits = _ours("flashinfer_full_verify").packbits
            shim.__doc__ = "FlashInfer verify and decode attention names backed by the gfx950 paged-attention kernels."
            sys.modules["flashinfer"] = shim
            done["flashinfer"] = "registered"
        else:
            done["flashinfer"] = "present"
    return done


def _ensure_package(name: str) -> None:
    if not name or name in sys.modules:
        return
    parent, _, leaf = name.rpartition(".")
    _ensure_package(parent)
    mod = _types.ModuleType(name)
    mod.__path__ = []  # a namespace for the registered submodules
    sys.modules[name] = mod
    if parent:
        setattr(sys.modules[parent], leaf, mod)
