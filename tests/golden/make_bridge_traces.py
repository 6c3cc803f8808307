"""Writes ``bridge_traces.json``: the traces of ``bridge_trace.run`` over the
reference's ``KVTreeStore`` (``flashinfer_paged/kv.py``),
``SGLangRoutePoolBridge`` and ``SGLangFlashInferFrontierModelBackend``
(``flashinfer_paged/sglang_runtime.py``), on the oracle's host pools.

Run from the repository root, in a checkout that has the reference beside it:

    python tests/golden/make_bridge_traces.py [REFERENCE_SRC]

REFERENCE_SRC defaults to /root/reference/src.  Only torch-only reference
modules are imported; nothing of SGLang or FlashInfer is needed, except that
the reference's EXTEND forward builds SGLang's ForwardBatch.  The fallback
EXTEND here therefore makes the bridge calls of
``append_known_tokens_as_prefix`` (``sglang_runtime.py:1172-1254``) in their
order -- request row, ``allocate_extend_slots``, ``_write_req_token_row``, the
forward's KV write of the suffix slots, row free, ``set_prefix_slots``, prefix
tokens -- with the model's KV write made by the same stand-in model as the
decode steps.
"""

from __future__ import annotations

import json
import os
import sys
from types import SimpleNamespace

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

import bridge_trace  # noqa: E402
from oracle import route_pool  # noqa: E402


def reference_extend(backend, tokens) -> None:
    pool = backend.route_pool
    prefix_slots = pool.prefix_slot_ids
    prefix_len = len(backend.prefix_token_ids)
    seq_len = prefix_len + len(tokens)
    handle = SimpleNamespace(rid="atlas-known-prefix-extend", req_pool_idx=None)
    row = int(pool.req_to_token_pool.alloc([handle])[0])
    handle.req_pool_idx = row
    try:
        last = prefix_slots[-1:].to(torch.long)
        suffix = pool.allocate_extend_slots(prefix_lens=[prefix_len], seq_lens=[seq_len], last_locs=last)
        full = torch.cat([prefix_slots, suffix], dim=0)
        pool._write_req_token_row(row, full)
        backend.executor.forward_extend(input_ids=torch.tensor(tokens), out_cache_loc=suffix,
                                        positions=torch.arange(prefix_len, seq_len),
                                        req_pool_indices=torch.tensor([row]),
                                        seq_lens_cpu=torch.tensor([seq_len]))
    finally:
        pool.req_to_token_pool.free(handle)
    pool.set_prefix_slots(full)
    backend.prefix_token_ids = (*backend.prefix_token_ids, *[int(t) for t in tokens])


def main() -> None:
    src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src"
    sys.path.insert(0, src)
    from atlas_0709.flashinfer_paged import kv, sglang_runtime, types

    mods = SimpleNamespace(KVTreeStore=kv.KVTreeStore, SGLangRoutePoolBridge=sglang_runtime.SGLangRoutePoolBridge,
                           SGLangFlashInferFrontierModelBackend=sglang_runtime.SGLangFlashInferFrontierModelBackend,
                           DecodePhase=types.DecodePhase, RouteState=types.RouteState)
    out = {name: bridge_trace.run(mods, name, reference_extend, oracle_pools=route_pool)
           for name in bridge_trace.SCENARIOS}
    path = os.path.join(HERE, "bridge_traces.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print(f"wrote {path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
