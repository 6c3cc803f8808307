"""The allocation-free verify attention entry point (atlas_tree_verify_attn_noalloc)
against atlas_tree_verify_attn with a caller workspace: same plan, same
kernels, so outputs and LSEs must be equal bit for bit, on two calls in a row
(the second one smaller, reusing the device scratch the first one filled),
and plans beyond the scratch are refused."""

import ctypes

import pytest
import torch

from helpers import pkg

pytestmark = pytest.mark.gpu


def _case(dev, prefix_len, routes, seed):
    ffv = pkg("flashinfer_full_verify")
    wl = pkg("workloads")
    geom = wl.LLAMA_8B
    ps = 16
    spec, _ = ffv.build_deduplicated_tree_spec_from_paths(paths=routes, prefix_len=prefix_len, page_size=ps,
                                                          device=dev)
    kv_len = prefix_len + spec.node_count
    pages = (kv_len + ps - 1) // ps
    g = torch.Generator(device=dev).manual_seed(seed)
    kv = (torch.randn((pages + 8, 2, ps, geom.kv_heads, geom.head_dim), generator=g, device=dev) * 0.5).half()
    perm = torch.randperm(pages + 8, generator=torch.Generator().manual_seed(seed))[:pages]
    kv_indices = perm.to(torch.int32).to(dev)
    q = (torch.randn((spec.node_count, geom.q_heads, geom.head_dim), generator=g, device=dev) * 0.5).half()
    ws = torch.empty(64 * 1024 * 1024, dtype=torch.uint8, device=dev)
    w = ffv.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    last = torch.tensor([kv_len - (pages - 1) * ps], dtype=torch.int32, device=dev)
    w.plan(spec.qo_indptr, torch.tensor([0, pages], dtype=torch.int32, device=dev), kv_indices, last,
           geom.q_heads, geom.kv_heads, geom.head_dim, ps, custom_mask=spec.bool_mask, causal=False,
           q_data_type=torch.float16)
    return w, q, kv


def _noalloc(w, q, kv, out, lse, partial_rows=None):
    lib_mod = pkg("_lib")
    plan = w.current_plan
    es = kv.element_size()
    rc = lib_mod.load().atlas_tree_verify_attn_noalloc(
        lib_mod.ptr(q), q.stride(0), q.stride(1), lib_mod.ptr(kv), kv.stride(0) * es, kv.stride(1) * es,
        kv.stride(2) * es, kv.stride(3) * es, lib_mod.ptr(plan.qo_indptr), lib_mod.ptr(plan.kv_indptr), lib_mod.ptr(plan.kv_indices),
        plan.device_view(plan.kv_len_offset), plan.mask_mode, lib_mod.ptr(plan.tree_mask),
        plan.device_view(plan.col_offset), plan.mask_words, plan.device_view(plan.work_offset), plan.num_work,
        lib_mod.ptr(plan.page_windows) if plan.page_windows is not None else None,
        plan.device_view(plan.merge_offset) if plan.num_merge else None, plan.num_merge,
        plan.partial_rows if plan.num_merge else 0, plan.max_rows,
        plan.num_qo_heads, plan.num_kv_heads, plan.head_dim, plan.page_size, ctypes.c_float(plan.sm_scale),
        lib_mod.dtype_code(q.dtype), lib_mod.ptr(out), out.stride(0), out.stride(1), lib_mod.ptr(lse),
        plan.partial_rows if partial_rows is None else partial_rows, lib_mod.stream_of(q.device))
    return rc


def test_noalloc_equals_workspace_entry_point_twice(dev):
    forest = pkg("workloads").forest_routes(0)
    cases = [(16384, forest, 1), (1000, [(1, 2, 3, 4), (1, 2, 5, 6), (7, 8, 9, 10)], 2)]
    for prefix_len, routes, seed in cases:
        w, q, kv = _case(dev, prefix_len, routes, seed)
        plan = w.current_plan
        print(f"no-alloc attention: prefix {prefix_len}, {plan.num_work} items, {plan.num_merge} merges, "
              f"{plan.partial_rows} partial rows", flush=True)
        assert plan.num_merge > 0 and plan.partial_rows > 0
        ref_out, ref_lse = w.run(q, kv, return_lse=True)
        out = torch.full_like(ref_out, float("nan"))
        lse = torch.full_like(ref_lse, float("nan"))
        rc = _noalloc(w, q, kv, out, lse)
        pkg("_lib").check(rc, "atlas_tree_verify_attn_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
        assert torch.equal(lse.view(torch.int32), ref_lse.view(torch.int32))


def test_noalloc_refuses_plans_beyond_the_scratch(dev):
    lib_mod = pkg("_lib")
    w, q, kv = _case(dev, 2000, [(1, 2, 3, 4), (5, 6, 7, 8)], 3)
    out = torch.empty_like(q)
    lse = torch.empty((q.shape[0], q.shape[1]), dtype=torch.float32, device=dev)
    too_many = lib_mod.ATTN_SCRATCH_BYTES // (2 * 128 + 4) + 1
    rc = _noalloc(w, q, kv, out, lse, partial_rows=too_many)
    assert rc == lib_mod.ATLAS_EINVAL
    assert b"scratch" in lib_mod.load().atlas_last_error()
