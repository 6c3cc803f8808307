"""CPU restatement of the reference's paged-KV tree path -- TEST INFRASTRUCTURE.

This package checks the product and is never part of it: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it.  Every function cites the reference file:line it restates (paths relative
to the reference's ``src/atlas_0709/``).  Integer and byte work is numpy;
attention is the closed form ``softmax(Q K^T * scale + M) V`` in float64 (or
float32 when timed as the CPU baseline).

Pinning (what each function is checked against in ``tests/``):

* ``paged_metadata``      -- reference literals (test_paged_attention_metadata.py:24-67)
* ``dedup_tree``          -- reference literals (test_tree_dedup.py:6-35) + brute force
* ``ancestor_mask``       -- closed form from parents + brute-force ancestor walk
* ``masked_attention``    -- torch SDPA with a bool mask, page-permutation
                             invariance, one-node = decode, uniform-V identity
* ``write_suffix`` / ``commit`` / ``grow_capacity``
                          -- reference literals (test_target_kv_commit.py:28-73)
* ``move_kv``             -- reference FakeKVCache semantics and move lists
                             (test_tail_page_cow.py:14-16, :77-79, :111-113, :193-195)
* ``prune``               -- reference literals (test_tail_page_cow.py:241-293)
* ``PagedAllocator``      -- documented SGLang paged-allocator policy; decode /
                             extend slot rules checked against brute force.
                             SGLang's own allocator is absent: parity unpinned
                             against it (only against this restated policy).
* ``scoring``             -- reference literals (test_target_kv_commit.py:76-367)
* ``frontier``            -- reference literals of the frontier selection tests
                             (test_paged_frontier_selection.py:79-130, :189-275),
                             the Python-object order by brute force (utils.py:27-43),
                             torch ``topk(log_softmax)``: fp32 exactly, 16-bit rows
                             against torch's fp32 log-softmax rounded once (torch's
                             device kernel rounds there; its CPU 16-bit path does
                             not). The order of equal log-probs inside a parent's
                             top-k (ascending token) is parity unpinned: torch.topk
                             leaves it open.
* ``rope.apply_rope``     -- torch's own 16-bit elementwise ops on the CPU
                             (q * cos + rotate_half(q) * sin, bit for bit, f16
                             and bf16), the identity at angle 0, rotate_half at
                             cos 0 / sin 1, and a plain fp32 rotation within
                             one 16-bit rounding step
* ``route_pool``          -- host pools for the route-pool trace: the
                             ``PagedAllocator`` policy above, slot contents as
                             value ids with ``move_kv_cache`` = FakeKVCache
                             semantics (test_tail_page_cow.py:14-16), request
                             rows.  The bridge's host logic run over them is
                             pinned by the reference's bridge-test literals
                             (test_tail_page_cow.py:61-383,
                             test_req_row_incremental.py:151-473) and by the
                             content invariant "slot path of every route holds
                             the value ids of its prefix and nodes".
"""
