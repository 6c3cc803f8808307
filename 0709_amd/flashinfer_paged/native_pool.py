"""Native device pools behind the allocator / KV-pool / request-row protocols
the route-pool bridge drives (reference ``sglang_runtime.py:578-695``,
``:1059-1075``; SGLang 0.5.14's ``PagedTokenToKVPoolAllocator``,
``MHATokenToKVPool`` and ``ReqToTokenPool`` are absent here).

* ``NativePagedAllocator`` -- free list of page ids in HBM.  Policy: pages
  1..num_pages start free in ascending order (page 0 is the padding page);
  ``alloc`` takes pages from the head; ``free`` prepends the sorted unique
  pages of the freed slots; ``alloc_decode`` / ``alloc_extend`` assign slots
  on the device (gfx950 kernels) and advance the head by the page count the
  host derives from the CPU lengths.  The list lives at the tail of a
  num_pages-long buffer, so a prepend never runs out of room.
* ``NativeTokenToKVPool`` -- per-layer flat K and V pools ``[slots, Hkv, D]``
  in one allocation; ``move_kv_cache`` and ``set_kv_buffer`` are the all-layer
  HIP move / append kernels.
* ``NativeReqToTokenPool`` -- ``req_to_token`` table with an ascending free
  list of rows.
"""

from __future__ import annotations

from typing import Any, Sequence

import torch

from .. import _lib, kv_ops


class NativeTokenToKVPool:
    def __init__(self, *, size: int, page_size: int, dtype: torch.dtype, head_num: int, head_dim: int,
                 layer_num: int, device: str | torch.device) -> None:
        self.size = int(size)
        self.page_size = int(page_size)
        self.dtype = dtype
        self.head_num = int(head_num)
        self.head_dim = int(head_dim)
        self.layer_num = int(layer_num)
        self.device = torch.device(device)
        slots = self.size + self.page_size  # page 0 is the padding page
        self._storage = torch.zeros((2, self.layer_num, slots, self.head_num, self.head_dim), dtype=dtype,
                                    device=self.device)
        self.k_buffer = list(self._storage[0].unbind(0))
        self.v_buffer = list(self._storage[1].unbind(0))
        # the layer tables every all-layer call passes (fixed for the pool's life)
        self._geom = kv_ops.token_pool_geometry(self.k_buffer[0])
        self._k_ptrs = _lib.ptr_array([int(t.data_ptr()) for t in self.k_buffer])
        self._v_ptrs = _lib.ptr_array([int(t.data_ptr()) for t in self.v_buffer])

    def get_key_buffer(self, layer_id: int) -> torch.Tensor:
        return self.k_buffer[int(layer_id)]

    def get_value_buffer(self, layer_id: int) -> torch.Tensor:
        return self.v_buffer[int(layer_id)]

    def get_kv_buffer(self, layer_id: int):
        return self.k_buffer[int(layer_id)], self.v_buffer[int(layer_id)]

    def move_kv_cache(self, tgt_loc: torch.Tensor, src_loc: torch.Tensor) -> None:
        """``K[tgt] = K[src]; V[tgt] = V[src]`` in every layer, one launch."""
        kv_ops.move_slots(self.k_buffer, self.v_buffer, tgt_loc, src_loc,
                          layer_tables=(self._k_ptrs, self._v_ptrs, self._geom))

    def set_kv_buffer(self, layer: Any, loc: torch.Tensor, cache_k: torch.Tensor, cache_v: torch.Tensor, *args,
                      **kwargs) -> None:
        layer_id = int(getattr(layer, "layer_id", layer))
        kv_ops.append_token_pool([self.k_buffer[layer_id]], [self.v_buffer[layer_id]],
                                 [cache_k.reshape(-1, self.head_num, self.head_dim)],
                                 [cache_v.reshape(-1, self.head_num, self.head_dim)], loc)

    def set_kv_buffer_all_layers(self, loc: torch.Tensor, k_rows: Sequence[torch.Tensor],
                                 v_rows: Sequence[torch.Tensor]) -> None:
        """``set_kv_buffer`` of every layer in one launch (rows ``[n, Hkv, D]``
        per layer, in the pool dtype)."""
        if len(k_rows) != self.layer_num or len(v_rows) != self.layer_num:
            raise ValueError(f"one K and one V source per layer ({self.layer_num}) are required")
        kv_ops.append_token_pool(self.k_buffer, self.v_buffer, k_rows, v_rows, loc,
                                 layer_tables=(self._k_ptrs, self._v_ptrs, self._geom))


class NativePagedAllocator:
    """Paged token-slot allocator with its free list on the device."""

    def __init__(self, *, size: int, page_size: int, dtype: torch.dtype, device: str | torch.device,
                 kvcache: NativeTokenToKVPool | None = None, need_sort: bool = False) -> None:
        if int(size) % int(page_size) != 0:
            raise ValueError("pool size must be a multiple of page_size")
        self.size = int(size)
        self.page_size = int(page_size)
        self.dtype = dtype
        self.device = torch.device(device)
        self.num_pages = self.size // self.page_size
        self._kvcache = kvcache
        self.need_sort = bool(need_sort)
        self._buf = torch.empty(self.num_pages, dtype=torch.int64, device=self.device)
        self._head = 0
        self._offsets = torch.arange(self.page_size, dtype=torch.int64, device=self.device)
        self.clear()

    # -- state ------------------------------------------------------------
    def clear(self) -> None:
        self._buf.copy_(torch.arange(1, self.num_pages + 1, dtype=torch.int64))
        self._head = 0

    @property
    def free_pages(self) -> torch.Tensor:
        return self._buf[self._head:]

    def available_size(self) -> int:
        return (self.num_pages - self._head) * self.page_size

    def get_kvcache(self) -> NativeTokenToKVPool | None:
        return self._kvcache

    # -- allocation -------------------------------------------------------
    def alloc(self, need_size: int) -> torch.Tensor | None:
        need_size = int(need_size)
        if need_size % self.page_size != 0:
            raise ValueError("paged allocation must be a multiple of page_size")
        n = need_size // self.page_size
        if n > self.num_pages - self._head:
            return None
        pages = self._buf[self._head : self._head + n]
        self._head += n
        return (pages[:, None] * self.page_size + self._offsets[None, :]).reshape(-1)

    def alloc_decode(self, seq_lens: torch.Tensor, seq_lens_cpu: torch.Tensor, last_loc: torch.Tensor):
        bs = int(seq_lens_cpu.numel())
        new_pages = int(((seq_lens_cpu.to(torch.int64) - 1) % self.page_size == 0).sum())
        if new_pages > self.num_pages - self._head:
            return None
        out = torch.empty(bs, dtype=torch.int64, device=self.device)
        sl = seq_lens.to(device=self.device, dtype=torch.int64).contiguous()
        ll = last_loc.to(device=self.device, dtype=torch.int64).contiguous()
        lib = _lib.load()
        rc = lib.atlas_alloc_decode_slots(_lib.ptr(sl), _lib.ptr(ll), int(self.free_pages.data_ptr()), self.page_size,
                                          bs, _lib.ptr(out), _lib.stream_of(self.device))
        _lib.check(rc, "atlas_alloc_decode_slots")
        self._head += new_pages
        return out

    def alloc_extend(self, prefix_lens: torch.Tensor, prefix_lens_cpu: torch.Tensor, seq_lens: torch.Tensor,
                     seq_lens_cpu: torch.Tensor, last_loc: torch.Tensor, extend_num_tokens: int):
        ps = self.page_size
        pre = prefix_lens_cpu.to(torch.int64)
        seq = seq_lens_cpu.to(torch.int64)
        new_pages = int(((seq + ps - 1) // ps - (pre + ps - 1) // ps).sum())
        if new_pages > self.num_pages - self._head:
            return None
        bs = int(pre.numel())
        out = torch.empty(int(extend_num_tokens), dtype=torch.int64, device=self.device)
        p_dev = prefix_lens.to(device=self.device, dtype=torch.int64).contiguous()
        s_dev = seq_lens.to(device=self.device, dtype=torch.int64).contiguous()
        ll = last_loc.to(device=self.device, dtype=torch.int64).contiguous()
        lib = _lib.load()
        rc = lib.atlas_alloc_extend_slots(_lib.ptr(p_dev), _lib.ptr(s_dev), _lib.ptr(ll),
                                          int(self.free_pages.data_ptr()), ps, bs, _lib.ptr(out),
                                          _lib.stream_of(self.device))
        _lib.check(rc, "atlas_alloc_extend_slots")
        self._head += new_pages
        return out

    def consume_pages(self, n: int) -> None:
        """Advance the free-list head past ``n`` pages that a kernel has
        taken from ``free_pages`` (in order)."""
        n = int(n)
        if n < 0 or n > self.num_pages - self._head:
            raise RuntimeError(f"cannot take {n} pages: {self.num_pages - self._head} are free")
        self._head += n

    def free(self, free_index: torch.Tensor) -> None:
        if int(free_index.numel()) == 0:
            return
        pages = torch.unique(free_index.to(device=self.device, dtype=torch.int64) // self.page_size)
        self.free_pages_prepend(pages)

    def free_pages_prepend(self, pages: torch.Tensor) -> None:
        """Put already sorted, unique page ids at the head of the free list."""
        k = int(pages.numel())
        if k == 0:
            return
        if k > self._head:
            raise RuntimeError("freeing more pages than are allocated")
        self._buf[self._head - k : self._head].copy_(pages)
        self._head -= k


class NativeReqToTokenPool:
    """Request rows of token-slot ids with an ascending free list of rows."""

    def __init__(self, *, size: int, max_context_len: int, device: str | torch.device) -> None:
        self.size = int(size)
        self.max_context_len = int(max_context_len)
        self.device = torch.device(device)
        self.req_to_token = torch.zeros((self.size, self.max_context_len), dtype=torch.int64, device=self.device)
        self._free_rows = list(range(self.size))

    def available_size(self) -> int:
        return len(self._free_rows)

    def alloc(self, reqs: Sequence[Any]) -> list[int] | None:
        n = len(reqs)
        if n > len(self._free_rows):
            return None
        rows, self._free_rows = self._free_rows[:n], self._free_rows[n:]
        for req, row in zip(reqs, rows):
            if hasattr(req, "req_pool_idx"):
                req.req_pool_idx = row
        return rows

    def free(self, req: Any) -> None:
        row = getattr(req, "req_pool_idx", req)
        if row is None:
            return
        row = int(row)
        if row not in self._free_rows:
            self._free_rows.append(row)
            self._free_rows.sort()
        if hasattr(req, "req_pool_idx"):
            req.req_pool_idx = None

    # the bridge may write all routes' row slices of a frontier in one
    # tensor-index write
    batched_row_writes = True

    def write(self, indices, values: torch.Tensor) -> None:
        self.req_to_token[indices] = values.to(device=self.device, dtype=torch.int64)

    def clear(self) -> None:
        self._free_rows = list(range(self.size))


def create_native_pools(*, num_pages: int, page_size: int, dtype: torch.dtype, head_num: int, head_dim: int,
                        layer_num: int, max_running_requests: int, max_context_len: int,
                        device: str | torch.device):
    """Allocator + KV pool + request rows sized like the reference's
    ``create_sglang_memory_pool_bundle`` (``sglang_runtime.py:1552-1609``)."""
    size = int(num_pages) * int(page_size)
    kv = NativeTokenToKVPool(size=size, page_size=page_size, dtype=dtype, head_num=head_num, head_dim=head_dim,
                             layer_num=layer_num, device=device)
    alloc = NativePagedAllocator(size=size, page_size=page_size, dtype=dtype, device=device, kvcache=kv)
    req = NativeReqToTokenPool(size=max_running_requests, max_context_len=max_context_len, device=device)
    return req, kv, alloc
