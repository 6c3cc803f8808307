"""Host pools for the route-pool bridge's CPU trace (test infrastructure).

* ``OracleAllocator`` -- the paged free-list policy of ``paged_kv.PagedAllocator``
  (SGLang's ``PagedTokenToKVPoolAllocator`` as the reference drives it,
  ``sglang_runtime.py:578-684``; the real allocator's order is parity
  unpinned) behind the allocator protocol the bridge calls: ``alloc(n)``,
  ``alloc_decode(seq_lens, seq_lens_cpu, last_loc)``,
  ``alloc_extend(prefix_lens, prefix_lens_cpu, seq_lens, seq_lens_cpu,
  last_loc, n)``, ``free(slots)``, ``clear()``, ``get_kvcache()``.
* ``OracleKV`` -- the KV content of every slot as the value id last written
  to it; ``move_kv_cache`` is ``values[dst] = values[src]``, the semantics the
  reference's tests pin for SGLang's ``move_kv_cache``
  (tests/test_tail_page_cow.py:14-16).
* ``OracleReqPool`` -- request rows with an ascending free list of rows.
"""

from __future__ import annotations

import numpy as np
import torch

from .paged_kv import PagedAllocator


class OracleKV:
    def __init__(self, num_slots: int) -> None:
        self.values = np.full(int(num_slots), -1, dtype=np.int64)
        self.moves: list[tuple[list[int], list[int]]] = []

    def _checked(self, slots) -> np.ndarray:
        s = np.asarray(slots, dtype=np.int64).reshape(-1)
        if s.size and (s.min() < 0 or s.max() >= self.values.size):
            raise ValueError(f"slot outside the pool: [{s.min()}, {s.max()}] vs {self.values.size}")
        return s

    def write(self, slots, value_ids) -> None:
        self.values[self._checked(slots)] = np.asarray(value_ids, dtype=np.int64).reshape(-1)

    def move_kv_cache(self, dst: torch.Tensor, src: torch.Tensor) -> None:
        d = self._checked(dst.cpu().numpy())
        s = self._checked(src.cpu().numpy())
        if d.size != s.size or np.intersect1d(d, s).size:
            raise ValueError("move_kv_cache needs equal-length, disjoint slot lists")
        self.values[d] = self.values[s]
        self.moves.append((d.tolist(), s.tolist()))


class OracleAllocator:
    def __init__(self, *, num_pages: int, page_size: int) -> None:
        self.policy = PagedAllocator(num_pages=int(num_pages), page_size=int(page_size))
        self.page_size = int(page_size)
        self.kv = OracleKV((int(num_pages) + 1) * int(page_size))

    @property
    def free_pages(self) -> list[int]:
        return list(self.policy.free_pages)

    def clear(self) -> None:
        self.policy.clear()

    def get_kvcache(self) -> OracleKV:
        return self.kv

    def alloc(self, need_size: int):
        out = self.policy.alloc(int(need_size))
        return None if out is None else torch.tensor(out, dtype=torch.long)

    def alloc_decode(self, seq_lens, seq_lens_cpu, last_loc):
        out = self.policy.alloc_decode([int(x) for x in seq_lens_cpu], [int(x) for x in last_loc.cpu()])
        return None if out is None else torch.tensor(out, dtype=torch.long)

    def alloc_extend(self, prefix_lens, prefix_lens_cpu, seq_lens, seq_lens_cpu, last_loc, extend_num_tokens):
        out = self.policy.alloc_extend([int(x) for x in prefix_lens_cpu], [int(x) for x in seq_lens_cpu],
                                       [int(x) for x in last_loc.cpu()])
        return None if out is None else torch.tensor(out, dtype=torch.long)

    def free(self, slots) -> None:
        self.policy.free([int(x) for x in torch.as_tensor(slots).cpu()])


class OracleReqPool:
    def __init__(self, *, size: int, max_context_len: int) -> None:
        self.req_to_token = torch.zeros((int(size), int(max_context_len)), dtype=torch.long)
        self.free_rows = list(range(int(size)))

    def alloc(self, reqs):
        if len(reqs) > len(self.free_rows):
            return None
        rows, self.free_rows = self.free_rows[: len(reqs)], self.free_rows[len(reqs):]
        for req, row in zip(reqs, rows):
            if hasattr(req, "req_pool_idx"):
                req.req_pool_idx = row
        return rows

    def free(self, req) -> None:
        row = getattr(req, "req_pool_idx", req)
        if row is None:
            return
        if int(row) not in self.free_rows:
            self.free_rows = sorted(self.free_rows + [int(row)])
        if hasattr(req, "req_pool_idx"):
            req.req_pool_idx = None

    def write(self, indices, values) -> None:
        self.req_to_token[indices] = values.cpu()

    def clear(self) -> None:
        self.free_rows = list(range(int(self.req_to_token.shape[0])))
