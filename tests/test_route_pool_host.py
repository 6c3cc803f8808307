"""Route-pool bridge host logic on CPU with test fakes: leases, tail-page
copy-on-write, request-row writes, promotion and prune.  Expected values are
the literals of the reference's own tests (tests/test_tail_page_cow.py and
tests/test_req_row_incremental.py, lines cited per test); the fake allocator
hands out monotone pages from 10 and the fake KV cache applies
``values[dst] = values[src]``, as the reference's fakes do."""

from types import SimpleNamespace

import pytest
import torch

from helpers import pkg


def _mods():
    sr = pkg("flashinfer_paged.sglang_runtime")
    ty = pkg("flashinfer_paged.types")
    return sr, ty


class MoveRecorder:
    def __init__(self):
        self.values = torch.arange(512, dtype=torch.float32)
        self.moves = []

    def move_kv_cache(self, dst, src):
        self.values[dst] = self.values[src]
        self.moves.append((dst.tolist(), src.tolist()))


class MonotoneAllocator:
    def __init__(self, page_size):
        self.page_size = page_size
        self.next_page = 10
        self.kv_cache = MoveRecorder()
        self.freed = []

    def alloc(self, count):
        assert count % self.page_size == 0
        n = count // self.page_size
        pages = torch.arange(self.next_page, self.next_page + n)
        self.next_page += n
        return (pages[:, None] * self.page_size + torch.arange(self.page_size)[None, :]).reshape(-1)

    def get_kvcache(self):
        return self.kv_cache

    def free(self, slots):
        self.freed.extend(slots.tolist())


class RowTable:
    def __init__(self, fill=0):
        self.req_to_token = torch.full((8, 128), fill, dtype=torch.long)
        self.write_log = []
        self.freed = []

    def write(self, indices, values):
        self.req_to_token[indices] = values
        row, pos = indices
        if isinstance(row, int) and isinstance(pos, slice):
            self.write_log.append((row, int(pos.start or 0), int(pos.stop or 0), values.tolist()))

    def free(self, handle):
        self.freed.append(handle)

    def clear(self):
        pass


class FailingRows(RowTable):
    def write(self, indices, values):
        raise RuntimeError("synthetic write failure")


class FailRowOneTwice(RowTable):
    """Rejects both the slice and the tensor-index form of one write to row 1."""

    def __init__(self):
        super().__init__(-1)
        self.left = 2

    def write(self, indices, values):
        row = indices[0]
        hit = int(row) == 1 if isinstance(row, int) else bool(torch.all(row == 1).item())
        if hit and self.left:
            self.left -= 1
            raise RuntimeError("synthetic one-shot row failure")
        super().write(indices, values)


class RecyclingRows(RowTable):
    def __init__(self):
        super().__init__(-1)
        self.available = list(range(8))

    def alloc(self, handles):
        if len(handles) > len(self.available):
            return None
        return torch.tensor([self.available.pop(0) for _ in handles], dtype=torch.long)

    def free(self, handle):
        super().free(handle)
        idx = getattr(handle, "req_pool_idx", None)
        if idx is not None and int(idx) not in self.available:
            self.available.append(int(idx))
            self.available.sort()


class NoSliceRows(RowTable):
    def write(self, indices, values):
        row, pos = indices
        if isinstance(row, int) and isinstance(pos, slice):
            raise TypeError("slice API unavailable")
        super().write(indices, values)


def bridge(page_size=4, rows=None, page_metadata=True):
    sr, _ = _mods()
    return sr.SGLangRoutePoolBridge(req_to_token_pool=rows or RowTable(), token_to_kv_pool_allocator=MonotoneAllocator(page_size),
                                    page_size=page_size, device="cpu", use_page_attention_metadata=page_metadata)


def route(route_id, committed, nodes=(), parent=None, pending=7):
    _, ty = _mods()
    return ty.RouteState(route_id=route_id, stage1_root_id=route_id, parent_route_id=parent,
                         materialized_leaf_node_id=nodes[-1] if nodes else None, pending_token_id=pending,
                         cumulative_logprob=0.0, stage1_depth=len(nodes), stage2_depth=0,
                         kv_view=ty.RouteKVView(prefix=ty.PrefixKVView(committed_length=committed), node_ids=tuple(nodes)))


def ids(*r):
    return [SimpleNamespace(route_id=x) for x in r]


L = lambda *x: torch.tensor(x, dtype=torch.long)  # noqa: E731


# ----------------------------------------------------------- copy-on-write
def test_shared_partial_tail_copies_one_writer():
    # test_tail_page_cow.py:61-79
    b = bridge()
    tail = L(0, 1, 2)
    out = b._copy_partial_tail_pages(ids(1, 2), [tail, tail])
    assert out[0] is tail and out[1].tolist() == [40, 41, 42]
    assert (b.cow_pages_copied, b.cow_tokens_copied) == (1, 3)
    c = b.hot_path_counters()
    assert c["hot_path_host_transfer_batches"] == 1 and c["hot_path_host_transfer_elements"] == 2
    assert b.token_to_kv_pool_allocator.kv_cache.moves == [([40, 41, 42], [0, 1, 2])]


def test_n_writers_copy_n_minus_one_pages_in_one_move():
    # test_tail_page_cow.py:82-96; the copies of one frontier go in one move call
    b = bridge()
    tail = L(0, 1)
    out = b._copy_partial_tail_pages(ids(1, 2, 3), [tail, tail, tail])
    assert out[0] is tail and out[1].tolist() == [40, 41] and out[2].tolist() == [44, 45]
    assert (b.cow_pages_copied, b.cow_tokens_copied) == (2, 4)
    assert b.token_to_kv_pool_allocator.kv_cache.moves == [([40, 41, 44, 45], [0, 1, 0, 1])]


def test_same_page_different_valid_lengths_copied():
    # test_tail_page_cow.py:99-113
    b = bridge()
    short, long = L(0, 1), L(0, 1, 2)
    out = b._copy_partial_tail_pages(ids(1, 2), [short, long])
    assert out[0] is short and out[1].tolist() == [40, 41, 42]
    assert (b.cow_pages_copied, b.cow_tokens_copied) == (1, 3)
    assert b.token_to_kv_pool_allocator.kv_cache.moves == [([40, 41, 42], [0, 1, 2])]


def test_prefix_slices_on_same_partial_page_share_lease():
    # test_tail_page_cow.py:116-157
    b = bridge()
    b.set_prefix_slots(L(0, 1, 2))
    rs = [route(1, 2, pending=7), route(2, 3, pending=8)]
    paths = [b._slot_path_for_route(r) for r in rs]
    assert b.route_tail_page_keys[1] == b.route_tail_page_keys[2]
    out = b._copy_partial_tail_pages(rs, paths)
    assert out[0].tolist() == [0, 1] and out[1].tolist() == [40, 41, 42]
    assert b.cow_pages_copied == 1
    assert b.hot_path_counters()["hot_path_host_transfer_batches"] == 0


def test_distinct_partial_pages_not_copied():
    # test_tail_page_cow.py:160-172
    b = bridge()
    a, c = L(0, 1, 2), L(4, 5, 6)
    out = b._copy_partial_tail_pages(ids(1, 2), [a, c])
    assert out[0] is a and out[1] is c
    assert (b.cow_pages_copied, b.cow_tokens_copied) == (0, 0)
    assert b.token_to_kv_pool_allocator.kv_cache.moves == []


def test_private_cow_tails_not_copied_again():
    # test_tail_page_cow.py:175-195
    b = bridge(page_size=8)
    tail = L(0, 1, 2)
    out = b._copy_partial_tail_pages(ids(1, 2), [tail, tail])
    assert b.cow_pages_copied == 1
    cont = [torch.cat((out[0], L(3))), torch.cat((out[1], L(83)))]
    again = b._copy_partial_tail_pages(ids(1, 2), cont)
    assert again[0] is cont[0] and again[1] is cont[1]
    assert (b.cow_pages_copied, b.cow_tokens_copied) == (1, 3)
    assert b.token_to_kv_pool_allocator.kv_cache.moves == [([80, 81, 82], [0, 1, 2])]


def test_cow_branches_write_without_contamination():
    # test_tail_page_cow.py:198-215
    b = bridge()
    tail = L(0, 1, 2)
    out = b._copy_partial_tail_pages(ids(1, 2), [tail, tail])
    kv = b.token_to_kv_pool_allocator.kv_cache
    s0, s1 = int(out[0][-1]) + 1, int(out[1][-1]) + 1
    kv.values[s0], kv.values[s1] = 111.0, 222.0
    assert out[0].tolist() == [0, 1, 2] and out[1].tolist() == [40, 41, 42]
    assert kv.values[out[0]].tolist() == [0.0, 1.0, 2.0] and kv.values[out[1]].tolist() == [0.0, 1.0, 2.0]
    assert float(kv.values[s0]) == 111.0 and float(kv.values[s1]) == 222.0


def test_full_tail_page_and_single_writer_need_no_cow():
    # test_tail_page_cow.py:218-238
    b = bridge()
    full = L(0, 1, 2, 3)
    out = b._copy_partial_tail_pages(ids(1, 2), [full, full])
    assert out[0] is full and out[1] is full
    part = L(0, 1, 2)
    assert b._copy_partial_tail_pages(ids(1), [part])[0] is part
    assert b.cow_pages_copied == 0


# ----------------------------------------------------------- promote / prune
def test_reference_counts_promotion_and_release():
    # test_tail_page_cow.py:241-277
    b = bridge()
    b.set_prefix_slots(L(0, 1))
    sel = route(1, 2, nodes=(1,))
    b.route_slot_paths = {1: L(0, 1, 40), 2: L(0, 1, 40, 41), 3: L(0, 1, 44)}
    b.owned_page_ids.update({10, 11})
    assert b.page_reference_counts() == {0: 4, 10: 2, 11: 1}
    b.commit_route_as_prefix(sel)
    b.retain_route_rows([2])
    assert b.page_reference_counts() == {0: 2, 10: 2}
    assert b.owned_page_ids == {0, 10, 11}
    assert b.release_unreferenced_node_slots([]) == 1
    assert b.page_reference_counts() == {0: 2, 10: 2}
    assert b.owned_page_ids == {0, 10}
    assert b.token_to_kv_pool_allocator.freed == [44]


def test_pending_owned_pages_materialised_once():
    # test_tail_page_cow.py:280-295
    b = bridge()
    b.set_prefix_slots(L(0, 1))
    b.route_slot_paths[1] = L(0, 1, 40)
    b._record_pending_owned_slots(L(40, 41, 44))
    assert b.release_unreferenced_node_slots([]) == 1
    assert b.pending_owned_slot_tensors == [] and b.owned_page_ids == {0, 10}
    assert b.token_to_kv_pool_allocator.freed == [44]
    assert b.release_unreferenced_node_slots([]) == 0
    assert b.token_to_kv_pool_allocator.freed == [44]


def test_tail_lease_through_reconcile_retain_commit_clear():
    # test_tail_page_cow.py:298-348
    b = bridge()
    b.set_prefix_slots(L(40, 41, 42))
    parent = route(1, 3)
    _, ty = _mods()
    kids = [ty.RouteState(route_id=r, stage1_root_id=r, parent_route_id=1, materialized_leaf_node_id=None,
                          pending_token_id=8, cumulative_logprob=0.0, stage1_depth=0, stage2_depth=0,
                          kv_view=parent.kv_view.fork()) for r in (2, 3)]
    b._slot_path_for_route(parent)
    b.reconcile_route_rows([parent], kids)
    key = b.route_tail_page_keys[1]
    assert b.route_tail_page_keys[2] == key and b.route_tail_page_keys[3] == key
    b.retain_route_rows([2])
    b.commit_route_as_prefix(kids[0])
    assert b.prefix_slot_count == 3 and b.prefix_page_ids == {10}
    assert b.prefix_tail_page_key == key and b.prefix_partial_tail_keys == {0: key}
    assert b.route_tail_page_keys == {2: key}
    b.clear_physical_state()
    assert (b.prefix_slot_count, b.prefix_page_ids, b.prefix_tail_page_key, b.prefix_partial_tail_keys,
            b.route_tail_page_keys) == (0, set(), None, {}, {})


def test_prefix_metadata_full_partial_empty():
    # test_tail_page_cow.py:351-371
    b = bridge()
    b.set_prefix_slots(torch.arange(40, 48))
    assert (b.prefix_slot_count, b.prefix_page_ids, b.prefix_tail_page_key, b.prefix_partial_tail_keys) == (
        8, {10, 11}, None, {})
    b.set_prefix_slots(torch.arange(40, 45))
    k = b.prefix_tail_page_key
    assert b.prefix_slot_count == 5 and b.prefix_page_ids == {10, 11} and k is not None
    assert b.prefix_partial_tail_keys == {1: k}
    b.set_prefix_slots(torch.empty(0, dtype=torch.long))
    assert (b.prefix_slot_count, b.prefix_page_ids, b.prefix_tail_page_key, b.prefix_partial_tail_keys) == (
        0, set(), None, {})


def test_full_rewrite_counters():
    # test_tail_page_cow.py:374-383
    b = bridge()
    b._write_req_token_row(3, L(4, 5, 6, 7))
    b._write_req_token_row(3, L(4, 5, 6, 7, 8))
    c = b.hot_path_counters()
    assert (c["req_row_write_calls"], c["req_row_elements_written"], c["req_row_full_rewrite_calls"],
            c["req_row_full_rewrite_elements"]) == (2, 9, 2, 9)


# ----------------------------------------------------------- request rows
def test_full_init_then_inherited_row_appends():
    # test_req_row_incremental.py:151-196
    b = bridge(rows=RowTable(-1), page_metadata=False)
    parent = route(1, 4)
    b.route_slot_paths[1] = L(0, 1, 2, 3)
    b.bind_existing_route_row(1, 0)
    _, md = b.prepare_frontier([parent], output_slot_ids=L(4))
    rt = b.req_to_token_pool
    assert rt.req_to_token[0, :5].tolist() == [0, 1, 2, 3, 4]
    assert md.seq_lens_sum == 5 and md.seq_lens_cpu.device.type == "cpu" and md.seq_lens_cpu.tolist() == [5]
    assert b.route_rows[1].written_length == 5 and rt.write_log == [(0, 0, 5, [0, 1, 2, 3, 4])]
    child = route(2, 4, nodes=(100,), parent=1)
    b.reconcile_route_rows([parent], [child])
    b.prepare_frontier([child], output_slot_ids=L(5))
    assert rt.req_to_token[0, :6].tolist() == [0, 1, 2, 3, 4, 5]
    assert b.route_rows[2].written_length == 6 and rt.write_log[-1] == (0, 5, 6, [5])
    c = b.hot_path_counters()
    assert (c["req_row_full_init_calls"], c["req_row_full_init_elements"], c["req_row_append_calls"],
            c["req_row_append_elements"], c["req_row_cow_patch_calls"], c["req_row_elements_written"]) == (
        1, 5, 1, 1, 0, 6)


def _two_writers(b, rows):
    rs = [route(1, 5), route(2, 5)]
    shared = L(0, 1, 2, 3, 4)
    for i, r in enumerate(rs):
        b.route_slot_paths[r.route_id] = shared
        b.bind_existing_route_row(r.route_id, i, written_length=5)
        rows.req_to_token[i, :5] = shared
    return rs


def test_cow_row_patches_only_dirty_tail():
    # test_req_row_incremental.py:199-233
    rows = RowTable(-1)
    b = bridge(rows=rows, page_metadata=False)
    rs = _two_writers(b, rows)
    b.prepare_frontier(rs, output_slot_ids=L(5, 41))
    assert rows.req_to_token[0, :6].tolist() == [0, 1, 2, 3, 4, 5]
    assert rows.req_to_token[1, :6].tolist() == [0, 1, 2, 3, 40, 41]
    assert b.route_slot_paths[2].tolist() == [0, 1, 2, 3, 40, 41]
    assert rows.write_log == [(0, 5, 6, [5]), (1, 4, 6, [40, 41])]
    c = b.hot_path_counters()
    assert (c["cow_pages_copied"], c["cow_tokens_copied"], c["req_row_full_init_calls"], c["req_row_append_calls"],
            c["req_row_append_elements"], c["req_row_cow_patch_calls"], c["req_row_cow_patch_elements"],
            c["req_row_elements_written"]) == (1, 1, 0, 1, 1, 1, 2, 3)


def test_fork_reuses_first_child_row_and_inits_sibling():
    # test_req_row_incremental.py:236-266
    rows = RecyclingRows()
    b = bridge(rows=rows, page_metadata=False)
    parent = route(1, 5)
    shared = L(0, 1, 2, 3, 4)
    b.route_slot_paths[1] = shared
    b.bind_existing_route_row(1, 0, written_length=5)
    rows.available.remove(0)
    rows.req_to_token[0, :5] = shared
    kids = [route(2, 5, parent=1), route(3, 5, parent=1)]
    b.reconcile_route_rows([parent], kids)
    b.prepare_frontier(kids, output_slot_ids=L(5, 41))
    assert b.route_rows[2].req_pool_index == 0 and b.route_rows[3].req_pool_index == 1
    assert rows.req_to_token[0, :6].tolist() == [0, 1, 2, 3, 4, 5]
    assert rows.req_to_token[1, :6].tolist() == [0, 1, 2, 3, 40, 41]
    c = b.hot_path_counters()
    assert (c["req_row_append_calls"], c["req_row_append_elements"], c["req_row_full_init_calls"],
            c["req_row_full_init_elements"], c["req_row_cow_patch_calls"]) == (1, 1, 1, 6, 0)


def test_released_then_reused_row_full_init():
    # test_req_row_incremental.py:269-294
    rows = RowTable(-1)
    b = bridge(rows=rows, page_metadata=False)
    old = SimpleNamespace(req_pool_idx=0)
    b.bind_existing_route_row(1, 0, handle=old, written_length=5)
    rows.req_to_token[0, :5] = L(0, 1, 2, 3, 4)
    b.release_route_rows([1])
    b.route_slot_paths[2] = L(8, 9, 10)
    b.bind_existing_route_row(2, 0)
    b.prepare_frontier([route(2, 3)], output_slot_ids=L(11))
    assert rows.freed == [old] and rows.req_to_token[0, :4].tolist() == [8, 9, 10, 11]
    assert rows.write_log == [(0, 0, 4, [8, 9, 10, 11])] and b.route_rows[2].written_length == 4
    c = b.hot_path_counters()
    assert (c["req_row_full_init_calls"], c["req_row_full_init_elements"], c["req_row_append_calls"]) == (1, 4, 0)


def test_recycled_row_full_inits():
    # test_req_row_incremental.py:297-323
    rows = RecyclingRows()
    b = bridge(rows=rows, page_metadata=False)
    old = route(1, 3)
    b.route_slot_paths[1] = L(8, 9, 10)
    first = int(b.ensure_route_rows([old])[0])
    b.prepare_frontier([old], output_slot_ids=L(11))
    b.release_route_rows([1])
    new = route(2, 2)
    b.route_slot_paths[2] = L(20, 21)
    again = int(b.ensure_route_rows([new])[0])
    b.prepare_frontier([new], output_slot_ids=L(22))
    assert first == again == 0 and b.route_rows[2].written_length == 3
    assert rows.req_to_token[0, :3].tolist() == [20, 21, 22]
    c = b.hot_path_counters()
    assert (c["req_row_full_init_calls"], c["req_row_full_init_elements"], c["req_row_append_calls"]) == (2, 7, 0)


def test_promotion_does_not_rewrite_row():
    # test_req_row_incremental.py:326-355
    rows = RowTable(-1)
    b = bridge(rows=rows, page_metadata=False)
    b.set_prefix_slots(L(0, 1, 2, 3))
    sel = route(1, 4, nodes=(100,))
    b.route_slot_paths[1] = L(0, 1, 2, 3, 4)
    b.bind_existing_route_row(1, 0, written_length=5)
    rows.req_to_token[0, :5] = b.route_slot_paths[1]
    before = b.hot_path_counters()
    b.commit_route_as_prefix(sel)
    b.retain_route_rows([1])
    assert b.hot_path_counters() == before and rows.write_log == []
    assert b.route_rows[1].written_length == 5 and b.prefix_slot_ids.tolist() == [0, 1, 2, 3, 4]
    b.prepare_frontier([route(1, 5)], output_slot_ids=L(5))
    assert rows.write_log == [(0, 5, 6, [5])]
    c = b.hot_path_counters()
    assert (c["req_row_append_calls"], c["req_row_append_elements"], c["req_row_full_init_calls"]) == (1, 1, 0)


def test_validation_accepts_cow_alias_rejects_unowned():
    # test_req_row_incremental.py:358-384
    rows = RowTable(-1)
    b = bridge(rows=rows, page_metadata=False)
    b.set_prefix_slots(L(0, 1, 2, 3))
    r = route(45, 4, nodes=(100, 101))
    b.node_slot_ids = {100: 4, 101: 5}
    b.route_slot_paths[45] = L(0, 1, 2, 3, 40, 41)
    b.owned_page_ids.add(10)
    b.bind_existing_route_row(45, 0, written_length=6)
    rows.req_to_token[0, :6] = b.route_slot_paths[45]
    b.validate_route_physical_state(r)
    b.owned_page_ids.remove(10)
    with pytest.raises(RuntimeError, match="unowned KV pages"):
        b.validate_route_physical_state(r)


def test_failed_write_leaves_counters():
    # test_req_row_incremental.py:387-405
    b = bridge(rows=FailingRows(), page_metadata=False)
    with pytest.raises(RuntimeError, match="failed to write"):
        b._write_req_token_slice(0, 0, L(1, 2), write_kind="full_init")
    c = b.hot_path_counters()
    assert (c["req_row_write_calls"], c["req_row_elements_written"], c["req_row_full_init_calls"]) == (0, 0, 0)


def test_tensor_index_fallback_counts_once():
    # test_req_row_incremental.py:408-425
    rows = NoSliceRows(-1)
    b = bridge(rows=rows, page_metadata=False)
    b._write_req_token_slice(2, 3, L(17, 18), write_kind="cow_patch")
    assert rows.req_to_token[2, 3:5].tolist() == [17, 18]
    c = b.hot_path_counters()
    assert (c["req_row_write_calls"], c["req_row_elements_written"], c["req_row_cow_patch_calls"],
            c["req_row_cow_patch_elements"]) == (1, 2, 1, 2)


def test_failed_cow_patch_keeps_dirty_range_for_retry():
    # test_req_row_incremental.py:428-473
    rows = FailRowOneTwice()
    b = bridge(rows=rows, page_metadata=False)
    rs = _two_writers(b, rows)
    with pytest.raises(RuntimeError, match="failed to write"):
        b.prepare_frontier(rs, output_slot_ids=L(5, 41))
    assert b.route_slot_paths[2].tolist() == [0, 1, 2, 3, 40]
    assert b.route_rows[2].written_length == 5 and b.route_rows[2].pending_dirty_start == 4
    assert rows.req_to_token[1, :5].tolist() == [0, 1, 2, 3, 4]
    b.prepare_frontier([rs[1]], output_slot_ids=L(41))
    assert rows.req_to_token[1, :6].tolist() == [0, 1, 2, 3, 40, 41]
    assert b.route_rows[2].written_length == 6 and b.route_rows[2].pending_dirty_start is None
    assert rows.write_log[-1] == (1, 4, 6, [40, 41])
    c = b.hot_path_counters()
    assert (c["req_row_write_calls"], c["req_row_append_calls"], c["req_row_cow_patch_calls"]) == (2, 1, 1)


# ----------------------------------------------------------- errors and metadata
def test_prepare_frontier_errors():
    b = bridge(page_metadata=False)
    with pytest.raises(ValueError, match="cannot be empty"):
        b.prepare_frontier([])
    b.route_slot_paths[1] = L(0, 1)
    b.bind_existing_route_row(1, 0)
    with pytest.raises(ValueError, match="one slot per active route"):
        b.prepare_frontier([route(1, 2)], output_slot_ids=L(2, 3))
    with pytest.raises(RuntimeError, match="does not match logical KV"):
        b._slot_path_for_route(route(1, 5))
    with pytest.raises(RuntimeError, match="duplicate output KV slots"):
        b.route_slot_paths[2] = L(4, 5)
        b.bind_existing_route_row(2, 1)
        b.prepare_frontier([route(1, 2), route(2, 2)], output_slot_ids=L(9, 9))


def test_page_metadata_refuses_host_tensors():
    # The page-metadata builder is a HIP kernel: host slot paths fail loudly.
    b = bridge(page_size=4, rows=RowTable(-1))
    b.route_slot_paths[1] = L(0, 1, 2, 3, 40)
    b.bind_existing_route_row(1, 0)
    with pytest.raises(RuntimeError, match="HIP device tensors"):
        b.prepare_frontier([route(1, 5)], output_slot_ids=L(41))


def test_allocation_errors_name_the_allocator_calls():
    sr, _ = _mods()

    class Broken:
        def alloc(self, n):
            return None

    b = sr.SGLangRoutePoolBridge(req_to_token_pool=RowTable(), token_to_kv_pool_allocator=Broken(), page_size=4,
                                 device="cpu")
    with pytest.raises(RuntimeError, match=r"alloc\(3,\): returned None"):
        b.allocate_token_slots(3)
    with pytest.raises(RuntimeError, match="cannot allocate 2 COW pages"):
        b._allocate_full_pages(2)
    with pytest.raises(ValueError):
        b.allocate_token_slots(0)


class OverlappingAllocator(MonotoneAllocator):
    """Hands out page 0 again: a destination that is also a source page."""

    def alloc(self, count):
        n = count // self.page_size
        pages = torch.zeros(n, dtype=torch.long)
        return (pages[:, None] * self.page_size + torch.arange(self.page_size)[None, :]).reshape(-1)


def test_cow_rejects_destination_pages_that_overlap_sources():
    sr, _ = _mods()
    b = sr.SGLangRoutePoolBridge(req_to_token_pool=RowTable(), token_to_kv_pool_allocator=OverlappingAllocator(4),
                                 page_size=4, device="cpu", use_page_attention_metadata=True)
    tail = L(0, 1, 2)
    with pytest.raises(RuntimeError, match="overlap"):
        b._copy_partial_tail_pages(ids(1, 2), [tail, tail])
    assert b.token_to_kv_pool_allocator.kv_cache.moves == []


def test_fused_frontier_step_needs_native_pools():
    """The one-launch frontier step of many requests applies only to
    distinct bridges over one set of native pools; host pools (and a bridge
    given twice) keep the per-request calls."""
    sr, _ = _mods()
    b = sr.SGLangRoutePoolBridge(req_to_token_pool=RowTable(), token_to_kv_pool_allocator=MonotoneAllocator(4),
                                 page_size=4, device="cpu")
    assert not sr.fused_frontier_supported([b])
    assert not sr.fused_frontier_supported([])
    with pytest.raises(ValueError, match="native pools"):
        sr.prepare_frontiers([b], [ids(1)])


def test_fused_step_flags_raise_in_prepare_frontier_order():
    """Check words of a fused step (one per route): a skipped descriptor of
    any route first, then per request the copy-on-write overlap, duplicate
    decode slots and page layout checks, in the order prepare_frontier
    records them; a request's checks read only its own routes' words."""
    sr, _ = _mods()
    pm = pkg("flashinfer_paged.paged_metadata")
    lib = pkg("_lib")
    bad_desc, layout, dup, cow = (lib.FRONTIER_BAD_DESCRIPTOR, lib.FRONTIER_BAD_LAYOUT, lib.FRONTIER_DUPLICATE_SLOT,
                                  lib.FRONTIER_COW_OVERLAP)
    spans = [(0, 2), (2, 3)]
    cases = [
        ([0, 0, bad_desc], "out of range", True),
        ([layout, cow | dup], "overlap", False),
        ([dup, layout], "duplicate output KV slots", False),
        ([0, layout], pm.LAYOUT_MESSAGE[:40], False),
    ]
    for words, message, everywhere in cases:
        flags = sr._StepFlags(torch.tensor(words + [0], dtype=torch.int64), spans)
        with pytest.raises(RuntimeError, match=message):
            flags.check(0, True)
        if everywhere:
            with pytest.raises(RuntimeError, match=message):
                flags.check(1, True)
        else:
            flags.check(1, True)  # the other request's words are clear
    sr._StepFlags(torch.tensor([0, layout, 0], dtype=torch.int64), spans).check(0, False)  # layout not validated


def test_pending_step_checks_read_once_and_raise_in_order():
    """The words of every fused step with a check pending on a set of
    bridges are brought to the host once; the checks then raise in the order
    recorded, and a bridge's pending list is empty after its checks ran."""
    sr, _ = _mods()
    lib = pkg("_lib")

    class Bridge:
        check_pending_device_checks = sr.SGLangRoutePoolBridge.check_pending_device_checks

        def __init__(self, checks):
            self.pending_device_checks = checks

    spans = [(0, 2), (2, 4)]
    good = sr._StepFlags(torch.zeros(4, dtype=torch.int64), spans)
    bad = sr._StepFlags(torch.tensor([0, 0, 0, lib.FRONTIER_DUPLICATE_SLOT], dtype=torch.int64), spans)
    a = Bridge([sr._StepCheck(good, 0, True), sr._StepCheck(bad, 0, True)])
    b = Bridge([sr._StepCheck(good, 1, True), sr._StepCheck(bad, 1, True)])
    sr._prefetch_step_flags([a, b])
    assert good._host == [0] * 4 and bad._host == [0, 0, 0, lib.FRONTIER_DUPLICATE_SLOT]
    a.check_pending_device_checks()
    assert a.pending_device_checks == []
    with pytest.raises(RuntimeError, match="duplicate output KV slots"):
        b.check_pending_device_checks()
    assert b.pending_device_checks == []


def test_batched_workload_on_host_pools_equals_per_request_calls():
    """On host pools the batched drafter workload falls back to one bridge
    call per request and leaves the same state."""
    dw = pkg("drafter_workload")
    from oracle.route_pool import OracleAllocator, OracleReqPool

    def run(batched):
        alloc = OracleAllocator(num_pages=640, page_size=64)
        rows = OracleReqPool(size=128, max_context_len=4096)
        wl = dw.DrafterForkWorkload(plans=dw.config5_plans(3, 64, 4), req_pool=rows, allocator=alloc, page_size=64,
                                    device="cpu", writer=lambda s, v: alloc.kv.write(s.numpy(), v.numpy()),
                                    use_page_attention_metadata=False, batched=batched)
        wl.run()
        return (list(alloc.free_pages), alloc.kv.values.tolist(),
                [{r: p.tolist() for r, p in q.bridge.route_slot_paths.items()} for q in wl.requests],
                [q.bridge.hot_path_counters() for q in wl.requests])

    assert run(True) == run(False)


def test_multi_request_commit_and_prune_refusals_on_host_pools():
    """The multi-request commit and prune refuse mismatched list lengths
    before any state changes; on host pools they make one call per request,
    so the stats equal the per-request calls'."""
    dw = pkg("drafter_workload")
    sr, _ = _mods()
    from oracle.route_pool import OracleAllocator, OracleReqPool

    def setup():
        alloc = OracleAllocator(num_pages=640, page_size=64)
        rows = OracleReqPool(size=128, max_context_len=4096)
        wl = dw.DrafterForkWorkload(plans=dw.config5_plans(3, 64, 9), req_pool=rows, allocator=alloc, page_size=64,
                                    device="cpu", writer=lambda s, v: alloc.kv.write(s.numpy(), v.numpy()),
                                    use_page_attention_metadata=False, batched=True)
        wl.prefill()
        wl.stage1()
        return wl, alloc

    wl, alloc = setup()
    backends = [r.backend for r in wl.requests]
    picks = wl.select_commits()
    free_before = list(alloc.free_pages)
    with pytest.raises(ValueError):
        sr.SGLangFlashInferFrontierModelBackend.commit_stage1_and_promote_many(
            backends, [c for c, _ in picks][:2], [k for _, k in picks])
    with pytest.raises(ValueError):
        sr.release_unreferenced_node_slots_many([r.bridge for r in wl.requests], [[]])
    assert list(alloc.free_pages) == free_before
    got = sr.SGLangFlashInferFrontierModelBackend.commit_stage1_and_promote_many(
        backends, [c for c, _ in picks], [k for _, k in picks])
    wl2, alloc2 = setup()
    ref = [r.backend.commit_stage1_and_promote(committed_route=c, retained_routes=k)
           for r, (c, k) in zip(wl2.requests, wl2.select_commits())]
    assert [s for _, s in got] == [s for _, s in ref]
    assert list(alloc.free_pages) == list(alloc2.free_pages)
    bridges = [r.bridge for r in wl.requests]
    for b in bridges:
        b.retain_route_rows([])
    counts = sr.release_unreferenced_node_slots_many(bridges, [[] for _ in bridges])
    for b in [r.bridge for r in wl2.requests]:
        b.retain_route_rows([])
    assert counts == [b.release_unreferenced_node_slots([]) for b in [r.bridge for r in wl2.requests]]
    assert list(alloc.free_pages) == list(alloc2.free_pages)
