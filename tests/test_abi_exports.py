"""The C-ABI library loads and exports every entry point include/*.h declares
(no compute calls: runs without a GPU)."""

import ctypes
import re
from pathlib import Path

from helpers import ROOT, pkg


def _declared_symbols() -> set[str]:
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = header.read_text()
        names.update(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(atlas_\w+)\s*\(", text, flags=re.M))
    return names


def test_header_declares_entry_points():
    names = _declared_symbols()
    assert {"atlas_tree_verify_attn", "atlas_kv_move_slots", "atlas_kv_commit_paged", "atlas_prune_pages"} <= names


def test_library_exports_every_declared_symbol():
    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    for name in sorted(_declared_symbols()):
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
    # The ctypes signature table covers the same set.
    assert set(lib_mod.exported_symbols()) == _declared_symbols()


def test_abi_version_and_error_string():
    lib = pkg("_lib").load()
    assert lib.atlas_abi_version() == 18
    assert isinstance(lib.atlas_last_error(), bytes)


def test_argument_errors_are_reported_without_device_work():
    """Invalid arguments are rejected before any launch (no GPU needed)."""
    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    rc = lib.atlas_kv_move_slots(None, None, 0, 1, 16, 16, 16, None, None, 4, None)
    assert rc == lib_mod.ATLAS_EINVAL
    assert b"" != lib.atlas_last_error()
    rc = lib.atlas_tree_verify_attn(
        None, 0, 0,            # q, strides
        None, 0, 0, 0, 0,      # kv cache, page stride, V offset, token stride, head stride
        None, None, None, None,  # qo_indptr, kv_indptr, kv_indices, kv_len
        0, None, None, 1,      # mask mode, tree mask, mask column start, mask words
        None, 0, None,         # work list, page windows
        None, 0, 0,            # merge list, its partial rows
        1, 32, 8, 96, 16,      # rows per item, Hq, Hkv, head_dim (unsupported), page size
        ctypes.c_float(0.1), 0,
        None, 0, 0, None,      # out, out strides, lse
        None, 0, None,         # workspace, bytes, stream
    )
    assert rc == lib_mod.ATLAS_EINVAL
    try:
        lib_mod.check(rc, "probe")
    except ValueError as exc:
        assert "probe" in str(exc)
    else:
        raise AssertionError("check() did not raise")


def test_gather_logprobs_workspace_contract_without_device_work():
    """The scoring call sizes its workspace from (rows, vocab) and refuses a
    smaller one before any launch."""
    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    need = lib.atlas_gather_logprobs_workspace_bytes(34, 128256)
    assert need > 34 * 8 and lib.atlas_gather_logprobs_workspace_bytes(0, 10) < 0
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: the call refuses first
    rc = lib.atlas_gather_logprobs(fake, 128256, 34, None, 0, 0, 128256, lib_mod.DTYPE_F16, fake, fake, 4, None,
                                   fake, fake, need - 1, None)
    assert rc == lib_mod.ATLAS_EINVAL and b"workspace" in lib.atlas_last_error()


def test_every_entry_point_refuses_null_buffers_before_device_work():
    """Every compute entry point, called with NULL for every pointer and 1
    for every count (``float`` arguments 1.0), returns ATLAS_EINVAL with a
    message, without touching a device (this runs without a GPU)."""
    import ctypes

    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    queries = {"atlas_last_error", "atlas_abi_version", "atlas_gather_logprobs_workspace_bytes",
               "atlas_frontier_workspace_bytes", "atlas_tree_spec_bytes"}
    ints = (ctypes.c_int, ctypes.c_int64, ctypes.c_int32, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_uint64)
    checked = []
    for name, argtypes in lib_mod._SIGNATURES.items():
        if name in queries:
            continue
        args = [1 if t in ints else 1.0 if t in (ctypes.c_float, ctypes.c_double) else None for t in argtypes]
        rc = getattr(lib, name)(*args)
        assert rc == lib_mod.ATLAS_EINVAL, f"{name} returned {rc}"
        assert lib.atlas_last_error(), f"{name} left no error message"
        checked.append(name)
    assert len(checked) == len(_declared_symbols()) - len(queries)


def _verify_args(name, **over):
    """Arguments of a verify entry point with valid shapes (Llama-3.1-8B:
    Hq 32, Hkv 8, head_dim 128, page 16, fp16, one work item and one merge
    item) and never-dereferenced stand-in device pointers; ``over`` replaces
    named ones."""
    import ctypes

    fake = ctypes.c_void_p(1 << 20)
    row = 2 * 128 + 4
    a = dict(q=fake, q_st=32 * 128, q_sh=128, kv=fake, page_stride=2 * 16 * 8 * 256, v_off=16 * 8 * 256,
             token_stride=8 * 256, head_stride=256, qo=fake, kvp=fake, kvi=fake, kvl=fake, mask_mode=1, tree=fake, col=fake, words=1,
             work=fake, nwork=1, win=None, merge=fake, nmerge=1, merge_rows=64, rows=64, hq=32, hkv=8, d=128,
             ps=16, scale=ctypes.c_float(0.088), dtype=0, out=fake, o_st=32 * 128, o_sh=128, lse=None)
    a.update(over)
    head = [a[k] for k in ("q", "q_st", "q_sh", "kv", "page_stride", "v_off", "token_stride", "head_stride", "qo",
                           "kvp", "kvi",
                           "kvl", "mask_mode", "tree", "col", "words", "work", "nwork", "win", "merge", "nmerge",
                           "merge_rows", "rows", "hq", "hkv", "d", "ps", "scale", "dtype", "out", "o_st", "o_sh",
                           "lse")]
    if name == "atlas_tree_verify_attn_noalloc":
        return head + [a.get("partial_rows", 64), None]
    ws = [a.get("ws", fake), a.get("ws_bytes", 64 * row)]
    if name == "atlas_tree_verify_attn_append":
        return head + ws + [fake, fake, 8 * 128, 128, None, None, 0, None]
    return head + ws + [None]


VERIFY_ENTRIES = ("atlas_tree_verify_attn", "atlas_tree_verify_attn_append", "atlas_tree_verify_attn_noalloc")


def test_verify_entry_points_name_the_null_buffer():
    """With valid shapes, a NULL buffer is what the refusal names, before the
    device (or the allocation-free entry point's device scratch) is touched."""
    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    for name in VERIFY_ENTRIES:
        for key, what in (("q", b"q, kv_cache and out"), ("kv", b"q, kv_cache and out"),
                          ("out", b"q, kv_cache and out"), ("kvi", b"indptr / indices"),
                          ("work", b"work list"), ("merge", b"merge list")):
            rc = getattr(lib, name)(*_verify_args(name, **{key: None}))
            assert rc == lib_mod.ATLAS_EINVAL, (name, key, rc)
            msg = lib.atlas_last_error()
            assert what in msg and b"NULL" in msg, (name, key, msg)
        if name != "atlas_tree_verify_attn_noalloc":
            rc = getattr(lib, name)(*_verify_args(name, ws=None))
            assert rc == lib_mod.ATLAS_EINVAL and b"workspace must not be NULL" in lib.atlas_last_error()


def test_verify_entry_points_refuse_too_few_partial_rows():
    """The merge items' partial-row count travels with the merge list; a
    workspace or a partial_rows below it is refused before any device work."""
    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    row = 2 * 128 + 4
    for name in VERIFY_ENTRIES:
        if name == "atlas_tree_verify_attn_noalloc":
            bad = _verify_args(name, merge_rows=65, partial_rows=64)
        else:
            bad = _verify_args(name, merge_rows=65, ws_bytes=64 * row)
        rc = getattr(lib, name)(*bad)
        assert rc == lib_mod.ATLAS_EINVAL, (name, rc)
        assert b"merge items reference 65 partial rows" in lib.atlas_last_error(), name
        rc = getattr(lib, name)(*_verify_args(name, merge_rows=0))
        assert rc == lib_mod.ATLAS_EINVAL and b"merge items reference 0" in lib.atlas_last_error(), name


def test_prune_by_paths_limits_without_device_work():
    """atlas_prune_pages_paths refuses more than ATLAS_PRUNE_MAX_PATHS paths
    or pools beyond one workgroup's bitmap (ATLAS_EUNSUPPORTED: the caller
    prunes through atlas_prune_pages) and a path with NULL slots or a negative
    length (ATLAS_EINVAL), before any launch."""
    import ctypes

    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    fake = ctypes.c_void_p(1 << 20)
    paths = (lib_mod.SlotPath * 65)()
    for p in paths:
        p.slots, p.len = 1 << 20, 4

    def call(n, num_pages=4096, arr=paths):
        return lib.atlas_prune_pages_paths(fake, fake, num_pages, arr, n, 0, 16, fake, fake, None)

    assert call(65) == lib_mod.ATLAS_EUNSUPPORTED and b"64 paths" in lib.atlas_last_error()
    assert call(1, num_pages=lib_mod.PRUNE_PATHS_MAX_PAGES + 1) == lib_mod.ATLAS_EUNSUPPORTED
    bad = (lib_mod.SlotPath * 2)()
    bad[0].slots, bad[0].len = 1 << 20, 3
    bad[1].slots, bad[1].len = None, 2
    assert call(2, arr=bad) == lib_mod.ATLAS_EINVAL and b"path 1" in lib.atlas_last_error()
    bad[1].slots, bad[1].len = 1 << 20, -1
    assert call(2, arr=bad) == lib_mod.ATLAS_EINVAL


def test_frontier_host_descriptors_limit_without_device_work():
    """A frontier step whose descriptors travel in the launch's arguments
    takes at most FRONTIER_MAX_HOST_ROUTES routes; more are refused as
    unsupported before any buffer is read or any launch."""
    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: the call refuses first
    n = lib_mod.FRONTIER_MAX_HOST_ROUTES + 1
    rc = lib.atlas_pool_prepare_frontier_host(fake, fake, fake, n, fake, 4, 16, 64, fake, 4, 64, fake, 64, fake,
                                              None, None, 0, fake, fake, fake, fake, 64, fake, fake, None)
    assert rc == lib_mod.ATLAS_EUNSUPPORTED
    assert b"at most" in lib.atlas_last_error()


def test_tree_spec_upload_refusals_without_device_work():
    """The one-launch spec upload refuses a spec shorter than its tree block
    and unaligned spec buffers before any launch."""
    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    a, b = ctypes.c_void_p(1 << 20), ctypes.c_void_p(2 << 20)  # never dereferenced: the calls refuse first
    assert lib.atlas_tree_spec_upload(a, 15, 4, 8, b, b, None) == lib_mod.ATLAS_EINVAL  # 15 < 4 * 4
    assert b"tree block" in lib.atlas_last_error()
    assert lib.atlas_tree_spec_upload(ctypes.c_void_p((1 << 20) + 8), 64, 4, 8, b, b, None) == lib_mod.ATLAS_EINVAL
    assert b"aligned" in lib.atlas_last_error()


def test_header_constants_match_the_binding():
    """Every ``#define ATLAS_X value`` of include/ that the Python binding
    mirrors (as ``ATLAS_X`` or ``X``) has the same value there, and the
    limits and codes the runtime passes to the library are among them."""
    lib_mod = pkg("_lib")
    defines = {}
    for header in (ROOT / "include").glob("*.h"):
        for name, value in re.findall(r"^#define (ATLAS_\w+) \(?(-?\d+)\)?", header.read_text(), flags=re.M):
            defines[name] = int(value)
    checked = set()
    for name, value in defines.items():
        for py in (name, name[len("ATLAS_"):]):
            if hasattr(lib_mod, py):
                assert getattr(lib_mod, py) == value, f"{py} = {getattr(lib_mod, py)} but the header says {value}"
                checked.add(name)
    assert {"ATLAS_FRONTIER_MAX_HOST_ROUTES", "ATLAS_FRONTIER_BAD_DESCRIPTOR", "ATLAS_FRONTIER_COW_OVERLAP",
            "ATLAS_SELECT_MAX_ENTRIES", "ATLAS_ROUND_BF16", "ATLAS_PRUNE_MAX_PATHS", "ATLAS_ATTN_SCRATCH_BYTES",
            "ATLAS_MAX_LAYERS_PER_LAUNCH", "ATLAS_EUNSUPPORTED", "ATLAS_MASK_TREE"} <= checked


def test_gather_limits_without_device_work():
    """The read-back gather refuses more than GATHER_MAX_SEGMENTS segments
    and a segment with values but no source, before any launch; nothing to
    gather is no launch at all."""
    lib_mod = pkg("_lib")
    lib = lib_mod.load()
    segs = (lib_mod.I64Segment * (lib_mod.GATHER_MAX_SEGMENTS + 1))()
    assert lib.atlas_gather_i64(segs, lib_mod.GATHER_MAX_SEGMENTS + 1, None, None) == lib_mod.ATLAS_EINVAL
    segs[0].count = 3  # NULL source
    assert lib.atlas_gather_i64(segs, 1, None, None) == lib_mod.ATLAS_EINVAL
    assert b"segment 0" in lib.atlas_last_error()
    segs[0].count = 0
    assert lib.atlas_gather_i64(segs, 2, None, None) == lib_mod.ATLAS_OK
