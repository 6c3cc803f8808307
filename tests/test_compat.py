"""The package installs under the reference's import names: hot-path names are
patched into already-loaded reference modules, or this package's modules are
registered when the reference is absent."""

import importlib.util
import sys
import types

import pytest

from helpers import pkg


@pytest.fixture
def clean_modules():
    saved = {k: v for k, v in sys.modules.items() if k == "flashinfer" or k.startswith("atlas_0709")}
    for k in saved:
        del sys.modules[k]
    yield
    for k in [k for k in sys.modules if k == "flashinfer" or k.startswith("atlas_0709")]:
        del sys.modules[k]
    sys.modules.update(saved)


def test_registers_modules_when_reference_absent(clean_modules):
    if importlib.util.find_spec("atlas_0709") is not None or importlib.util.find_spec("flashinfer") is not None:
        pytest.skip("a real atlas_0709 / flashinfer is importable here")
    compat = pkg("compat")
    done = compat.install_atlas_0709_alias(flashinfer=True)
    assert set(done.values()) == {"registered"} and "flashinfer" in done
    from atlas_0709.flashinfer_paged.sglang_runtime import SGLangRoutePoolBridge
    from atlas_0709.flashinfer_full_verify import build_deduplicated_tree_spec_from_paths
    import flashinfer

    assert SGLangRoutePoolBridge is pkg("flashinfer_paged.sglang_runtime").SGLangRoutePoolBridge
    assert build_deduplicated_tree_spec_from_paths is pkg("flashinfer_full_verify").build_deduplicated_tree_spec_from_paths
    assert flashinfer.BatchPrefillWithPagedKVCacheWrapper is pkg("tree_attention").BatchPrefillWithPagedKVCacheWrapper
    assert flashinfer.BatchDecodeWithPagedKVCacheWrapper is pkg("decode_attention").BatchDecodeWithPagedKVCacheWrapper
    from atlas_0709.flashinfer_full_verify import make_decode_wrapper, plan_decode_wrapper
    assert make_decode_wrapper is pkg("decode_attention").make_decode_wrapper
    assert plan_decode_wrapper is pkg("decode_attention").plan_decode_wrapper


def test_patches_only_hot_path_names_of_loaded_reference_modules(clean_modules):
    compat = pkg("compat")
    fake = {}
    for name, (_, names) in compat.HOT_PATH.items():
        m = types.ModuleType(name)
        for n in names:
            setattr(m, n, object())
        m.unrelated_name = "kept"
        sys.modules[name] = fake[name] = m
    done = compat.install_atlas_0709_alias()
    assert set(done.values()) == {"patched"}
    for name, (rel, names) in compat.HOT_PATH.items():
        ours = pkg(rel)
        for n in names:
            assert getattr(fake[name], n) is getattr(ours, n), (name, n)
        assert fake[name].unrelated_name == "kept"
