"""MI355X-native paged-KV tree path of ATLAS 0709.

Drop-in modules (same names and call signatures as the reference package
``atlas_0709``) backed by hand-written gfx950 HIP kernels behind the C ABI in
``include/atlas0709.h``:

* ``flashinfer_full_verify`` -- tree dedup, TreeSpec / ancestor mask,
  ``write_suffix_kv``, paged prefix conversion, the verify-attention plan;
* ``tree_attention``         -- ``BatchPrefillWithPagedKVCacheWrapper`` (plan/run);
* ``kv_ops``                 -- all-layer append, move (COW) and commit kernels;
* ``flashinfer_paged``       -- paged metadata, route-pool bridge, native pools;
* ``target_runtime``         -- Target commit / capacity / scoring / selection.

The package directory name starts with a digit, so import it with
``importlib.import_module("0709_amd")``; ``compat.install_atlas_0709_alias()``
registers it under the reference's module names.
"""

from . import _lib

__all__ = ["_lib"]
__version__ = "0.1.0"
