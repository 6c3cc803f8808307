"""Drafter-side paged-KV pieces (drop-in for ``atlas_0709.flashinfer_paged``):
paged metadata, route-pool bridge (tail-page COW, promote, prune) and the
native paged pools it drives."""
