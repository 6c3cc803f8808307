"""Oracle: the rotary embedding of the verify layer step, rounded per op (numpy).

Test infrastructure only (see oracle/__init__.py).  Restates
apply_rope_with_cos_sin (flashinfer_full_verify.py:324-333) and rotate_half
(:227-229) as the reference runs them on 16-bit tensors, where every
elementwise op computes in fp32 and rounds its result to the tensor's dtype:

    out = rnd(rnd(x * cos) + rnd(rotate_half(x) * sin)),
    rotate_half(x) = cat(-x[..., D/2:], x[..., :D/2])

with cos / sin of shape [tokens, D] broadcast over heads (cos[:, None, :]).
The tables themselves are inputs (the caller builds them with rope_cos_sin,
:259-301).
"""

from __future__ import annotations

import numpy as np


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round fp32 values to fp16 or bf16 (round to nearest even) and return
    them as fp32."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        r = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
        out = r.astype(np.uint32).view(np.float32)
        return np.where(np.isnan(x), np.float32(np.nan), out)
    raise ValueError(f"dtype must be 'f16' or 'bf16', got {dtype!r}")


def rotate_half(x: np.ndarray) -> np.ndarray:
    h = x.shape[-1] // 2
    return np.concatenate((-x[..., h:], x[..., :h]), axis=-1)


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str) -> np.ndarray:
    """x [tokens, heads, D] (values of the dtype, held as fp32), cos / sin
    [tokens, D] -> the rotated x, fp32 holding values of the dtype."""
    x = np.asarray(x, dtype=np.float32)
    c = np.asarray(cos, dtype=np.float32)[:, None, :]
    s = np.asarray(sin, dtype=np.float32)[:, None, :]
    a = round_to(x * c, dtype)
    b = round_to(rotate_half(x) * s, dtype)
    return round_to(a + b, dtype)

