"""Shared helpers of the test-suite (imports the package by its directory name)."""

import importlib
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pkg(name: str = ""):
    return importlib.import_module("0709_amd" + (f".{name}" if name else ""))


def bits16(t):
    """View a 16-bit float tensor/array as uint16 for bit-exact comparison."""
    import numpy as np
    import torch

    if isinstance(t, torch.Tensor):
        return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    return np.asarray(t).view(np.uint16)
