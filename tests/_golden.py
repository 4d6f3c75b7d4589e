"""Loader for the committed golden fixtures under tests/golden/ (made by tests/golden/make_golden.py)."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name: str) -> dict[str, torch.Tensor]:
    with np.load(GOLDEN / name, allow_pickle=False) as z:
        out = {}
        for k in z.files:
            a = z[k]
            if a.dtype == np.uint16:
                out[k] = torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
            else:
                out[k] = torch.from_numpy(np.array(a))
        return out
