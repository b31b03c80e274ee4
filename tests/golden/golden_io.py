"""Reading and writing the golden fixtures: ``.npz`` archives of plain
arrays (no pickled objects). bf16 tensors are stored as their uint16 bit
patterns under a name ending in ``__bf16``, so every fixture round-trips
bit for bit."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
BF16 = "__bf16"


def save(name: str, arrays: dict) -> Path:
    out = {}
    for key, value in arrays.items():
        if isinstance(value, torch.Tensor):
            if value.dtype == torch.bfloat16:
                out[key + BF16] = value.contiguous().view(torch.int16).numpy().view(np.uint16)
            else:
                out[key] = value.contiguous().numpy()
        else:
            out[key] = np.asarray(value)
    path = HERE / f"{name}.npz"
    np.savez_compressed(path, **out)
    return path


def load(name: str) -> dict:
    """Fixture ``name`` as torch tensors (bf16 restored from its bits)."""
    result = {}
    with np.load(HERE / f"{name}.npz", allow_pickle=False) as data:
        for key in data.files:
            array = data[key]
            if key.endswith(BF16):
                result[key[:-len(BF16)]] = torch.from_numpy(
                    array.view(np.int16).copy()).view(torch.bfloat16)
            else:
                result[key] = torch.from_numpy(array.copy())
    return result
