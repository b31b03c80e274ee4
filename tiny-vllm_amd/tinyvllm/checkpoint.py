"""safetensors weight loading (reference: tinyvllm/checkpoint.py:84-143)."""
from __future__ import annotations

import json
from pathlib import Path

import torch


def checkpoint_files(model_dir: str | Path) -> list[Path]:
    """Shards named by model.safetensors.index.json, else every *.safetensors."""
    root = Path(model_dir)
    index = root / "model.safetensors.index.json"
    if index.exists():
        weight_map = json.loads(index.read_text(encoding="utf-8"))["weight_map"]
        return [root / name for name in sorted(set(weight_map.values()))]
    files = sorted(root.glob("*.safetensors"))
    if not files:
        raise ValueError(f"no safetensors checkpoint in {root}")
    return files


@torch.no_grad()
def load_weights(model, model_dir: str | Path) -> None:
    """Route every checkpoint tensor through ``model.load_weight``; fail if a
    required tensor is missing or loaded twice."""
    from safetensors import safe_open

    device = next(model.parameters()).device
    loaded: set[str] = set()
    for path in checkpoint_files(model_dir):
        with safe_open(str(path), framework="pt", device="cpu") as f:
            for name in f.keys():
                target = model.load_weight(name, f.get_tensor(name).to(device))
                if target in loaded:
                    raise ValueError(f"weight loaded twice: {name}")
                loaded.add(target)
    missing = set(model.required_weight_names) - loaded
    if missing:
        raise ValueError(f"missing weights: {sorted(missing)[:5]} ...")
