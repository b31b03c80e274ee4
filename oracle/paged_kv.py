"""Paged-KV arithmetic restated on the CPU (test infrastructure only).

Reference: tinyvllm/paged_kv.py:53-127 (layout, write via index_copy_, read
via index_select), tinyvllm/cache.py:696-711 (_slot_for_position),
tinyvllm/runtime/contracts.py:108-116 (logical-order read slots),
tinyvllm/runtime/inputs.py:94-98 (graph padding: slot -1, length 0).
"""
from __future__ import annotations

import numpy as np
import torch


def slot_for_position(table: list[int] | np.ndarray, position: int, block_size: int) -> int:
    """cache.py:696-711: physical slot of logical token ``position``."""
    return int(table[position // block_size]) * block_size + position % block_size


def slot_mapping(table, start: int, end: int, block_size: int) -> np.ndarray:
    """Slots of positions [start, end) (batch.py:232-244 + cache.py:567-573)."""
    return np.array([slot_for_position(table, p, block_size) for p in range(start, end)],
                    dtype=np.int64)


def read_slots(table, length: int, block_size: int) -> torch.Tensor:
    """contracts.py:108-116: physical slots of positions [0, length) in order."""
    positions = torch.arange(length, dtype=torch.long)
    physical = torch.as_tensor(np.asarray(table, dtype=np.int64))[positions // block_size]
    return physical * block_size + positions % block_size


def kv_write(key_cache: torch.Tensor, value_cache: torch.Tensor, slots: torch.Tensor,
             key: torch.Tensor, value: torch.Tensor) -> None:
    """paged_kv.py:68-108 (index_copy_), plus kv_store.cu:42-44: slot -1 skips."""
    keep = slots >= 0
    key_cache.index_copy_(0, slots[keep], key[keep])
    value_cache.index_copy_(0, slots[keep], value[keep])


def kv_read(key_cache: torch.Tensor, value_cache: torch.Tensor, slots: torch.Tensor):
    """paged_kv.py:111-127 (index_select)."""
    return key_cache.index_select(0, slots), value_cache.index_select(0, slots)
