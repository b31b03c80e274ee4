"""KV-cache scatter (reference wrapper: tinyvllm/kernels/kv_store.py:10-30)."""
from __future__ import annotations

import torch

from tinyvllm._validation import _check_non_negative_int
from tinyvllm.kernels._extension import (
    cache_format, check, dtype_code, load_kernels, require_gpu, stream_of,
)
from tinyvllm.paged_kv import PagedKVCache


def store_kv(
    cache: PagedKVCache,
    layer_idx: int,
    slots: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
) -> None:
    """Scatter CPU-validated real slots; -1 skips internal graph padding."""
    _check_non_negative_int("layer_idx", layer_idx)
    if layer_idx >= cache.num_layers:
        raise ValueError("layer_idx is out of range")
    lib = load_kernels()
    key_cache, value_cache = cache.key[layer_idx], cache.value[layer_idx]
    device = require_gpu(key, value, key_cache, value_cache, slots)
    if key.dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError("KV store requires float16 or bfloat16")
    if key_cache.stride() != value_cache.stride():
        raise RuntimeError("K/V caches must share one layout")
    for tensor in (value,) if cache.fp8 else (value, key_cache, value_cache):
        if tensor.dtype != key.dtype:
            raise RuntimeError("KV dtype mismatch")
    if key.dim() != 3 or value.dim() != 3:
        raise RuntimeError("KV tensors must have three dimensions")
    if value.shape != key.shape:
        raise RuntimeError("K/V shape mismatch")
    if tuple(key.shape[1:]) != tuple(key_cache.shape[1:]) or key.shape[1] == 0:
        raise RuntimeError("KV head geometry mismatch")
    if key.stride(2) != 1 or value.stride(2) != 1:
        raise RuntimeError("K/V rows must have unit last stride")
    if slots.dtype != torch.long or slots.dim() != 1 or not slots.is_contiguous() \
            or slots.numel() != key.shape[0]:
        raise RuntimeError("slots must be contiguous GPU int64 matching token rows")
    check(lib.tvllm_store_kv(
        key.data_ptr(), value.data_ptr(),
        key.stride(0), key.stride(1), value.stride(0), value.stride(1),
        key_cache.data_ptr(), value_cache.data_ptr(), slots.data_ptr(),
        key.shape[0], key.shape[1], key.shape[2], key_cache.shape[0],
        key_cache.stride(0), key_cache.stride(1), dtype_code(key.dtype), *cache_format(cache), stream_of(device),
    ))


def apply_table_updates(table: torch.Tensor, updates: torch.Tensor) -> None:
    """In place on the device: ``table[updates[1 + 2i]] = updates[2 + 2i]``
    for ``i < updates[0]`` (the count is read on the device, so a captured
    graph applies each step's own upload). Both int64, contiguous, 1-D."""
    lib = load_kernels()
    device = require_gpu(table, updates)
    for tensor in (table, updates):
        if tensor.dtype != torch.long or tensor.dim() != 1 or not tensor.is_contiguous():
            raise RuntimeError("apply_table_updates takes contiguous 1-D int64 tensors")
    if updates.numel() < 1:
        raise RuntimeError("updates needs its count word")
    capacity = (updates.numel() - 1) // 2
    check(lib.tvllm_apply_table_updates(table.data_ptr(), table.numel(), updates.data_ptr(),
                                        capacity, stream_of(device)))
