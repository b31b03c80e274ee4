"""Paged KV-cache storage (reference: tinyvllm/paged_kv.py:10-139).

Layout contract (kept identical to the reference, paged_kv.py:53-65):
``key``/``value`` are ``[num_layers, num_blocks * block_size, num_kv_heads,
head_dim]``; token position p of a request whose block table is ``table``
lives at slot ``table[p // block_size] * block_size + p % block_size``.
One slot row of one layer is ``num_kv_heads * head_dim`` contiguous elements
(2 KiB for Qwen3's 8 x 128 bf16), so a 16-token page of one layer is 32 KiB
of contiguous HBM.

Slots and block ids are validated on the CPU before lowering (ModelRunner);
this class checks shapes/devices only and never synchronises on GPU values.

Optional FP8 layout (no reference counterpart): ``dtype=torch.float8_e4m3fn``
keeps the same shapes with one byte per element, half the bytes of bf16.
Writes store ``fp8(clamp(x * (1 / k_scale), -448, 448))`` (nearest-even),
reads see ``stored * k_scale`` (likewise ``v_scale`` for V); the kernels fold
the scales into the softmax scale and the output normalisation.
"""
from __future__ import annotations

import torch

from tinyvllm._validation import _check_non_negative_int, _check_positive_int

FP8_DTYPE = torch.float8_e4m3fn
_MODEL_DTYPES = (torch.float16, torch.bfloat16)


class PagedKVCache:
    """Device storage only. Slots must come from a validated CPU batch."""

    def __init__(
        self,
        *,
        num_layers: int,
        num_blocks: int,
        block_size: int,
        num_kv_heads: int,
        head_dim: int,
        device: torch.device | str,
        dtype: torch.dtype,
        k_scale: float = 1.0,
        v_scale: float = 1.0,
    ) -> None:
        for name, value in (
            ("num_layers", num_layers),
            ("num_blocks", num_blocks),
            ("block_size", block_size),
            ("num_kv_heads", num_kv_heads),
            ("head_dim", head_dim),
        ):
            _check_positive_int(name, value)
        for name, value in (("k_scale", k_scale), ("v_scale", v_scale)):
            if type(value) not in (int, float) or not 0.0 < value < float("inf"):
                raise ValueError(f"{name} must be a positive finite number")
        if dtype != FP8_DTYPE and (k_scale != 1.0 or v_scale != 1.0):
            raise ValueError("KV scales apply to an FP8 cache only")
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = device
        self.dtype = dtype
        self.fp8 = dtype == FP8_DTYPE
        self.k_scale = float(k_scale)
        self.v_scale = float(v_scale)
        self.num_layers = num_layers
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.num_slots = num_blocks * block_size
        shape = (num_layers, self.num_slots, num_kv_heads, head_dim)
        self.key = torch.empty(shape, device=device, dtype=dtype)
        self.value = torch.empty_like(self.key)

    @staticmethod
    def bytes_per_block(
        *, num_layers: int, block_size: int, num_kv_heads: int, head_dim: int,
        dtype: torch.dtype,
    ) -> int:
        """K + V bytes one block occupies across all layers."""
        element = torch.empty((), dtype=dtype).element_size()
        return 2 * num_layers * block_size * num_kv_heads * head_dim * element

    def write(
        self,
        layer_idx: int,
        slots: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
    ) -> None:
        """cache[layer][slots[t]] = key[t], value[t] (scatter on the GPU)."""
        self._check_indices(layer_idx, slots)
        expected = (slots.numel(), self.num_kv_heads, self.head_dim)
        if tuple(key.shape) != expected or tuple(value.shape) != expected:
            raise ValueError("K/V rows do not match the slot mapping")
        if key.device != self.device or value.device != self.device:
            raise ValueError("K/V tensors must use the cache device")
        allowed = _MODEL_DTYPES if self.fp8 else (self.dtype,)
        if key.dtype not in allowed or value.dtype != key.dtype:
            raise ValueError("K/V tensors must use the cache dtype")
        from tinyvllm.kernels.kv_store import store_kv

        store_kv(self, layer_idx, slots, key, value)

    def read(
        self,
        layer_idx: int,
        slots: torch.Tensor,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Gather rows ``slots`` of one layer (logical order of the caller);
        an FP8 cache returns the dequantised rows (float32)."""
        self._check_indices(layer_idx, slots)
        keys = self.key[layer_idx].index_select(0, slots)
        values = self.value[layer_idx].index_select(0, slots)
        if self.fp8:
            return keys.float() * self.k_scale, values.float() * self.v_scale
        return keys, values

    def _check_indices(self, layer_idx: int, slots: torch.Tensor) -> None:
        _check_non_negative_int("layer_idx", layer_idx)
        if layer_idx >= self.num_layers:
            raise ValueError("layer_idx is out of range")
        if not isinstance(slots, torch.Tensor):
            raise TypeError("slots must be a torch.Tensor")
        if slots.ndim != 1 or slots.dtype is not torch.long:
            raise ValueError("slots must be a one-dimensional int64 tensor")
        if slots.device != self.device:
            raise ValueError("slots must use the cache device")
