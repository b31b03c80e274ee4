"""Paged KV-cache storage (reference: tinyvllm/paged_kv.py:10-139).

Layout contract (kept identical to the reference, paged_kv.py:53-65):
``key``/``value`` are ``[num_layers, num_blocks * block_size, num_kv_heads,
head_dim]`` tensors; token position p of a request whose block table is
``table`` lives at slot ``table[p // block_size] * block_size + p %
block_size``, and ``key[layer][slot]`` is that token's [kv_heads, head_dim]
row, indexed exactly as in the reference.

Storage underneath: ``layout="token_major"`` (default) stores that shape
contiguously, as the reference does: one slot row of one layer is
``num_kv_heads * head_dim`` elements (2 KiB for Qwen3's 8 x 128 bf16), and a
16-token page of one KV head is 16 pieces of 256 bytes at a 2 KiB stride.
``layout="head_major"`` (beyond the reference) stores ``[num_layers,
num_kv_heads, num_slots, head_dim]`` and makes ``key``/``value`` permuted
views of it, so that page is 4 KiB of contiguous HBM. Gathered 4 KiB pages
stream at 6.6-6.7 TB/s on MI355X when at least four waves read each head,
the 256-byte pieces at 6.3-6.35 TB/s; with two waves per head the pieces
read faster (5.25 vs 5.05 TB/s), since the heads of a token then arrive
together. So head-major pays for few rows with long contexts (Qwen3-32B,
16 rows at 16-32k: 253 -> 238 us per decode call) and costs at many rows
(Qwen3-8B, 64 rows at 2k: 87.5 -> 90.3 us). The kernels take the views'
slot and head strides, so they serve either.

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
LAYOUTS = ("head_major", "token_major")


def resolve_layout(layout: str, max_rows: int, kv_heads: int) -> str:
    """``layout``, with "auto" resolved for a cache read by at most
    ``max_rows`` decode rows at once: head-major below 256 (row, KV head)
    pairs (few rows, so long contexts split into many waves per head),
    token-major otherwise."""
    if layout == "auto":
        return "head_major" if max_rows * kv_heads < 256 else "token_major"
    if layout not in LAYOUTS:
        raise ValueError(f"layout must be 'auto' or one of {LAYOUTS}")
    return layout


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
        layout: str = "token_major",
    ) -> None:
        if layout not in LAYOUTS:
            raise ValueError(f"layout must be one of {LAYOUTS}")
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
        self.layout = layout
        if layout == "head_major":
            shape = (num_layers, num_kv_heads, self.num_slots, head_dim)
            self.key = torch.empty(shape, device=device, dtype=dtype).permute(0, 2, 1, 3)
            self.value = torch.empty(shape, device=device, dtype=dtype).permute(0, 2, 1, 3)
        else:
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
