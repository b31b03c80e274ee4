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


# ------------------------------------------------------------ FP8 layout --
# The optional FP8 KV layout has no reference counterpart; its definition is
# OCP FP8 E4M3 ("e4m3fn": 1 sign, 4 exponent bits with bias 7, 3 mantissa
# bits, no infinities, NaN = S.1111.111, max 448), stored = nearest-even
# E4M3 of clamp(x * (1 / scale), -448, 448) computed in float32, read back as
# stored * scale.

FP8_MAX = 448.0


def e4m3_value(code: int) -> float:
    """Closed form of one E4M3 code (the textbook definition)."""
    sign = -1.0 if code & 0x80 else 1.0
    exponent = (code >> 3) & 0xF
    mantissa = code & 0x7
    if exponent == 0xF and mantissa == 0x7:
        return float("nan")
    if exponent == 0:
        return sign * (mantissa / 8.0) * 2.0 ** -6
    return sign * (1.0 + mantissa / 8.0) * 2.0 ** (exponent - 7)


def e4m3_table() -> np.ndarray:
    """Values of all 256 codes (float64)."""
    return np.array([e4m3_value(c) for c in range(256)], dtype=np.float64)


def fp8_inverse_scale(scale: float) -> np.float32:
    """1 / scale rounded to float32, as the kernels compute it."""
    return np.float32(1.0) / np.float32(scale)


def fp8_quantize(x: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """uint8 E4M3 codes of clamp(x * (1/scale)) (float32 product, nearest-even).
    Uses torch's float8_e4m3fn cast, pinned against ``e4m3_table`` by the
    oracle tests (nearest value, ties to an even mantissa)."""
    inv = torch.tensor(float(fp8_inverse_scale(scale)), dtype=torch.float32)
    y = (x.float() * inv).clamp(-FP8_MAX, FP8_MAX)
    return y.to(torch.float8_e4m3fn).view(torch.uint8)


def fp8_dequantize(codes: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """float32 values stored * scale of uint8 E4M3 codes."""
    return codes.view(torch.float8_e4m3fn).float() * torch.tensor(scale, dtype=torch.float32)
