"""Fused pointwise ops (reference wrappers: tinyvllm/kernels/pointwise.py:7-55;
host contracts tinyvllm/kernels/pointwise.cu:453-680).

Outputs are allocated here with ``torch.empty`` (inside graph capture they
come from the graph's private pool) and filled by the HIP kernels on the
current stream.
"""
from __future__ import annotations

import torch

from tinyvllm.kernels._extension import (
    check, dtype_code, load_kernels, require_gpu, stream_of,
)


def _rows(x: torch.Tensor) -> tuple[int, int, int, int, int]:
    """(tokens, heads, width, token_stride, head_stride) of a 2D/3D row tensor."""
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise RuntimeError("pointwise input must be float16, bfloat16 or float32")
    if x.dim() not in (2, 3):
        raise RuntimeError("pointwise input must be a strided 2D or 3D tensor")
    if x.shape[-1] <= 0 or x.stride(-1) != 1:
        raise RuntimeError("pointwise rows must have positive width and last stride 1")
    if x.dim() == 3:
        return x.shape[0], x.shape[1], x.shape[2], x.stride(0), x.stride(1)
    return x.shape[0], 1, x.shape[1], x.stride(0), 0


def _check_weight(x: torch.Tensor, weight: torch.Tensor) -> None:
    if (weight.device != x.device or weight.dtype != x.dtype or weight.dim() != 1
            or weight.numel() != x.shape[-1] or not weight.is_contiguous()):
        raise RuntimeError(
            "RMSNorm weight must be contiguous [width] with input device and dtype"
        )


def rms_norm(
    x: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
) -> torch.Tensor:
    """Normalize strided 2D/3D rows without packing a temporary input."""
    lib = load_kernels()
    device = require_gpu(x, weight)
    tokens, heads, width, ts, hs = _rows(x)
    _check_weight(x, weight)
    out = torch.empty(x.shape, dtype=x.dtype, device=device)
    if out.numel():
        check(lib.tvllm_rms_norm(
            x.data_ptr(), tokens, heads, width, ts, hs, weight.data_ptr(),
            None, 0, out.data_ptr(), None, float(eps), dtype_code(x.dtype),
            stream_of(device),
        ))
    return out


def add_rms_norm(
    x: torch.Tensor,
    residual: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Return normalized and rounded residual sums without modifying inputs."""
    lib = load_kernels()
    device = require_gpu(x, residual, weight)
    tokens, heads, width, ts, hs = _rows(x)
    _check_weight(x, weight)
    if (x.dim() != 2 or residual.dtype != x.dtype or residual.shape != x.shape
            or residual.stride(-1) != 1):
        raise RuntimeError(
            "residual must match the 2D input shape, device and dtype, with last stride 1"
        )
    out = torch.empty(x.shape, dtype=x.dtype, device=device)
    merged = torch.empty(x.shape, dtype=x.dtype, device=device)
    if out.numel():
        check(lib.tvllm_rms_norm(
            x.data_ptr(), tokens, heads, width, ts, hs, weight.data_ptr(),
            residual.data_ptr(), residual.stride(0), out.data_ptr(),
            merged.data_ptr(), float(eps), dtype_code(x.dtype), stream_of(device),
        ))
    return out, merged


def add_rms_norm_partials(
    partials: torch.Tensor,
    residual: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
) -> tuple[torch.Tensor, torch.Tensor]:
    """add_rms_norm whose x is ``round(partials.sum(0))``: the fp32 split-K
    partial products [splits, tokens, width] of a projection, summed and
    rounded to the residual's dtype inside the kernel (no reference
    counterpart; it replaces F.linear's rounding + add_rms_norm)."""
    lib = load_kernels()
    device = require_gpu(partials, residual, weight)
    if (partials.dtype != torch.float32 or partials.dim() != 3
            or not partials.is_contiguous()):
        raise RuntimeError("partials must be contiguous fp32 [splits, tokens, width]")
    splits, tokens, width = partials.shape
    if (residual.dim() != 2 or tuple(residual.shape) != (tokens, width)
            or residual.stride(-1) != 1 or residual.dtype not in (torch.float16, torch.bfloat16)):
        raise RuntimeError("residual must be a half-precision [tokens, width] tensor")
    _check_weight(residual, weight)
    out = torch.empty((tokens, width), dtype=residual.dtype, device=device)
    merged = torch.empty((tokens, width), dtype=residual.dtype, device=device)
    if out.numel():
        check(lib.tvllm_add_rms_norm_partials(
            partials.data_ptr(), splits, tokens * width, tokens, width, weight.data_ptr(),
            residual.data_ptr(), residual.stride(0), out.data_ptr(), merged.data_ptr(),
            float(eps), dtype_code(residual.dtype), stream_of(device),
        ))
    return out, merged


def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """Fuse the activation and gate/up product, preserving intermediate rounding."""
    lib = load_kernels()
    device = require_gpu(x)
    tokens, heads, width, ts, hs = _rows(x)
    if width % 2:
        raise RuntimeError("SiLU input width must be even")
    shape = list(x.shape)
    shape[-1] //= 2
    out = torch.empty(shape, dtype=x.dtype, device=device)
    if out.numel():
        check(lib.tvllm_silu_and_mul(
            x.data_ptr(), tokens, heads, width, ts, hs, out.data_ptr(),
            dtype_code(x.dtype), stream_of(device),
        ))
    return out


def _check_qk(query, key, query_weight, key_weight, cos, sin):
    if query.dim() != 3 or key.dim() != 3 or query.shape[0] != key.shape[0] \
            or query.shape[2] != key.shape[2] or key.dtype != query.dtype:
        raise RuntimeError("Q/K must match token count, head width, device and dtype")
    if query.dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError("Q/K must use float16 or bfloat16")
    if query.stride(2) != 1 or key.stride(2) != 1:
        raise RuntimeError("pointwise rows must have positive width and last stride 1")
    if query.shape[2] % 2:
        raise RuntimeError("RoPE input must be [tokens, heads, even head_dim]")
    _check_weight(query, query_weight)
    _check_weight(key, key_weight)
    for table in (cos, sin):
        if (table.dtype != query.dtype or table.dim() != 3
                or table.shape[0] != query.shape[0] or table.shape[1] != 1
                or table.shape[2] != query.shape[2] // 2 or not table.is_contiguous()):
            raise RuntimeError(
                "RoPE cos/sin must be contiguous [tokens, 1, head_dim/2] "
                "with input device and dtype"
            )


def qk_norm_rope(
    query: torch.Tensor,
    key: torch.Tensor,
    query_weight: torch.Tensor,
    key_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    query_eps: float = 1e-6,
    key_eps: float = 1e-6,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Normalize and rotate strided Q/K rows, preserving each rounding step."""
    lib = load_kernels()
    device = require_gpu(query, key, query_weight, key_weight, cos, sin)
    _check_qk(query, key, query_weight, key_weight, cos, sin)
    q_out = torch.empty(query.shape, dtype=query.dtype, device=device)
    k_out = torch.empty(key.shape, dtype=key.dtype, device=device)
    if query.shape[0]:
        check(lib.tvllm_qk_norm_rope(
            query.data_ptr(), query.stride(0), query.stride(1),
            key.data_ptr(), key.stride(0), key.stride(1),
            query_weight.data_ptr(), key_weight.data_ptr(), cos.data_ptr(),
            sin.data_ptr(), query.shape[0], query.shape[1], key.shape[1],
            query.shape[2], float(query_eps), float(key_eps),
            q_out.data_ptr(), k_out.data_ptr(), None, 0, 0, None, None, None, 0, 0, 0,
            dtype_code(query.dtype), dtype_code(query.dtype), 1.0, 1.0, stream_of(device),
        ))
    return q_out, k_out


def qk_norm_rope_store(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    query_weight: torch.Tensor,
    key_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    query_eps: float,
    key_eps: float,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slots: torch.Tensor,
    *,
    key_out: bool = False,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """qk_norm_rope with the slot-mapped KV write fused in (no reference
    counterpart: the reference runs store_kv after it,
    runtime/attention.py:219-233). The rotated K and the V rows go straight to
    ``key_cache/value_cache[slots[t]]`` (slot -1 skips). Returns the rotated
    Q and, if ``key_out``, a dense copy of the rotated K. An FP8 E4M3 cache
    (``torch.float8_e4m3fn``) stores ``fp8(clamp(x / scale))`` of each element
    with the given ``k_scale``/``v_scale``."""
    lib = load_kernels()
    device = require_gpu(query, key, value, query_weight, key_weight, cos, sin,
                         key_cache, value_cache, slots)
    _check_qk(query, key, query_weight, key_weight, cos, sin)
    if value.shape != key.shape or value.dtype != key.dtype or value.stride(2) != 1:
        raise RuntimeError("V must match K's shape and dtype with unit last stride")
    if (key_cache.dim() != 3 or tuple(key_cache.shape[1:]) != tuple(key.shape[1:])
            or value_cache.shape != key_cache.shape
            or value_cache.stride() != key_cache.stride() or key_cache.stride(2) != 1
            or value_cache.dtype != key_cache.dtype
            or key_cache.dtype not in (key.dtype, torch.float8_e4m3fn)):
        raise RuntimeError("KV caches must be [slots, kv_heads, dim] views of one layout "
                           "with unit last stride")
    if slots.dtype != torch.long or slots.dim() != 1 or not slots.is_contiguous() \
            or slots.numel() != key.shape[0]:
        raise RuntimeError("slots must be contiguous GPU int64 matching token rows")
    q_out = torch.empty(query.shape, dtype=query.dtype, device=device)
    k_out = torch.empty(key.shape, dtype=key.dtype, device=device) if key_out else None
    if query.shape[0]:
        check(lib.tvllm_qk_norm_rope(
            query.data_ptr(), query.stride(0), query.stride(1),
            key.data_ptr(), key.stride(0), key.stride(1),
            query_weight.data_ptr(), key_weight.data_ptr(), cos.data_ptr(),
            sin.data_ptr(), query.shape[0], query.shape[1], key.shape[1],
            query.shape[2], float(query_eps), float(key_eps),
            q_out.data_ptr(), k_out.data_ptr() if k_out is not None else None,
            value.data_ptr(), value.stride(0), value.stride(1),
            key_cache.data_ptr(), value_cache.data_ptr(), slots.data_ptr(),
            key_cache.shape[0], key_cache.stride(0), key_cache.stride(1),
            dtype_code(query.dtype), dtype_code(key_cache.dtype),
            float(k_scale), float(v_scale), stream_of(device),
        ))
    return q_out, k_out
