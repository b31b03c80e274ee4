"""Pointwise layer arithmetic restated on the CPU (test infrastructure only).

Each function applies the reference kernels' rounding points, which restate
the PyTorch/HF expressions (tinyvllm/kernels/pointwise.cu:95-116 rotate_pair,
:128-214 rms_norm_kernel, :260-321 silu_and_mul, :325-450 qk_norm_rope) on
fp32 intermediates; ``round`` is a cast to the storage dtype. With
dtype=float32 every rounding is the identity, which is what the pins against
transformers' fp32 Qwen3 modules use.
RoPE tables follow tinyvllm/layers.py:167-245 (fp32 inv_freq/cos/sin, gathered
per position, then cast to the storage dtype).
"""
from __future__ import annotations

import torch


def _round(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return x.to(dtype).float()


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """pointwise.cu:128-214 without residual: y = r(r(x * rsqrt(mean(x^2)+eps)) * w)."""
    dtype = x.dtype
    xf = x.float()
    inv = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (_round(xf * inv, dtype) * weight.float()).to(dtype)


def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                 eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor]:
    """pointwise.cu:156-162 + rms_norm: x = r(x + residual) first; returns (y, x)."""
    dtype = x.dtype
    merged = (x.float() + residual.float()).to(dtype)
    return rms_norm(merged, weight, eps), merged


def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """pointwise.cu:260-321: out = r(r(silu(g)) * u), [g | u] = halves of x."""
    dtype = x.dtype
    half = x.shape[-1] // 2
    g, u = x[..., :half].float(), x[..., half:].float()
    act = _round(g / (1.0 + torch.exp(-g)), dtype)
    return (act * u).to(dtype)


def rope_tables(positions: torch.Tensor, head_dim: int, theta: float,
                dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """layers.py:185-245: [tokens, 1, head_dim/2] cos/sin in the storage dtype."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    freqs = positions.float()[:, None] * inv_freq[None, :]
    return freqs.cos().to(dtype).unsqueeze(1), freqs.sin().to(dtype).unsqueeze(1)


def rope_tables_from_max(positions: torch.Tensor, head_dim: int, theta: float,
                         max_position: int, dtype: torch.dtype):
    """Exactly layers.py:192-245: outer(arange(max_position), inv_freq) then
    index_select(positions) -- identical values to rope_tables (same fp32 ops)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    table = torch.outer(torch.arange(max_position, dtype=torch.float32), inv_freq)
    cos = table.cos().index_select(0, positions).to(dtype).unsqueeze(1)
    sin = table.sin().index_select(0, positions).to(dtype).unsqueeze(1)
    return cos, sin


def qk_norm_rope(q: torch.Tensor, k: torch.Tensor, qw: torch.Tensor, kw: torch.Tensor,
                 cos: torch.Tensor, sin: torch.Tensor, q_eps: float = 1e-6,
                 k_eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor]:
    """pointwise.cu:325-450 with rotate_pair (:95-116): per-head RMSNorm then
    half-split RoPE, o1 = r(r(n1 c) - r(n2 s)), o2 = r(r(n2 c) + r(n1 s))."""

    def one(x, w, eps):
        dtype = x.dtype
        n = rms_norm(x, w, eps).float()
        half = x.shape[-1] // 2
        n1, n2 = n[..., :half], n[..., half:]
        c, s = cos.float(), sin.float()
        o1 = _round(n1 * c, dtype) - _round(n2 * s, dtype)
        o2 = _round(n2 * c, dtype) + _round(n1 * s, dtype)
        return torch.cat([o1, o2], dim=-1).to(dtype)

    return one(q, qw, q_eps), one(k, kw, k_eps)
