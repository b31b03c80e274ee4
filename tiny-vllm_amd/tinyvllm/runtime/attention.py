"""Attention backends over the paged KV cache
(reference: tinyvllm/runtime/attention.py:12-348).

``HipAttention`` (the default, "hip") runs everything on the gfx950 kernels:
  * decode-only steps (head dim 128, GQA group <= 16): one kernel per layer
    does QK-norm + RoPE, the slot-mapped KV write and split-K paged decode
    attention;
  * other steps, ``prepare_qkv``: QK-norm + RoPE with the KV write fused in;
  * decode rows (query length 1): split-K paged decode attention;
  * multi-query rows (fresh prompts and chunks with history): MFMA paged
    prefill attention, reading the just-written chunk from the cache too;
  * other head dims (up to 256; the reference dispatches 32, 64, 128, 256)
    take the same calls, served by the library's general kernel.
``SDPAAttention`` ("reference") is the reference's own torch algorithm
(gather in logical order + ``F.scaled_dot_product_attention``) kept for
cross-checking; it is only used when selected explicitly.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from tinyvllm.kernels.kv_store import store_kv
from tinyvllm.kernels.paged_decode import (
    paged_decode_attention,
    paged_decode_qk_norm_rope,
    paged_decode_qk_norm_rope_partials,
)
from tinyvllm.kernels.paged_prefill import paged_prefill_attention
from tinyvllm.kernels.pointwise import qk_norm_rope, qk_norm_rope_store
from tinyvllm.paged_kv import PagedKVCache
from tinyvllm.runtime.contracts import ModelInput

BACKENDS = ("hip", "reference")


class HipAttention:
    """Fused KV write, paged decode and paged chunked prefill on HIP kernels."""

    def __init__(self, model_input: ModelInput, cache: PagedKVCache, *,
                 decode_workspace: torch.Tensor | None = None) -> None:
        self.kv = model_input.kv
        self.cache = cache
        self.decode_workspace = decode_workspace
        self._written_layer = -1
        self._fused = None

    def fuses_decode(self, num_heads: int) -> bool:
        """Decode-only steps whose shape the fused decode kernel takes (head
        dim 128, GQA group <= 16): QK-norm + RoPE + KV write + attention in
        one launch. Other head dims run the unfused kernels (QK-norm + RoPE
        with the KV write, then the general paged-attention kernel)."""
        group = num_heads // self.cache.num_kv_heads
        return (self.kv.prefill is None and self.kv.decode is not None
                and self.cache.head_dim == 128 and 1 <= group <= 16)

    def takes_qkv_partials(self, num_heads: int) -> bool:
        """Decode-only steps: the fused decode kernel can take the qkv
        projection as split-K partials (``attend_qkv_partials``)."""
        return self.fuses_decode(num_heads)

    def attend_qkv_partials(self, layer_idx, parts, num_heads, q_weight, k_weight, cos, sin,
                            q_eps, k_eps, *, scale):
        """QK-norm + RoPE + KV write + paged decode of a decode-only step from
        the qkv projection's fp32 split-K partials [4, tokens, width]."""
        output = torch.empty((parts.shape[1], num_heads, 128), dtype=q_weight.dtype,
                             device=parts.device)
        paged_decode_qk_norm_rope_partials(parts, num_heads, q_weight, k_weight, cos, sin,
                                           q_eps, k_eps, self.cache, layer_idx,
                                           self.kv.decode, self.kv.slot_mapping, output,
                                           scale=scale, workspace=self.decode_workspace)
        return output

    def prepare_qkv(self, layer_idx, q, k, v, q_weight, k_weight, cos, sin, q_eps, k_eps):
        """Decode-only steps: keep the raw Q/K/V for the fused decode kernel
        (QK-norm + RoPE + KV write + attention in one launch). Otherwise
        normalise/rotate Q and K and write K/V into their cache slots in one
        kernel and return (q, None, None) - K/V now live in the cache."""
        if self.fuses_decode(q.shape[1]):
            self._fused = (layer_idx, k, v, q_weight, k_weight, cos, sin, q_eps, k_eps)
            return q, None, None
        q, _ = qk_norm_rope_store(
            q, k, v, q_weight, k_weight, cos, sin, q_eps, k_eps,
            self.cache.key[layer_idx], self.cache.value[layer_idx], self.kv.slot_mapping,
            k_scale=self.cache.k_scale, v_scale=self.cache.v_scale,
        )
        self._written_layer = layer_idx
        return q, None, None

    def __call__(self, layer_idx: int, q: torch.Tensor, k: torch.Tensor | None,
                 v: torch.Tensor | None, *, scale: float) -> torch.Tensor:
        output = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        fused, self._fused = self._fused, None
        if fused is not None and fused[0] == layer_idx:
            _, k_raw, v_raw, qw, kw, cos, sin, q_eps, k_eps = fused
            paged_decode_qk_norm_rope(q, k_raw, v_raw, qw, kw, cos, sin, q_eps, k_eps,
                                      self.cache, layer_idx, self.kv.decode,
                                      self.kv.slot_mapping, output, scale=scale,
                                      workspace=self.decode_workspace)
            return output
        if self._written_layer != layer_idx:
            store_kv(self.cache, layer_idx, self.kv.slot_mapping, k, v)
        if self.kv.decode is not None:
            paged_decode_attention(q, self.cache, layer_idx, self.kv.decode, output,
                                   scale=scale, workspace=self.decode_workspace)
        if self.kv.prefill is not None:
            paged_prefill_attention(q, self.cache, layer_idx, self.kv.prefill, output,
                                    scale=scale)
        return output


class SDPAAttention:
    """The reference's torch path: per-row gather + SDPA (attention.py:12-151).

    Needs the CPU-side batch geometry (query/context lengths and tables)."""

    def __init__(self, model_input: ModelInput, cache: PagedKVCache, *,
                 q_offsets, context_lens_before, context_lens_after, block_tables) -> None:
        self.kv = model_input.kv
        self.cache = cache
        self.q_offsets = q_offsets
        self.before = context_lens_before
        self.after = context_lens_after
        self.read_slots = []
        bs = cache.block_size
        for table, length in zip(block_tables, context_lens_after):
            positions = torch.arange(length, dtype=torch.long)
            physical = torch.tensor(table, dtype=torch.long)[positions // bs]
            self.read_slots.append((physical * bs + positions % bs).to(cache.device))

    def __call__(self, layer_idx, q, k, v, *, scale):
        store_kv(self.cache, layer_idx, self.kv.slot_mapping, k, v)
        output = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        for index, slots in enumerate(self.read_slots):
            start, end = self.q_offsets[index], self.q_offsets[index + 1]
            keys, values = self.cache.read(layer_idx, slots)
            keys, values = keys.to(q.dtype), values.to(q.dtype)
            before, after = self.before[index], self.after[index]
            query = q[start:end].transpose(0, 1).unsqueeze(0)
            mask = None
            if end - start > 1 and before > 0:
                qpos = torch.arange(before, after, device=q.device)[:, None]
                mask = (torch.arange(after, device=q.device)[None, :] <= qpos)[None, None]
            attended = F.scaled_dot_product_attention(
                query, keys.transpose(0, 1).unsqueeze(0), values.transpose(0, 1).unsqueeze(0),
                attn_mask=mask, is_causal=mask is None and end - start > 1, scale=scale,
                enable_gqa=q.shape[1] != self.cache.num_kv_heads,
            )
            output[start:end].copy_(attended.squeeze(0).transpose(0, 1))
        return output


def check_backend(name: str, model: torch.nn.Module) -> str:
    """Validate a backend choice against the model once, at construction
    (reference attention.py:314-348). "cuda" is accepted as the reference's
    name for its native-kernel backend and maps to "hip"."""
    if name == "cuda":
        name = "hip"
    if name not in BACKENDS:
        raise ValueError(f"unsupported attention backend: {name}")
    parameter = next(model.parameters())
    config = model.config
    if parameter.device.type != "cuda" or parameter.dtype not in (torch.float16,
                                                                   torch.bfloat16):
        raise ValueError("GPU attention requires float16 or bfloat16 weights on the GPU")
    if name == "hip" and not (0 < config.head_dim <= 256 and config.head_dim % 2 == 0):
        raise ValueError("the hip backend's paged kernels take even head dims up to 256")
    if config.num_attention_heads % config.num_key_value_heads:
        raise ValueError("query heads must be divisible by KV heads")
    from tinyvllm.kernels._extension import load_kernels

    load_kernels()  # fail at construction, before KV allocation
    return name


__all__ = ["HipAttention", "SDPAAttention", "check_backend", "BACKENDS", "qk_norm_rope"]
