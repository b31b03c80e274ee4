"""Paged decode attention (reference wrapper: tinyvllm/kernels/paged_decode.py:10-32;
host contract tinyvllm/kernels/paged_decode.cu:469-669)."""
from __future__ import annotations

import torch

from tinyvllm.kernels._extension import (
    cache_format, check, dtype_code, load_kernels, require_gpu, stream_of,
)
from tinyvllm.paged_kv import PagedKVCache
from tinyvllm.runtime.contracts import SingleQueryMetadata


def decode_workspace_bytes(
    num_rows: int, num_heads: int, num_kv_heads: int, head_dim: int,
    max_context_len: int, block_size: int,
) -> int:
    """Split-K scratch the decode kernel needs for this geometry."""
    return int(load_kernels().tvllm_paged_decode_workspace_size(
        num_rows, num_heads, num_kv_heads, head_dim, max_context_len, block_size,
    ))


def decode_split_plan(
    num_rows: int, num_heads: int, num_kv_heads: int, head_dim: int,
    max_context_len: int, block_size: int,
) -> int:
    """Opaque id of the split-K decomposition for this geometry (equal ids:
    identical launches)."""
    return int(load_kernels().tvllm_paged_decode_split_plan(
        num_rows, num_heads, num_kv_heads, head_dim, max_context_len, block_size,
    ))


def paged_decode_attention(
    q: torch.Tensor,
    cache: PagedKVCache,
    layer_idx: int,
    metadata: SingleQueryMetadata,
    output: torch.Tensor,
    *,
    scale: float,
    workspace: torch.Tensor | None = None,
) -> None:
    """Fill selected rows on the current stream; zero-length padding yields zeros.

    ``workspace`` (optional, uint8, >= decode_workspace_bytes) holds split-K
    partials; when omitted it is allocated from torch's caching allocator
    (inside graph capture that is the graph's private pool).
    """
    lib = load_kernels()
    k, v = cache.key[layer_idx], cache.value[layer_idx]
    rows = metadata.query_rows
    blocks = metadata.block_table_ids
    offsets = metadata.block_table_offsets
    lengths = metadata.context_lens
    device = require_gpu(q, k, v, output, rows, blocks, offsets, lengths)
    if q.dim() != 3:
        raise RuntimeError("Q must be a GPU [tokens, heads, dim] tensor")
    if k.stride() != v.stride():
        raise RuntimeError("K/V caches must share one layout")
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError("Q must use float16 or bfloat16")
    if (k.dtype != q.dtype and not cache.fp8) or output.dtype != q.dtype:
        raise RuntimeError("Q/K/V/output must share device and dtype")
    if output.shape != q.shape or q.stride(2) != 1 or output.stride(2) != 1:
        raise RuntimeError("output must match Q shape with unit last stride")
    for tensor in (rows, blocks, offsets, lengths):
        if tensor.dtype != torch.long or tensor.dim() != 1 or not tensor.is_contiguous():
            raise RuntimeError(
                "metadata must be contiguous GPU int64 vectors on Q's device"
            )
    if rows.numel() != lengths.numel() or offsets.numel() != rows.numel() + 1:
        raise RuntimeError("metadata lengths must align")
    num_rows = rows.numel()
    if num_rows == 0:
        return
    heads, dim = q.shape[1], q.shape[2]
    max_len = metadata.max_context_len or cache.num_slots
    need = int(lib.tvllm_paged_decode_workspace_size(
        num_rows, heads, cache.num_kv_heads, dim, max_len, cache.block_size,
    ))
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=device)
    check(lib.tvllm_paged_decode(
        q.data_ptr(), q.stride(0), q.stride(1),
        k.data_ptr(), v.data_ptr(),
        output.data_ptr(), output.stride(0), output.stride(1),
        rows.data_ptr(), blocks.data_ptr(), offsets.data_ptr(), lengths.data_ptr(),
        num_rows, heads, cache.num_kv_heads, dim, cache.num_slots, k.stride(0), k.stride(1),
        cache.block_size, max_len, float(scale),
        workspace.data_ptr() if need else None, need,
        dtype_code(q.dtype), *cache_format(cache), stream_of(device),
    ))


def paged_decode_qk_norm_rope(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    query_weight: torch.Tensor,
    key_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    query_eps: float,
    key_eps: float,
    cache: PagedKVCache,
    layer_idx: int,
    metadata: SingleQueryMetadata,
    slots: torch.Tensor,
    output: torch.Tensor,
    *,
    scale: float,
    workspace: torch.Tensor | None = None,
) -> None:
    """One decode step's QK-norm + RoPE, slot-mapped KV write and paged
    attention in one kernel (no reference counterpart: it replaces
    qk_norm_rope + store_kv + paged_decode_attention when every row is a
    decode row). ``q``/``k``/``v`` are the raw projections [tokens, heads,
    128]; ``cos``/``sin`` the [tokens, 1, 64] RoPE tables; ``slots`` the
    write slot of each token (-1 skips); ``metadata.query_rows`` index those
    tokens. The K rows written equal ``qk_norm_rope_store``'s bit for bit."""
    lib = load_kernels()
    kc, vc = cache.key[layer_idx], cache.value[layer_idx]
    m = metadata
    device = require_gpu(q, k, v, query_weight, key_weight, cos, sin, slots, kc, output,
                         m.query_rows, m.block_table_ids, m.block_table_offsets,
                         m.context_lens)
    if q.dim() != 3 or k.dim() != 3 or v.shape != k.shape or q.shape[2] != 128:
        raise RuntimeError("Q/K/V must be [tokens, heads, 128] tensors")
    if q.dtype not in (torch.float16, torch.bfloat16) or any(
            t.dtype != q.dtype for t in (k, v, query_weight, key_weight, cos, sin, output)) \
            or (kc.dtype != q.dtype and not cache.fp8):
        raise RuntimeError("Q/K/V, weights, RoPE tables and cache must share a half dtype")
    if vc.stride() != kc.stride():
        raise RuntimeError("K/V caches must share one layout")
    if any(t.stride(-1) != 1 for t in (q, k, v, output)) or output.shape != q.shape:
        raise RuntimeError("Q/K/V/output rows must have unit last stride")
    if (query_weight.shape != (128,) or key_weight.shape != (128,)
            or not query_weight.is_contiguous() or not key_weight.is_contiguous()):
        raise RuntimeError("norm weights must be contiguous [128]")
    tokens = q.shape[0]
    for table in (cos, sin):
        if table.numel() != tokens * 64 or not table.is_contiguous():
            raise RuntimeError("RoPE tables must be contiguous [tokens, 1, 64]")
    if (slots.dtype != torch.long or slots.dim() != 1 or not slots.is_contiguous()
            or slots.numel() != tokens):
        raise RuntimeError("slots must be contiguous int64 [tokens]")
    for tensor in (m.query_rows, m.block_table_ids, m.block_table_offsets, m.context_lens):
        if tensor.dtype != torch.long or tensor.dim() != 1 or not tensor.is_contiguous():
            raise RuntimeError("metadata must be contiguous GPU int64 vectors")
    num_rows = m.query_rows.numel()
    if m.context_lens.numel() != num_rows or m.block_table_offsets.numel() != num_rows + 1:
        raise RuntimeError("metadata lengths must align")
    if num_rows == 0:
        return
    heads = q.shape[1]
    max_len = m.max_context_len or cache.num_slots
    need = int(lib.tvllm_paged_decode_workspace_size(
        num_rows, heads, cache.num_kv_heads, 128, max_len, cache.block_size))
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=device)
    check(lib.tvllm_paged_decode_qk_norm_rope(
        q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1), query_weight.data_ptr(),
        key_weight.data_ptr(), cos.data_ptr(), sin.data_ptr(), float(query_eps),
        float(key_eps), slots.data_ptr(), kc.data_ptr(), vc.data_ptr(), output.data_ptr(),
        output.stride(0), output.stride(1), m.query_rows.data_ptr(),
        m.block_table_ids.data_ptr(), m.block_table_offsets.data_ptr(),
        m.context_lens.data_ptr(), num_rows, heads, cache.num_kv_heads, 128,
        cache.num_slots, kc.stride(0), kc.stride(1), cache.block_size, max_len, float(scale),
        workspace.data_ptr() if need else None, need, dtype_code(q.dtype),
        *cache_format(cache), stream_of(device),
    ))


QKV_PARTS = 4  # slices of the split-K qkv projection the fused kernel sums


def paged_decode_qk_norm_rope_partials(
    parts: torch.Tensor,
    num_heads: int,
    query_weight: torch.Tensor,
    key_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    query_eps: float,
    key_eps: float,
    cache: PagedKVCache,
    layer_idx: int,
    metadata: SingleQueryMetadata,
    slots: torch.Tensor,
    output: torch.Tensor,
    *,
    scale: float,
    workspace: torch.Tensor | None = None,
) -> None:
    """``paged_decode_qk_norm_rope`` fed by the qkv projection's split-K
    partials (no reference counterpart): ``parts`` is the fp32 [4, tokens,
    (heads + 2 * kv_heads) * 128] result of a batched GEMM over four slices
    of the reduction, and each raw Q/K/V element is the in-order fp32 sum of
    its slices rounded once to the model dtype, summed inside the kernel's
    prologue (no launch of its own)."""
    lib = load_kernels()
    kc, vc = cache.key[layer_idx], cache.value[layer_idx]
    m = metadata
    device = require_gpu(parts, query_weight, key_weight, cos, sin, slots, kc, output,
                         m.query_rows, m.block_table_ids, m.block_table_offsets,
                         m.context_lens)
    width = (num_heads + 2 * cache.num_kv_heads) * 128
    if (parts.dtype != torch.float32 or parts.dim() != 3 or parts.shape[0] != QKV_PARTS
            or parts.shape[2] != width or parts.stride(2) != 1):
        raise RuntimeError(f"parts must be float32 [{QKV_PARTS}, tokens, {width}] with unit "
                           "last stride")
    dtype = query_weight.dtype
    if dtype not in (torch.float16, torch.bfloat16) or any(
            t.dtype != dtype for t in (key_weight, cos, sin, output)) \
            or (kc.dtype != dtype and not cache.fp8):
        raise RuntimeError("weights, RoPE tables, output and cache must share a half dtype")
    if vc.stride() != kc.stride():
        raise RuntimeError("K/V caches must share one layout")
    tokens = parts.shape[1]
    if output.shape != (tokens, num_heads, 128) or output.stride(-1) != 1:
        raise RuntimeError("output must be [tokens, heads, 128] with unit last stride")
    if (query_weight.shape != (128,) or key_weight.shape != (128,)
            or not query_weight.is_contiguous() or not key_weight.is_contiguous()):
        raise RuntimeError("norm weights must be contiguous [128]")
    for table in (cos, sin):
        if table.numel() != tokens * 64 or not table.is_contiguous():
            raise RuntimeError("RoPE tables must be contiguous [tokens, 1, 64]")
    if (slots.dtype != torch.long or slots.dim() != 1 or not slots.is_contiguous()
            or slots.numel() != tokens):
        raise RuntimeError("slots must be contiguous int64 [tokens]")
    for tensor in (m.query_rows, m.block_table_ids, m.block_table_offsets, m.context_lens):
        if tensor.dtype != torch.long or tensor.dim() != 1 or not tensor.is_contiguous():
            raise RuntimeError("metadata must be contiguous GPU int64 vectors")
    num_rows = m.query_rows.numel()
    if m.context_lens.numel() != num_rows or m.block_table_offsets.numel() != num_rows + 1:
        raise RuntimeError("metadata lengths must align")
    if num_rows == 0:
        return
    max_len = m.max_context_len or cache.num_slots
    need = int(lib.tvllm_paged_decode_workspace_size(
        num_rows, num_heads, cache.num_kv_heads, 128, max_len, cache.block_size))
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=device)
    check(lib.tvllm_paged_decode_qk_norm_rope_partials(
        parts.data_ptr(), parts.stride(0), parts.stride(1), query_weight.data_ptr(),
        key_weight.data_ptr(), cos.data_ptr(), sin.data_ptr(), float(query_eps),
        float(key_eps), slots.data_ptr(), kc.data_ptr(), vc.data_ptr(), output.data_ptr(),
        output.stride(0), output.stride(1), m.query_rows.data_ptr(),
        m.block_table_ids.data_ptr(), m.block_table_offsets.data_ptr(),
        m.context_lens.data_ptr(), num_rows, num_heads, cache.num_kv_heads, 128,
        cache.num_slots, kc.stride(0), kc.stride(1), cache.block_size, max_len, float(scale),
        workspace.data_ptr() if need else None, need, dtype_code(dtype),
        *cache_format(cache), stream_of(device),
    ))
