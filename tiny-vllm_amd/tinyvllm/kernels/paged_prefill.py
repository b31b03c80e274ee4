"""Chunked-prefill paged attention on MFMA tiles.

Replaces the reference's per-row gather + SDPA for query chunks with history
(tinyvllm/runtime/attention.py:102-151, 235-285) and its optional FlashInfer
wrapper (runtime/prefill.py:15-225).
"""
from __future__ import annotations

import threading
from contextlib import contextmanager

import torch

from tinyvllm.kernels._extension import (
    cache_format, check, dtype_code, load_kernels, require_gpu, stream_of,
)
from tinyvllm.paged_kv import PagedKVCache
from tinyvllm.runtime.contracts import MultiQueryMetadata


def paged_prefill_attention(
    q: torch.Tensor,
    cache: PagedKVCache,
    layer_idx: int,
    metadata: MultiQueryMetadata,
    output: torch.Tensor,
    *,
    scale: float,
) -> None:
    """Causal (lower-right) attention of each item's query chunk over its
    paged context; writes the items' rows of ``output`` in place."""
    lib = load_kernels()
    k, v = cache.key[layer_idx], cache.value[layer_idx]
    m = metadata
    device = require_gpu(q, k, v, output, m.query_offsets, m.block_table_ids,
                         m.block_table_offsets, m.context_lens)
    if k.stride() != v.stride():
        raise RuntimeError("K/V caches must share one layout")
    if q.dim() != 3 or output.shape != q.shape:
        raise RuntimeError("Q/output must be [tokens, heads, dim] tensors")
    if q.dtype not in (torch.float16, torch.bfloat16) or output.dtype != q.dtype \
            or (k.dtype != q.dtype and not cache.fp8):
        raise RuntimeError("Q/K/V/output must share a float16 or bfloat16 dtype")
    if q.stride(2) != 1 or output.stride(2) != 1:
        raise RuntimeError("Q/output rows must have unit last stride")
    for tensor in (m.query_offsets, m.block_table_ids, m.block_table_offsets,
                   m.context_lens):
        if tensor.dtype != torch.long or tensor.dim() != 1 or not tensor.is_contiguous():
            raise RuntimeError("metadata must be contiguous GPU int64 vectors")
    items = m.context_lens.numel()
    if m.query_offsets.numel() != items + 1 or m.block_table_offsets.numel() != items + 1:
        raise RuntimeError("metadata lengths must align")
    if items == 0 or m.max_query_len == 0:
        return
    cache_dtype, k_scale, v_scale = cache_format(cache)
    guard = _guard(device, int(lib.tvllm_paged_prefill_workspace_size(
        dtype_code(q.dtype), cache_dtype)))
    check(lib.tvllm_paged_prefill(
        q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(),
        output.data_ptr(), output.stride(0), output.stride(1),
        m.query_offsets.data_ptr(), m.block_table_ids.data_ptr(),
        m.block_table_offsets.data_ptr(), m.context_lens.data_ptr(),
        items, m.max_query_len, q.shape[1], cache.num_kv_heads, q.shape[2],
        cache.num_slots, k.stride(0), k.stride(1), cache.block_size, float(scale),
        None if guard is None else guard.data_ptr(), 0 if guard is None else guard.numel(),
        dtype_code(q.dtype), cache_dtype, k_scale, v_scale, stream_of(device),
    ))


_GUARDS: dict[tuple[torch.device, int], torch.Tensor] = {}
_OWNED = threading.local()

# Bytes of the largest fallback guard any call needs (two int32 words).
GUARD_BYTES = 8


@contextmanager
def fallback_guard(guard: torch.Tensor):
    """Calls inside this context use ``guard`` (zero-initialised uint8 of
    GUARD_BYTES on the calls' device) as their fallback guard. A captured
    graph owns its guard this way for the graph's lifetime, instead of one
    keyed by the capture stream's handle, which torch may hand to another
    stream once the capture stream is gone."""
    if guard.dtype != torch.uint8 or guard.numel() < GUARD_BYTES or not guard.is_cuda:
        raise ValueError(f"a fallback guard is a CUDA uint8 tensor of >= {GUARD_BYTES} bytes")
    previous = getattr(_OWNED, "guard", None)
    _OWNED.guard = guard
    try:
        yield guard
    finally:
        _OWNED.guard = previous


def _guard(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """The zero-initialised fallback guard: the one ``fallback_guard``
    installed, else that of ``device``'s current stream (calls on one stream
    are ordered, so they can share it; the kernels leave it zero)."""
    if nbytes == 0:
        return None
    owned = getattr(_OWNED, "guard", None)
    if owned is not None:
        if owned.device != device or owned.numel() < nbytes:
            raise RuntimeError("the installed fallback guard does not fit this call")
        return owned
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    guard = _GUARDS.get(key)
    if guard is None or guard.numel() < nbytes:
        guard = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        _GUARDS[key] = guard
    return guard
