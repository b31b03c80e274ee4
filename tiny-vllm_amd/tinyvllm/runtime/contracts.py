"""Device-side inputs of one model forward (reference: tinyvllm/runtime/contracts.py).

The attention backend protocol, the decode (single-query) metadata and the
chunked-prefill (multi-query) metadata are lowered once per step and shared
by every layer.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Protocol

import torch


class AttentionBackend(Protocol):
    """Per-step attention over flat, normalized and rotated Q/K/V
    (reference: runtime/contracts.py:11-24)."""

    def __call__(
        self,
        layer_idx: int,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        *,
        scale: float,
    ) -> torch.Tensor:
        """Return attention output shaped [tokens, query_heads, head_dim]."""
        ...


@dataclass(frozen=True, slots=True)
class SingleQueryMetadata:
    """Single-query tables; context_len=0 denotes internal graph padding
    (reference: runtime/contracts.py:27-34).

    ``max_context_len`` is an upper bound on every ``context_lens`` entry
    (the engine's max_model_len, or the batch maximum in eager mode); it only
    sizes the split-K decomposition. None means "bounded by the cache".

    Row r's table is ``block_table_ids[block_table_offsets[r]:][:ceil(
    context_lens[r] / block_size)]``: a CSR (offsets ascending, as the
    reference builds them) is one layout, the decode step's device-resident
    tables (one pitched row per request slot) another; the kernels read
    only ``block_table_offsets[r]``. In the pitched layout the offsets are
    not ascending and ``block_table_offsets[r + 1] - block_table_offsets[r]``
    is no row's table size: padding rows and the closing entry hold the
    table capacity (one past the end), as the reference pads them.
    """

    query_rows: torch.Tensor
    block_table_ids: torch.Tensor
    block_table_offsets: torch.Tensor
    context_lens: torch.Tensor
    max_context_len: int | None = None


@dataclass(frozen=True, slots=True)
class MultiQueryMetadata:
    """Chunked-prefill items that read paged history (no reference type: the
    reference gathers K/V per row in Python, runtime/contracts.py:108-116).

    ``query_offsets`` is a CSR over the flat token axis (items with a query
    length of 0 or 1 have empty ranges here); ``context_lens`` counts the
    cached tokens each item attends to, including its own chunk.
    """

    query_offsets: torch.Tensor
    block_table_ids: torch.Tensor
    block_table_offsets: torch.Tensor
    context_lens: torch.Tensor
    max_query_len: int


@dataclass(frozen=True, slots=True)
class PagedKVMetadata:
    """KV write slots plus the read metadata of each attention path."""

    slot_mapping: torch.Tensor
    decode: SingleQueryMetadata | None = None
    prefill: MultiQueryMetadata | None = None


@dataclass(frozen=True, slots=True)
class ModelInput:
    """Device inputs shared by all layers of one flat model forward."""

    input_ids: torch.Tensor
    positions: torch.Tensor
    sample_token_indices: torch.Tensor | None
    kv: PagedKVMetadata
