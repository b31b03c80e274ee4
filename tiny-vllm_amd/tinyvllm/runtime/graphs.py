"""hipGraph capture and replay of the whole decode step
(reference: tinyvllm/runtime/graphs.py:12-139).

One graph per batch-size bucket holds the block-table update and token
resolution -> embedding -> all layers (fused
QK-norm/RoPE/KV-write, split-K paged decode, GEMMs, norms) -> LM head ->
sampling kernel, reading only the fixed ``DecodeInputs`` views. A replay is
a single host call, so the per-step host cost no longer scales with
layers x kernels. The reference caps capture at 16 rows and runs larger
batches eagerly; here buckets cover every size up to ``max_num_seqs``.
All graphs share one memory pool (they are replayed one at a time on the
runner's stream, and outputs are consumed before the next replay).
"""
from __future__ import annotations

import torch

from tinyvllm.kernels.paged_decode import decode_split_plan
from tinyvllm.kernels.sampling import resolve_tokens, sample
from tinyvllm.paged_kv import PagedKVCache
from tinyvllm.runtime.attention import HipAttention
from tinyvllm.runtime.inputs import DecodeInputs


def context_buckets(max_model_len: int) -> tuple[int, ...]:
    """Context bounds a bucket's graphs are captured for: the decode kernel's
    split-K plan depends on the bound, and a graph baked for max_model_len
    over-splits short contexts (few rows at 64 tokens would run 64 splits
    and a merge launch per layer)."""
    return tuple(sorted({b for b in (256, 512, 1024, 4096) if b < max_model_len} | {max_model_len}))


def bucket_sizes(limit: int) -> tuple[int, ...]:
    """1, 2, 4, 8, then multiples of 8 (multiples of 16 past 128) up to limit."""
    sizes = [s for s in (1, 2, 4) if s < limit]
    size = 8
    while size < limit:
        sizes.append(size)
        size += 8 if size < 128 else 16
    sizes.append(limit)
    return tuple(sorted(set(sizes)))


class DecodeGraphs:
    """Startup-only capture; the runner keeps model, cache and inputs alive."""

    def __init__(self, stream: torch.cuda.Stream) -> None:
        self.stream = stream
        # size -> [(context bound, graph, logits, tokens)] ascending by bound
        self.entries: dict[int, list[tuple[int, torch.cuda.CUDAGraph, torch.Tensor,
                                           torch.Tensor]]] = {}
        self.tokens: torch.Tensor | None = None
        self.pool = None

    @torch.inference_mode()
    def capture(self, model: torch.nn.Module, inputs: DecodeInputs, cache: PagedKVCache,
                workspace: torch.Tensor | None, *,
                sizes: tuple[int, ...] | None = None,
                tokens: torch.Tensor | None = None) -> None:
        """Capture one graph per bucket size (default: ``bucket_sizes`` up to
        the input capacity). ``tokens`` (int64, >= capacity rows) receives
        every replay's sampled ids; a replay first takes its input ids from
        the previous step's rows there wherever the uploaded token sources
        say so."""
        limit = min(inputs.capacity, cache.num_blocks)
        sizes = bucket_sizes(limit) if sizes is None else tuple(
            sorted({min(int(x), limit) for x in sizes}))
        # Dummy rows: one distinct block each, context 1, greedy.
        d = inputs.d
        n = limit
        d["tokens"][:n].zero_()
        d["positions"][:n].zero_()
        d["slots"][:n].copy_(inputs.rows[:n] * cache.block_size)
        d["offsets"][:n + 1].copy_(torch.arange(n + 1, device=inputs.device))
        d["lengths"][:n].fill_(1)
        inputs.table[:n].copy_(inputs.rows[:n])
        d["updates"][:1].zero_()
        if tokens is None:
            tokens = torch.zeros(inputs.capacity, dtype=torch.long, device=inputs.device)
        if tokens.dtype != torch.long or tokens.numel() < inputs.capacity:
            raise ValueError("graph token buffer must hold capacity int64 rows")
        self.tokens = tokens
        # Build dtype-cast RoPE tables before capture.
        model.model.rotary_emb(inputs.d["positions"][:1], next(model.parameters()).dtype)

        side = torch.cuda.Stream(device=inputs.device)
        side.wait_stream(self.stream)
        self.pool = torch.cuda.graph_pool_handle()
        try:
            with torch.cuda.stream(side):
                for size in reversed(sizes):
                    for bound in self._bounds(model, inputs, cache, size):
                        self._capture_one(model, inputs, cache, workspace, size, bound, side)
        finally:
            side.synchronize()
            # Leave the padding state behind for the first real batch.
            d["slots"].fill_(-1)
            d["lengths"].zero_()
            inputs.forget_tables()  # the capture overwrote table rows
            torch.cuda.current_stream(inputs.device).synchronize()
        self.entries = dict(sorted(self.entries.items()))

    @staticmethod
    def _bounds(model, inputs: DecodeInputs, cache: PagedKVCache, size: int) -> list[int]:
        """Context bounds needing their own graph at this size: within a run
        of bounds with the same split plan, the largest serves them all."""
        cfg = model.config
        bounds: list[int] = []
        last = None
        for bound in reversed(context_buckets(inputs.max_model_len)):
            plan = decode_split_plan(size, cfg.num_attention_heads, cache.num_kv_heads,
                                     cache.head_dim, bound, cache.block_size)
            if plan != last:
                bounds.append(bound)
                last = plan
        return sorted(bounds)

    def _capture_one(self, model, inputs, cache, workspace, size, bound, side) -> None:
        model_input = inputs.view(size, max_context_len=bound)
        params = inputs.sampling_views(size)
        out = self.tokens[:size]
        sources = inputs.d["sources"][:size]

        def step():
            inputs.apply_table_updates()
            resolve_tokens(model_input.input_ids, sources, self.tokens)
            attention = HipAttention(model_input, cache, decode_workspace=workspace)
            hidden = model(model_input.input_ids, model_input.positions, attention=attention)
            logits = model.compute_logits(hidden)
            sample(logits, *params, out=out)
            return logits

        for _ in range(2):
            step()
        side.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self.pool, stream=side):
            logits = step()
        self.entries.setdefault(size, []).append((bound, graph, logits, out))
        self.entries[size].sort(key=lambda e: e[0])

    def bucket(self, count: int) -> int | None:
        for size in self.entries:
            if count <= size:
                return size
        return None

    def replay(self, count: int, max_context: int | None = None
               ) -> tuple[torch.Tensor, torch.Tensor] | None:
        """Replay the smallest graph that fits ``count`` rows whose contexts
        are at most ``max_context`` (None: the largest bound);
        (logits[:count], tokens[:count])."""
        size = self.bucket(count)
        if size is None:
            return None
        entries = self.entries[size]
        chosen = entries[-1] if max_context is None else next(
            (e for e in entries if max_context <= e[0]), None)
        if chosen is None:
            return None
        _, graph, logits, tokens = chosen
        graph.replay()
        return logits[:count], tokens[:count]

    def close(self) -> None:
        self.stream.synchronize()
        self.entries.clear()
        self.pool = None
