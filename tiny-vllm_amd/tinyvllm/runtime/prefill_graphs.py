"""hipGraph capture and replay of chunked-prefill and mixed steps (beyond
the reference, which runs every prefill step eagerly:
runtime/runner.py:197-246).

A prefill step of a few short prompts is host-bound: each layer issues about
a dozen launches whose host cost exceeds their GPU time (Qwen3-0.6B, one
64-token prompt: ~5.8 ms of host launches for ~2.5 ms of kernels), so the
time to first token is the host's. A graph per (token, item) bucket replays
the whole step - embedding, every layer (QK-norm/RoPE with the fused KV
write, paged prefill attention, GEMMs, norms), the LM head on the sampled
rows and the sampling kernel - from fixed device inputs that one H2D copy
fills.

Eligible steps: at most ``max_tokens`` tokens and ``max_items`` items, not
all of them single-token (those are decode steps, with graphs of their own).
Every item, single-token ones included, goes through the paged prefill
kernel (a one-row query is a valid chunk); single-token items are allowed
only up to ``DECODE_CONTEXT_BOUND`` context tokens, beyond which the split-K
decode kernel of the eager path reads their context faster. Input ids may
name the previous step's sampled rows (``input_token_sources``), resolved on
the device inside the graph. The bucket's padding tokens write slot -1 and
belong to no item; its padding items have empty queries; padding sample rows
point at token 0 and are dropped. Other steps run eagerly.

Upload layout (bytes, T = max tokens, I = max items, P = table capacity):
  float32 [I] temperature | [I] top_p |
  int64 [T] tokens | [T] token sources | [T] positions | [T] slots |
  [I + 1] query offsets |
  [I + 1] table offsets | [I] context lengths | [I] sample rows |
  [I] top_k | [I] seeds | [I] counters | [P] block ids (items' tables packed)
Only the prefix up to the last used block id is copied.
"""
from __future__ import annotations

import numpy as np
import torch

from tinyvllm._validation import _check_positive_int
from tinyvllm.batch import PreparedBatch
from tinyvllm.kernels.paged_prefill import GUARD_BYTES, fallback_guard
from tinyvllm.kernels.sampling import resolve_tokens, sample
from tinyvllm.paged_kv import PagedKVCache
from tinyvllm.runtime.attention import HipAttention
from tinyvllm.runtime.contracts import ModelInput, MultiQueryMetadata, PagedKVMetadata

TOKEN_BUCKETS = (32, 64, 128, 192, 256, 384, 512, 768, 1024, 1536, 2048)
ITEM_BUCKETS = (1, 2, 4, 8, 16)
DECODE_CONTEXT_BOUND = 1024

_INT_FIELDS = ("tokens", "sources", "positions", "slots", "q_offsets", "t_offsets", "lengths",
               "sample_rows", "top_k", "seeds", "counters", "blocks")


def _signed64(value: int) -> int:
    return value - (1 << 64) if value >= (1 << 63) else value


class PrefillInputs:
    """Runner-owned fixed storage; ``view`` results stay valid forever and
    their contents change at every ``prepare``."""

    def __init__(self, *, max_tokens: int, max_items: int, max_model_len: int,
                 block_size: int, device: torch.device | str) -> None:
        for name, value in (("max_tokens", max_tokens), ("max_items", max_items),
                            ("max_model_len", max_model_len), ("block_size", block_size)):
            _check_positive_int(name, value)
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("prefill inputs require a GPU device")
        t, n = max_tokens, max_items
        self.max_tokens, self.max_items = t, n
        self.block_size = block_size
        self.max_model_len = max_model_len
        pitch = -(-max_model_len // block_size)
        self.table_capacity = n * pitch
        sizes = {"tokens": t, "sources": t, "positions": t, "slots": t, "q_offsets": n + 1,
                 "t_offsets": n + 1, "lengths": n, "sample_rows": n, "top_k": n,
                 "seeds": n, "counters": n, "blocks": self.table_capacity}
        self.float_bytes = 8 * n
        total = self.float_bytes + 8 * sum(sizes.values())
        self._blocks_offset = total - 8 * self.table_capacity
        self.host = torch.zeros(total, dtype=torch.uint8, pin_memory=True)
        self.device_data = torch.zeros(total, dtype=torch.uint8, device=self.device)
        self.stream = torch.cuda.current_stream(self.device)
        self.upload_done = torch.cuda.Event()
        self.uploaded = False

        def carve(buffer: torch.Tensor):
            floats = buffer[:self.float_bytes].view(torch.float32)
            out = {"temperature": floats[:n], "top_p": floats[n:]}
            ints = buffer[self.float_bytes:].view(torch.int64)
            start = 0
            for name in _INT_FIELDS:
                out[name] = ints[start:start + sizes[name]]
                start += sizes[name]
            return out

        self.h = {k: v.numpy() for k, v in carve(self.host).items()}
        self.d = carve(self.device_data)

    @staticmethod
    def bucket(value: int, buckets: tuple[int, ...]) -> int | None:
        return next((b for b in buckets if value <= b), None)

    def buckets_for(self, batch: PreparedBatch) -> tuple[int, int] | None:
        """(token bucket, item bucket) of an eligible batch, else None."""
        if batch.num_items == 0 or max(batch.query_lens) < 2:
            return None
        if min(batch.query_lens) < 2 and any(
                n == 1 and c > DECODE_CONTEXT_BOUND
                for n, c in zip(batch.query_lens, batch.context_lens_after)):
            return None
        tokens = self.bucket(batch.num_query_tokens,
                             tuple(b for b in TOKEN_BUCKETS if b <= self.max_tokens))
        items = self.bucket(batch.num_items,
                            tuple(b for b in ITEM_BUCKETS if b <= self.max_items))
        if tokens is None or items is None or len(batch.kv_block_table_ids) > \
                self.table_capacity:
            return None
        return tokens, items

    def prepare(self, batch: PreparedBatch, counters) -> tuple[int, int] | None:
        """Upload an eligible validated batch and return its buckets."""
        buckets = self.buckets_for(batch)
        if buckets is None:
            return None
        if torch.cuda.current_stream(self.device) != self.stream:
            raise RuntimeError("the runner must stay on its creation stream")
        if self.uploaded:  # stream order cannot protect the host buffer
            self.upload_done.synchronize()
        tb, ib = buckets
        count, items, samples = batch.num_query_tokens, batch.num_items, batch.num_samples
        h = self.h
        h["tokens"][:count] = batch.input_ids
        h["tokens"][count:tb] = 0
        sources = batch.input_token_sources
        h["sources"][:count] = -1 if sources is None else sources
        h["sources"][count:tb] = -1
        h["positions"][:count] = batch.positions
        h["positions"][count:tb] = 0
        h["slots"][:count] = batch.kv_slot_mapping
        h["slots"][count:tb] = -1
        h["q_offsets"][:items + 1] = batch.q_offsets
        h["q_offsets"][items + 1:ib + 1] = count
        offsets = np.asarray(batch.kv_block_table_offsets, dtype=np.int64)
        h["t_offsets"][:items + 1] = offsets
        h["t_offsets"][items + 1:ib + 1] = offsets[-1]
        h["lengths"][:items] = batch.context_lens_after
        h["lengths"][items:ib] = 0
        h["sample_rows"][:samples] = batch.sample_token_indices
        h["sample_rows"][samples:ib] = 0
        params = batch.sampling_params
        h["temperature"][:samples] = [p.temperature for p in params]
        h["top_p"][:samples] = [p.top_p for p in params]
        h["top_k"][:samples] = [p.top_k for p in params]
        h["seeds"][:samples] = [_signed64(p.seed) for p in params]
        h["counters"][:samples] = counters
        h["temperature"][samples:ib] = 0.0
        h["top_p"][samples:ib] = 1.0
        h["top_k"][samples:ib] = 0
        h["seeds"][samples:ib] = 0
        h["counters"][samples:ib] = 0
        ids = np.asarray(batch.kv_block_table_ids, dtype=np.int64)
        h["blocks"][:len(ids)] = ids
        size = self._blocks_offset + 8 * len(ids)
        self.device_data[:size].copy_(self.host[:size], non_blocking=True)
        self.upload_done.record(self.stream)
        self.uploaded = True
        return buckets

    def sources(self, tokens: int) -> torch.Tensor:
        return self.d["sources"][:tokens]

    def view(self, tokens: int, items: int) -> ModelInput:
        d = self.d
        return ModelInput(
            input_ids=d["tokens"][:tokens],
            positions=d["positions"][:tokens],
            sample_token_indices=d["sample_rows"][:items],
            kv=PagedKVMetadata(
                slot_mapping=d["slots"][:tokens],
                prefill=MultiQueryMetadata(
                    query_offsets=d["q_offsets"][:items + 1],
                    block_table_ids=d["blocks"],
                    block_table_offsets=d["t_offsets"][:items + 1],
                    context_lens=d["lengths"][:items],
                    max_query_len=tokens,
                ),
            ),
        )

    def sampling_views(self, items: int) -> tuple[torch.Tensor, ...]:
        """(temperature, top_k, top_p, seeds, counters) device views."""
        d = self.d
        return (d["temperature"][:items], d["top_k"][:items], d["top_p"][:items],
                d["seeds"][:items], d["counters"][:items])


class PrefillGraphs:
    """Startup-only capture of one graph per (token, item) bucket; the
    runner keeps model, cache and inputs alive."""

    def __init__(self, stream: torch.cuda.Stream) -> None:
        self.stream = stream
        self.entries: dict[tuple[int, int], tuple[torch.cuda.CUDAGraph, torch.Tensor,
                                                  torch.Tensor]] = {}
        self.pool = None
        # The prefill kernels' fallback guard of every captured graph: owned
        # here, so it lives exactly as long as the graphs that point at it.
        self.guard: torch.Tensor | None = None

    @torch.inference_mode()
    def capture(self, model: torch.nn.Module, inputs: PrefillInputs,
                cache: PagedKVCache, previous: torch.Tensor) -> None:
        """``previous``: the runner's buffer of the last step's sampled ids,
        which ``input_token_sources`` index."""
        # Dummy contents: items of equal length over block 0, no KV writes
        # (slot -1), greedy samples of each item's last token.
        d = inputs.d
        d["tokens"].zero_()
        d["sources"].fill_(-1)
        d["positions"].zero_()
        d["slots"].fill_(-1)
        d["blocks"].zero_()
        d["temperature"].zero_()
        d["top_p"].fill_(1.0)
        d["top_k"].zero_()
        d["seeds"].zero_()
        d["counters"].zero_()
        model.model.rotary_emb(d["positions"][:1], next(model.parameters()).dtype)
        side = torch.cuda.Stream(device=inputs.device)
        side.wait_stream(self.stream)
        self.pool = torch.cuda.graph_pool_handle()
        self.guard = torch.zeros(GUARD_BYTES, dtype=torch.uint8, device=inputs.device)
        try:
            with torch.cuda.stream(side), fallback_guard(self.guard):
                below = 0  # the previous token bucket
                for tokens in TOKEN_BUCKETS:
                    if tokens > inputs.max_tokens:
                        break
                    for items in ITEM_BUCKETS:
                        # Skip buckets no batch reaches (more than ``below``
                        # tokens need that many items of max_model_len).
                        if items > inputs.max_items or items > tokens or \
                                below >= items * inputs.max_model_len:
                            continue
                        self._capture_one(model, inputs, cache, previous, tokens, items,
                                          side)
                    below = tokens
        finally:
            side.synchronize()
            torch.cuda.current_stream(inputs.device).synchronize()

    def _capture_one(self, model, inputs, cache, previous, tokens, items, side) -> None:
        d = inputs.d
        per = min(tokens // items, inputs.max_model_len)  # the rest is padding
        blocks_per = -(-per // inputs.block_size)
        d["q_offsets"][:items + 1].copy_(torch.arange(items + 1, device=inputs.device) * per)
        d["t_offsets"][:items + 1].copy_(
            torch.arange(items + 1, device=inputs.device) * blocks_per)
        d["lengths"][:items].fill_(per)
        d["sample_rows"][:items].copy_(
            torch.arange(1, items + 1, device=inputs.device) * per - 1)
        model_input = inputs.view(tokens, items)
        params = inputs.sampling_views(items)
        sources = inputs.sources(tokens)

        def step():
            resolve_tokens(model_input.input_ids, sources, previous)
            attention = HipAttention(model_input, cache)
            hidden = model(model_input.input_ids, model_input.positions, attention=attention)
            logits = model.compute_logits(hidden, model_input.sample_token_indices)
            return logits, sample(logits, *params)

        for _ in range(2):
            step()
        side.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self.pool, stream=side):
            logits, out = step()
        self.entries[(tokens, items)] = (graph, logits, out)

    def replay(self, tokens: int, items: int) -> tuple[torch.Tensor, torch.Tensor] | None:
        entry = self.entries.get((tokens, items))
        if entry is None:
            return None
        graph, logits, out = entry
        graph.replay()
        return logits, out

    def close(self) -> None:
        self.stream.synchronize()
        self.entries.clear()
        self.pool = None
        self.guard = None
