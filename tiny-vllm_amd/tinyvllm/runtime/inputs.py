"""Fixed-address device inputs of the graph-replayed decode step
(reference: tinyvllm/runtime/inputs.py:14-137).

All per-step decode metadata - token ids, positions, write slots, block-table
CSR, context lengths and the sampling parameters - is packed into one pinned
host buffer and moved with a single asynchronous H2D copy into one device
buffer whose sub-views never move, so captured graphs can replay against them.

Layout (bytes, N = capacity rows, P = N * pages_per_row):
  float32 [N] temperature | float32 [N] top_p |
  int64 [N] tokens | [N] positions | [N] slots | [N + 1] table offsets |
  [N] context lengths | [N] top_k | [N] seeds | [N] sample counters |
  [N] token sources | [P] block ids
A token source j >= 0 replaces the row's token, on the device, by row j of
the previous step's sampled tokens (-1: keep the uploaded id).
Rows past the live count are padding: slot -1 (no KV write), length 0 (zero
attention output), greedy sampling.
"""
from __future__ import annotations

import torch

from tinyvllm._validation import _check_positive_int
from tinyvllm.batch import PreparedBatch
from tinyvllm.runtime.contracts import ModelInput, PagedKVMetadata, SingleQueryMetadata

_INT_FIELDS = ("tokens", "positions", "slots", "offsets", "lengths", "top_k", "seeds",
               "counters", "sources", "blocks")


class DecodeInputs:
    """Runner-owned storage; views returned by ``view`` stay valid forever,
    their contents change at every ``prepare``."""

    @staticmethod
    def device_bytes(*, max_num_seqs: int, max_model_len: int, block_size: int) -> int:
        pages = -(-max_model_len // block_size)
        return 4 * 2 * max_num_seqs + 8 * (9 * max_num_seqs + 1 + max_num_seqs * pages)

    def __init__(self, *, max_num_seqs: int, max_model_len: int, block_size: int,
                 device: torch.device | str) -> None:
        for name, value in (("max_num_seqs", max_num_seqs),
                            ("max_model_len", max_model_len), ("block_size", block_size)):
            _check_positive_int(name, value)
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("decode inputs require a GPU device")
        n = max_num_seqs
        self.capacity = n
        self.max_model_len = max_model_len
        self.block_size = block_size
        self.table_capacity = n * -(-max_model_len // block_size)
        sizes = {"tokens": n, "positions": n, "slots": n, "offsets": n + 1, "lengths": n,
                 "top_k": n, "seeds": n, "counters": n, "sources": n,
                 "blocks": self.table_capacity}
        self.float_bytes = 8 * n
        total = self.float_bytes + 8 * sum(sizes.values())
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
        self._blocks_offset = self.float_bytes + 8 * (9 * n + 1)
        self.rows = torch.arange(n, dtype=torch.long, device=self.device)
        # Graph capture and padding defaults: every row is padding.
        self._reset_padding(0, 0)
        self.device_data.copy_(self.host)

    def _reset_padding(self, count: int, table_size: int) -> None:
        h = self.h
        h["tokens"][count:] = 0
        h["positions"][count:] = 0
        h["slots"][count:] = -1
        h["offsets"][count + 1:] = table_size
        h["lengths"][count:] = 0
        h["temperature"][count:] = 0.0
        h["top_p"][count:] = 1.0
        h["top_k"][count:] = 0
        h["seeds"][count:] = 0
        h["counters"][count:] = 0
        h["sources"][count:] = -1

    def prepare(self, batch: PreparedBatch, counters) -> ModelInput | None:
        """Upload a validated all-decode batch; None if it is not one."""
        if torch.cuda.current_stream(self.device) != self.stream:
            raise RuntimeError("the runner must stay on its creation stream")
        count = batch.num_items
        if not 1 <= count <= self.capacity:
            raise ValueError("batch exceeds decode input request capacity")
        if batch.num_query_tokens != count or batch.num_samples != count:
            return None
        table_size = len(batch.kv_block_table_ids)
        if table_size > self.table_capacity:
            raise ValueError("batch exceeds decode input block-table capacity")
        # Stream order cannot protect the host buffer from an early CPU write.
        if self.uploaded:
            self.upload_done.synchronize()
        h = self.h
        self._reset_padding(count, table_size)
        h["tokens"][:count] = batch.input_ids
        h["positions"][:count] = batch.positions
        h["slots"][:count] = batch.kv_slot_mapping
        h["offsets"][:count + 1] = batch.kv_block_table_offsets
        h["lengths"][:count] = batch.context_lens_after
        h["blocks"][:table_size] = batch.kv_block_table_ids
        params = batch.sampling_params
        first = params[0]
        if all(p == first for p in params):  # one policy for the whole batch
            rows = [first]
        else:
            rows = params
        h["temperature"][:count] = [p.temperature for p in rows]
        h["top_p"][:count] = [p.top_p for p in rows]
        h["top_k"][:count] = [p.top_k for p in rows]
        h["seeds"][:count] = [p.seed - (1 << 64) if p.seed >= (1 << 63) else p.seed
                              for p in rows]
        h["counters"][:count] = counters
        sources = batch.input_token_sources
        h["sources"][:count] = -1 if sources is None else sources
        size = self._blocks_offset + 8 * table_size
        self.device_data[:size].copy_(self.host[:size], non_blocking=True)
        self.upload_done.record(self.stream)
        self.uploaded = True
        return self.view(count, table_size, max(batch.context_lens_after))

    def view(self, count: int, table_size: int | None = None,
             max_context_len: int | None = None) -> ModelInput:
        """Borrow fixed storage; graph capture uses the full table capacity.
        ``max_context_len`` bounds every row's context (default: the
        engine's max_model_len); it only sizes the decode split-K plan."""
        d = self.d
        table = d["blocks"] if table_size is None else d["blocks"][:table_size]
        rows = self.rows[:count]
        return ModelInput(
            input_ids=d["tokens"][:count],
            positions=d["positions"][:count],
            sample_token_indices=rows,
            kv=PagedKVMetadata(
                slot_mapping=d["slots"][:count],
                decode=SingleQueryMetadata(
                    query_rows=rows,
                    block_table_ids=table,
                    block_table_offsets=d["offsets"][:count + 1],
                    context_lens=d["lengths"][:count],
                    max_context_len=max_context_len or self.max_model_len,
                ),
            ),
        )

    def sampling_views(self, count: int) -> tuple[torch.Tensor, ...]:
        """(temperature, top_k, top_p, seeds, counters) device views."""
        d = self.d
        return (d["temperature"][:count], d["top_k"][:count], d["top_p"][:count],
                d["seeds"][:count], d["counters"][:count])
