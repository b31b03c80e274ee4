"""Fixed-address device inputs of the graph-replayed decode step
(reference: tinyvllm/runtime/inputs.py:14-137).

All per-step decode metadata - token ids, positions, write slots, context
lengths, the sampling parameters and the block-table changes - is packed
into one pinned host buffer and moved with a single asynchronous H2D copy
into one device buffer whose sub-views never move, so captured graphs can
replay against them.

Block tables stay on the device: one row of ``pitch`` ids per request slot
(``PreparedBatch.request_slots``), kept across steps. A step uploads only
the entries a row lacks - for a request already decoding in that slot with
the same table epoch, the pages appended since its last upload (usually
none, at most one per row) - as (index, id) pairs that
``tvllm_apply_table_updates`` writes at the head of the step. The reference
re-packs and uploads every table each step (inputs.py:70-117).

Upload layout (bytes, N = capacity rows, P = N * pitch):
  float32 [N] temperature | float32 [N] top_p |
  int64 [N] tokens | [N] positions | [N] slots | [N + 1] table offsets |
  [N] context lengths | [N] top_k | [N] seeds | [N] sample counters |
  [N] token sources | [1 + 2P] table updates (count, then index/id pairs)
Device only: int64 [P] block tables. Row r's table starts at offsets[r]
(its slot times the pitch).
A token source j >= 0 replaces the row's token, on the device, by row j of
the previous step's sampled tokens (-1: keep the uploaded id).
Rows past the live count are padding: slot -1 (no KV write), length 0 (zero
attention output), greedy sampling.
"""
from __future__ import annotations

import time

import numpy as np
import torch

from tinyvllm._validation import _check_positive_int
from tinyvllm.batch import PreparedBatch
from tinyvllm.kernels.kv_store import apply_table_updates
from tinyvllm.runtime.contracts import ModelInput, PagedKVMetadata, SingleQueryMetadata

_INT_FIELDS = ("tokens", "positions", "slots", "offsets", "lengths", "top_k", "seeds",
               "counters", "sources", "updates")


class DecodeInputs:
    """Runner-owned storage; views returned by ``view`` stay valid forever,
    their contents change at every ``prepare``."""

    @staticmethod
    def device_bytes(*, max_num_seqs: int, max_model_len: int, block_size: int) -> int:
        table = max_num_seqs * -(-max_model_len // block_size)
        return 4 * 2 * max_num_seqs + 8 * (9 * max_num_seqs + 1 + 1 + 2 * table) + 8 * table

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
        self.pitch = -(-max_model_len // block_size)
        self.table_capacity = n * self.pitch
        sizes = {"tokens": n, "positions": n, "slots": n, "offsets": n + 1, "lengths": n,
                 "top_k": n, "seeds": n, "counters": n, "sources": n,
                 "updates": 1 + 2 * self.table_capacity}
        self.float_bytes = 8 * n
        total = self.float_bytes + 8 * sum(sizes.values())
        self.host = torch.zeros(total, dtype=torch.uint8, pin_memory=True)
        self.device_data = torch.zeros(total, dtype=torch.uint8, device=self.device)
        self.table = torch.zeros(self.table_capacity, dtype=torch.long, device=self.device)
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
        self.d["blocks"] = self.table
        self._updates_offset = self.float_bytes + 8 * (9 * n + 1)
        # What each slot's device row holds: owner request, table epoch, pages.
        self._row_request = np.full(n, -1, dtype=np.int64)
        self._row_epoch = np.full(n, -1, dtype=np.int64)
        self._row_pages = np.zeros(n, dtype=np.int64)
        # Per-step cost counters (host packing time, bytes uploaded, table
        # entries uploaded) for measurement.
        self.stats = {"steps": 0, "host_ns": 0, "bytes": 0, "table_entries": 0}
        self.rows = torch.arange(n, dtype=torch.long, device=self.device)
        # Graph capture and padding defaults: every row is padding.
        self._reset_padding(0)
        self.h["updates"][0] = 0
        self.device_data.copy_(self.host)

    def forget_tables(self) -> None:
        """The device rows no longer match the host record (their contents
        were overwritten, e.g. by graph capture): upload whole tables next."""
        self._row_request.fill(-1)
        self._row_epoch.fill(-1)
        self._row_pages.fill(0)

    def _reset_padding(self, count: int) -> None:
        h = self.h
        h["tokens"][count:] = 0
        h["positions"][count:] = 0
        h["slots"][count:] = -1
        # One past the tables' end, as the reference pads (inputs.py:94-98):
        # never a row start, so a stray read of a padded row's table faults
        # loudly in a bounds check instead of aliasing request slot 0.
        h["offsets"][count:] = self.table_capacity
        h["lengths"][count:] = 0
        h["temperature"][count:] = 0.0
        h["top_p"][count:] = 1.0
        h["top_k"][count:] = 0
        h["seeds"][count:] = 0
        h["counters"][count:] = 0
        h["sources"][count:] = -1

    def _table_rows(self, batch: PreparedBatch, count: int) -> np.ndarray:
        """Each item's device table row; also uploads what those rows lack
        (writes the update list into the host buffer)."""
        offsets = np.asarray(batch.kv_block_table_offsets, dtype=np.int64)
        pages = np.diff(offsets)
        if len(pages) != count or (pages > self.pitch).any():
            raise ValueError("batch exceeds decode input block-table capacity")
        ids = np.asarray(batch.kv_block_table_ids, dtype=np.int64)
        rid = np.asarray(batch.request_ids, dtype=np.int64)
        if batch.request_slots is not None and batch.kv_table_epochs is not None:
            rows = np.asarray(batch.request_slots, dtype=np.int64)
            if len(rows) != count or rows.min() < 0 or rows.max() >= self.capacity \
                    or len(np.unique(rows)) != count:
                raise ValueError("request slots must be distinct and below capacity")
            epochs = np.asarray(batch.kv_table_epochs, dtype=np.int64)
            kept = ((self._row_request[rows] == rid) & (self._row_epoch[rows] == epochs)
                    & (self._row_pages[rows] <= pages))
            first = np.where(kept, self._row_pages[rows], 0)
        else:  # no slot/epoch record: rows in batch order, whole tables
            rows = np.arange(count, dtype=np.int64)
            epochs = np.full(count, -1, dtype=np.int64)
            first = np.zeros(count, dtype=np.int64)
        fresh = pages - first
        total = int(fresh.sum())
        upd = self.h["updates"]
        upd[0] = total
        if total:
            item = np.repeat(np.arange(count), fresh)
            k = np.arange(total) - np.repeat(np.cumsum(fresh) - fresh, fresh)
            page = first[item] + k
            upd[1:1 + 2 * total:2] = rows[item] * self.pitch + page
            upd[2:2 + 2 * total:2] = ids[offsets[item] + page]
        self._row_request[rows] = rid
        self._row_epoch[rows] = epochs
        self._row_pages[rows] = pages
        if batch.kv_table_epochs is None:  # nothing to compare against next time
            self._row_request[rows] = -1
        self.stats["table_entries"] += total
        return rows

    def prepare(self, batch: PreparedBatch, counters) -> ModelInput | None:
        """Upload a validated all-decode batch; None if it is not one."""
        if torch.cuda.current_stream(self.device) != self.stream:
            raise RuntimeError("the runner must stay on its creation stream")
        count = batch.num_items
        if not 1 <= count <= self.capacity:
            raise ValueError("batch exceeds decode input request capacity")
        if batch.num_query_tokens != count or batch.num_samples != count:
            return None
        started = time.perf_counter_ns()
        # Stream order cannot protect the host buffer from an early CPU write.
        if self.uploaded:
            self.upload_done.synchronize()
        h = self.h
        self._reset_padding(count)
        rows = self._table_rows(batch, count)
        h["tokens"][:count] = batch.input_ids
        h["positions"][:count] = batch.positions
        h["slots"][:count] = batch.kv_slot_mapping
        h["offsets"][:count] = rows * self.pitch
        h["lengths"][:count] = batch.context_lens_after
        params = batch.sampling_params
        first = params[0]
        if all(p == first for p in params):  # one policy for the whole batch
            prow = [first]
        else:
            prow = params
        h["temperature"][:count] = [p.temperature for p in prow]
        h["top_p"][:count] = [p.top_p for p in prow]
        h["top_k"][:count] = [p.top_k for p in prow]
        h["seeds"][:count] = [p.seed - (1 << 64) if p.seed >= (1 << 63) else p.seed
                              for p in prow]
        h["counters"][:count] = counters
        sources = batch.input_token_sources
        h["sources"][:count] = -1 if sources is None else sources
        size = self._updates_offset + 8 * (1 + 2 * int(h["updates"][0]))
        self.device_data[:size].copy_(self.host[:size], non_blocking=True)
        self.upload_done.record(self.stream)
        self.uploaded = True
        self.stats["steps"] += 1
        self.stats["bytes"] += size
        self.stats["host_ns"] += time.perf_counter_ns() - started
        return self.view(count, max_context_len=max(batch.context_lens_after))

    def apply_table_updates(self) -> None:
        """Write the uploaded table changes into the device tables (the first
        node of every decode step; reads the count on the device)."""
        apply_table_updates(self.table, self.d["updates"])

    def view(self, count: int, table_size: int | None = None,
             max_context_len: int | None = None) -> ModelInput:
        """Borrow fixed storage. ``max_context_len`` bounds every row's context
        (default: the engine's max_model_len); it only sizes the decode
        split-K plan. (``table_size`` is accepted for older callers; rows
        read their tables through the offsets.)"""
        d = self.d
        rows = self.rows[:count]
        return ModelInput(
            input_ids=d["tokens"][:count],
            positions=d["positions"][:count],
            sample_token_indices=rows,
            kv=PagedKVMetadata(
                slot_mapping=d["slots"][:count],
                decode=SingleQueryMetadata(
                    query_rows=rows,
                    block_table_ids=self.table,
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
