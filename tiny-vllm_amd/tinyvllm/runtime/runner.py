"""Model runner: validate a CPU batch, lower it, run the model, sample
(reference: tinyvllm/runtime/runner.py:15-262).

Decode-only batches go through ``DecodeInputs`` (one H2D copy) and a
replayed hipGraph that ends in the sampling kernel. Prefill and mixed
batches are lowered to ``ModelInput`` and run eagerly on the same kernels.
"""
from __future__ import annotations

import numpy as np
import torch
from torch import nn

from tinyvllm._validation import _check_positive_int
from tinyvllm.batch import PreparedBatch
from tinyvllm.kernels.paged_decode import decode_workspace_bytes
from tinyvllm.kernels.sampling import resolve_tokens, sample
from tinyvllm.paged_kv import PagedKVCache, resolve_layout
from tinyvllm.runtime.attention import HipAttention, SDPAAttention, check_backend
from tinyvllm.runtime.contracts import (
    ModelInput, MultiQueryMetadata, PagedKVMetadata, SingleQueryMetadata,
)
from tinyvllm.runtime.graphs import DecodeGraphs
from tinyvllm.runtime.inputs import DecodeInputs
from tinyvllm.runtime.prefill_graphs import (
    ITEM_BUCKETS,
    TOKEN_BUCKETS,
    PrefillGraphs,
    PrefillInputs,
)


class ModelRunner:
    """Owns one physical KV store; request ownership stays in the BlockManager."""

    def __init__(
        self,
        model: nn.Module,
        *,
        block_size: int,
        num_blocks: int,
        max_model_len: int | None = None,
        max_num_seqs: int = 64,
        attention_backend: str = "hip",
        enforce_eager: bool = False,
        graph_sizes: tuple[int, ...] | None = None,
        kv_cache_dtype: torch.dtype | None = None,
        kv_scales: tuple[float, float] = (1.0, 1.0),
        prefill_graph_tokens: int | None = None,
        kv_cache_layout: str = "auto",
    ) -> None:
        """``kv_cache_dtype``: None keeps K/V in the model dtype;
        ``torch.float8_e4m3fn`` stores them as FP8 E4M3 with ``kv_scales``
        (k_scale, v_scale) - a layout beyond the reference (hip backend).
        ``kv_cache_layout``: the cache's storage order (``PagedKVCache``'s
        ``layout``; both keep the reference's [layers, slots, heads, dim]
        view); "auto" picks head-major when fewer than 256 (row, KV head)
        pairs can decode at once (``max_num_seqs * num_kv_heads``: few rows,
        whose long contexts split into many waves per head), else
        token-major.
        ``prefill_graph_tokens``: prefill and mixed steps of up to this many
        tokens (and up to 16 items; single-token items of short context only)
        replay captured graphs (0: always eager; None: sized from the model,
        ``default_prefill_graph_tokens``; beyond the reference, which runs
        these steps eagerly)."""
        if prefill_graph_tokens is None:
            prefill_graph_tokens = default_prefill_graph_tokens(model)
        if type(prefill_graph_tokens) is not int or prefill_graph_tokens < 0:
            raise ValueError("prefill_graph_tokens must be a non-negative int")
        if type(enforce_eager) is not bool:
            raise TypeError("enforce_eager must be bool")
        self.model = model.eval()
        self.backend = check_backend(attention_backend, model)
        parameter = next(model.parameters())
        self.device = parameter.device
        self.dtype = parameter.dtype
        config = model.config
        if max_model_len is None:
            max_model_len = config.max_position_embeddings
        _check_positive_int("max_model_len", max_model_len)
        if max_model_len > config.max_position_embeddings:
            raise ValueError("max_model_len exceeds model position capacity")
        self.max_model_len = max_model_len
        self.vocab_size = config.vocab_size
        self.decode_inputs: DecodeInputs | None = None
        self.decode_graphs: DecodeGraphs | None = None
        self.prefill_inputs: PrefillInputs | None = None
        self.prefill_graphs: PrefillGraphs | None = None
        self.kv_cache: PagedKVCache | None = None
        self.decode_workspace: torch.Tensor | None = None
        # Sampled ids of the last launched step stay here on the device; the
        # next batch's input_token_sources index them (pipelined decode).
        self.sampled = torch.zeros(max_num_seqs, dtype=torch.long, device=self.device)
        self._prev_count = 0
        try:
            kv_dtype = self.dtype if kv_cache_dtype is None else kv_cache_dtype
            if kv_dtype not in (self.dtype, torch.float8_e4m3fn):
                raise ValueError("KV cache dtype must be the model dtype or float8_e4m3fn")
            self.kv_cache = PagedKVCache(
                num_layers=config.num_hidden_layers, num_blocks=num_blocks,
                block_size=block_size, num_kv_heads=config.num_key_value_heads,
                head_dim=config.head_dim, device=self.device, dtype=kv_dtype,
                k_scale=float(kv_scales[0]), v_scale=float(kv_scales[1]),
                layout=resolve_layout(kv_cache_layout, max_num_seqs,
                                      config.num_key_value_heads),
            )
            if self.backend == "hip":
                self.decode_inputs = DecodeInputs(
                    max_num_seqs=max_num_seqs, max_model_len=max_model_len,
                    block_size=block_size, device=self.device,
                )
                ws = decode_workspace_bytes(max_num_seqs, config.num_attention_heads,
                                            config.num_key_value_heads, config.head_dim,
                                            max_model_len, block_size)
                # Split count grows as rows shrink; size for the worst case.
                for rows in range(1, max_num_seqs + 1):
                    ws = max(ws, decode_workspace_bytes(
                        rows, config.num_attention_heads, config.num_key_value_heads,
                        config.head_dim, max_model_len, block_size))
                if ws:
                    self.decode_workspace = torch.empty(ws, dtype=torch.uint8,
                                                        device=self.device)
                if not enforce_eager:
                    self.decode_graphs = DecodeGraphs(self.decode_inputs.stream)
                    self.decode_graphs.capture(model, self.decode_inputs, self.kv_cache,
                                               self.decode_workspace,
                                               sizes=graph_sizes, tokens=self.sampled)
                    # A step writes at most one KV slot per token.
                    graph_tokens = min(prefill_graph_tokens, self.kv_cache.num_slots)
                    if graph_tokens:
                        self.prefill_inputs = PrefillInputs(
                            max_tokens=graph_tokens,
                            max_items=min(max(ITEM_BUCKETS), max_num_seqs),
                            max_model_len=max_model_len, block_size=block_size,
                            device=self.device)
                        self.prefill_graphs = PrefillGraphs(self.prefill_inputs.stream)
                        self.prefill_graphs.capture(model, self.prefill_inputs,
                                                    self.kv_cache, self.sampled)
        except Exception:
            self.clear()
            raise

    # ------------------------------------------------------------ checks --

    def _validate(self, batch: PreparedBatch, cache: PagedKVCache) -> None:
        """CPU checks before any transfer or KV write (reference runner.py:101-193),
        vectorised with numpy: slot = table[p // bs] * bs + p % bs for every
        written position, positions follow the planned prefix, block ids in
        range, no aliasing inside a row, and blocks shared between rows are
        read-only full prefixes."""
        count = batch.num_items
        tokens = batch.num_query_tokens
        bs = cache.block_size
        if count == 0 or len(batch.request_ids) != count:
            raise ValueError("request_ids must align with nonempty batch items")
        if len(set(batch.request_ids)) != count:
            raise ValueError("a request may appear only once in one batch")
        if (len(batch.q_offsets) != count + 1 or batch.q_offsets[0] != 0
                or batch.q_offsets[-1] != tokens or len(batch.context_lens_before) != count
                or len(batch.context_lens_after) != count or len(batch.positions) != tokens
                or len(batch.query_lens) != count):
            raise ValueError("batch token and context metadata must align")
        if (batch.kv_block_size != bs or batch.kv_num_blocks != cache.num_blocks
                or len(batch.kv_block_table_offsets) != count + 1
                or batch.kv_block_table_offsets[0] != 0
                or batch.kv_block_table_offsets[-1] != len(batch.kv_block_table_ids)
                or len(batch.kv_slot_mapping) != tokens):
            raise ValueError("paged KV geometry and metadata must align")
        ids = np.asarray(batch.kv_block_table_ids, dtype=np.int64)
        if ids.size and (ids.min() < 0 or ids.max() >= cache.num_blocks):
            raise ValueError("block ID is out of range")
        inp = np.asarray(batch.input_ids, dtype=np.int64)
        if inp.size and (inp.min() < 0 or inp.max() >= self.vocab_size):
            raise ValueError("input token ID is out of vocabulary range")
        qoff = np.asarray(batch.q_offsets, dtype=np.int64)
        qlen = np.diff(qoff)
        before = np.asarray(batch.context_lens_before, dtype=np.int64)
        after = np.asarray(batch.context_lens_after, dtype=np.int64)
        if ((qlen <= 0).any() or (qlen != np.asarray(batch.query_lens)).any()
                or (before < 0).any() or (after != before + qlen).any()
                or (after > self.max_model_len).any()):
            raise ValueError("invalid query or context length")
        item = np.repeat(np.arange(count), qlen)
        pos = np.asarray(batch.positions, dtype=np.int64)
        if (pos != before[item] + (np.arange(tokens) - qoff[item])).any():
            raise ValueError("positions must follow the planned KV prefix")
        toff = np.asarray(batch.kv_block_table_offsets, dtype=np.int64)
        tlen = np.diff(toff)
        if (tlen != -(-after // bs)).any():
            raise ValueError("block table length does not match context")
        # Blocks referenced more than once are the only ones that can alias
        # inside a row or be shared between rows; usually there are none.
        ordered = np.sort(ids)
        repeated = ordered[1:][ordered[1:] == ordered[:-1]]
        if repeated.size:
            owner = np.repeat(np.arange(count), tlen)
            if np.unique(owner * cache.num_blocks + ids).size != ids.size:
                raise ValueError("one request cannot alias its logical blocks")
            # Written blocks: logical index >= before // bs of their row.
            logical = np.arange(ids.size) - toff[owner]
            written = logical >= (before // bs)[owner]
            if np.isin(ids[written], repeated).any():
                raise ValueError("shared blocks must be complete read-only prefixes")
        expect = ids[toff[item] + pos // bs] * bs + pos % bs
        if (expect != np.asarray(batch.kv_slot_mapping, dtype=np.int64)).any():
            raise ValueError("write slots do not match block tables and positions")
        sources = batch.input_token_sources
        if sources is not None:
            src = np.asarray(sources, dtype=np.int64)
            if src.shape != (tokens,):
                raise ValueError("input_token_sources must have one entry per token")
            if src.size and (src.min() < -1 or src.max() >= getattr(self, "_prev_count", 0)):
                raise ValueError("input token source is not a row of the previous step")
        samples = batch.sample_token_indices
        if (len(batch.sample_request_ids) != batch.num_samples
                or len(batch.sampling_params) != batch.num_samples
                or any(a >= b for a, b in zip(samples, samples[1:]))):
            raise ValueError("sampling rows must be aligned and ordered")
        ends = dict(zip((int(e) - 1 for e in qoff[1:]), batch.request_ids))
        for index, request_id in zip(samples, batch.sample_request_ids):
            if ends.get(index) != request_id:
                raise ValueError("sampling rows do not match batch item boundaries")

    # ----------------------------------------------------------- lowering --

    def _lower(self, batch: PreparedBatch) -> ModelInput:
        """Eager-path metadata: decode rows (query length 1) and one multi-query
        CSR spanning the items with longer queries."""
        dev = self.device

        def t(values):
            return torch.tensor(values, dtype=torch.long).to(dev, non_blocking=True)

        qlen = batch.query_lens
        single = [i for i, n in enumerate(qlen) if n == 1]
        multi = [i for i, n in enumerate(qlen) if n > 1]
        toff = batch.kv_block_table_offsets
        decode = None
        if single:
            rows, blocks, offsets, lens = [], [], [0], []
            for i in single:
                rows.append(batch.q_offsets[i])
                blocks.extend(batch.kv_block_table_ids[toff[i]:toff[i + 1]])
                offsets.append(len(blocks))
                lens.append(batch.context_lens_after[i])
            decode = SingleQueryMetadata(t(rows), t(blocks), t(offsets), t(lens),
                                         max(lens))
        prefill = None
        if multi:
            lo, hi = multi[0], multi[-1] + 1
            q_offsets = batch.q_offsets[lo:hi + 1]
            prefill = MultiQueryMetadata(
                query_offsets=t(q_offsets),
                block_table_ids=t(batch.kv_block_table_ids[toff[lo]:toff[hi]]),
                block_table_offsets=t([o - toff[lo] for o in toff[lo:hi + 1]]),
                context_lens=t(batch.context_lens_after[lo:hi]),
                max_query_len=max(qlen[lo:hi]),
            )
        return ModelInput(
            input_ids=t(batch.input_ids),
            positions=t(batch.positions),
            sample_token_indices=t(batch.sample_token_indices) if batch.num_samples else None,
            kv=PagedKVMetadata(slot_mapping=t(batch.kv_slot_mapping), decode=decode,
                               prefill=prefill),
        )

    def _attention(self, batch: PreparedBatch, model_input: ModelInput):
        cache = self.kv_cache
        if self.backend == "reference":
            toff = batch.kv_block_table_offsets
            tables = [batch.kv_block_table_ids[toff[i]:toff[i + 1]]
                      for i in range(batch.num_items)]
            return SDPAAttention(model_input, cache, q_offsets=batch.q_offsets,
                                 context_lens_before=batch.context_lens_before,
                                 context_lens_after=batch.context_lens_after,
                                 block_tables=tables)
        return HipAttention(model_input, cache, decode_workspace=self.decode_workspace)

    # -------------------------------------------------------------- steps --

    @torch.inference_mode()
    def run(self, batch: PreparedBatch) -> torch.Tensor | None:
        """Return borrowed logits of the sampled rows (consume before the next run)."""
        out = self._run(batch, counters=None, want_tokens=False)
        return None if out is None else out[0]

    @torch.inference_mode()
    def run_and_sample(self, batch: PreparedBatch,
                       counters) -> tuple[torch.Tensor, torch.Tensor] | None:
        """(logits, sampled token ids) of the sampled rows, on the device."""
        return self._run(batch, counters=counters, want_tokens=True)

    def _run(self, batch, *, counters, want_tokens):
        cache = self.kv_cache
        if cache is None:
            raise RuntimeError("runner is closed")
        self._validate(batch, cache)
        if counters is None:
            counters = [0] * batch.num_samples
        self._prev_count = 0  # until this step's ids are in place
        out = self._forward(batch, counters, want_tokens)
        if out is None or out[1] is None:
            return out
        logits, tokens = out
        rows = tokens.numel()
        if rows <= self.sampled.numel():
            if tokens.data_ptr() != self.sampled.data_ptr():
                self.sampled[:rows].copy_(tokens)
                tokens = self.sampled[:rows]
            self._prev_count = rows
        return logits, tokens

    def _forward(self, batch, counters, want_tokens):
        cache = self.kv_cache
        if self.decode_inputs is not None:
            model_input = self.decode_inputs.prepare(batch, counters)
            if model_input is not None:
                if self.decode_graphs is not None:  # the graph applies the table updates
                    replayed = self.decode_graphs.replay(
                        batch.num_items, max(batch.context_lens_after))
                    if replayed is not None:
                        return replayed
                self.decode_inputs.apply_table_updates()
                if batch.input_token_sources is not None:
                    resolve_tokens(model_input.input_ids,
                                   self.decode_inputs.d["sources"][:batch.num_items],
                                   self.sampled)
                attention = HipAttention(model_input, cache,
                                         decode_workspace=self.decode_workspace)
                hidden = self.model(model_input.input_ids, model_input.positions,
                                    attention=attention)
                logits = self.model.compute_logits(hidden)
                tokens = None
                if want_tokens:
                    tokens = sample(logits, *self.decode_inputs.sampling_views(batch.num_items))
                return logits, tokens
        if self.prefill_graphs is not None:
            buckets = self.prefill_inputs.prepare(batch, counters)
            if buckets is not None:
                replayed = self.prefill_graphs.replay(*buckets)
                if replayed is not None:
                    logits, tokens = replayed
                    samples = batch.num_samples
                    if samples == 0:
                        return None
                    return logits[:samples], tokens[:samples] if want_tokens else None
        model_input = self._lower(batch)
        if batch.input_token_sources is not None:
            src = torch.tensor(np.asarray(batch.input_token_sources, dtype=np.int64)).to(
                self.device, non_blocking=True)
            if self.backend == "hip":
                resolve_tokens(model_input.input_ids, src, self.sampled)
            else:  # the torch path: same substitution with torch ops
                taken = self.sampled[src.clamp(min=0)]
                model_input.input_ids.copy_(torch.where(src >= 0, taken,
                                                        model_input.input_ids))
        hidden = self.model(model_input.input_ids, model_input.positions,
                            attention=self._attention(batch, model_input))
        if batch.num_samples == 0:
            return None
        logits = self.model.compute_logits(hidden, model_input.sample_token_indices)
        tokens = None
        if want_tokens:
            tokens = sample_rows(logits, batch.sampling_params, counters)
        return logits, tokens

    def clear(self) -> None:
        try:
            try:
                if self.prefill_graphs is not None:
                    self.prefill_graphs.close()
            finally:
                if self.decode_graphs is not None:
                    self.decode_graphs.close()
        finally:
            self.prefill_graphs = None
            self.prefill_inputs = None
            self.decode_graphs = None
            self.decode_inputs = None
            self.decode_workspace = None
            self.kv_cache = None
            self.model = None


# GEMM work of an eager prefill step whose launches the host can no longer
# outrun (~6 ms of dense-layer GEMMs on MI355X, about the host's launch time
# for a 28-64-layer eager step): bigger steps gain nothing from a graph.
_GRAPH_STEP_FLOP = 8e12


def default_prefill_graph_tokens(model: nn.Module) -> int:
    """The largest prefill-graph token bucket whose dense-layer GEMMs (2 flop
    per weight per token) stay within ``_GRAPH_STEP_FLOP``, at least the
    smallest bucket: 2048 for Qwen3-0.6B, 512 for 8B, 128 for 32B."""
    layers = getattr(getattr(model, "model", None), "layers", None)
    weights = sum(p.numel() for p in (layers.parameters() if layers is not None
                                      else model.parameters()))
    fitting = [b for b in TOKEN_BUCKETS if 2 * weights * b <= _GRAPH_STEP_FLOP]
    return max(fitting) if fitting else min(TOKEN_BUCKETS)


def sample_rows(logits: torch.Tensor, params, counters) -> torch.Tensor:
    """Sample each row of ``logits`` with its SamplingParams on the GPU."""
    from tinyvllm.kernels.sampling import argmax

    if all(p.greedy for p in params):
        return argmax(logits)
    dev = logits.device
    rows = len(params)
    floats = torch.tensor([[p.temperature for p in params], [p.top_p for p in params]],
                          dtype=torch.float32).to(dev, non_blocking=True)
    ints = torch.tensor([[p.top_k for p in params], [signed64(p.seed) for p in params],
                         list(counters)],
                        dtype=torch.long).to(dev, non_blocking=True)
    assert ints.shape[1] == rows
    return sample(logits, floats[0], ints[0], floats[1], ints[1], ints[2])


def signed64(value: int) -> int:
    """Reinterpret a 64-bit unsigned seed as the int64 with the same bits."""
    return value - (1 << 64) if value >= (1 << 63) else value
