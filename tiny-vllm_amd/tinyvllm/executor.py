"""Batch execution over a fixed paged KV store (reference: tinyvllm/executor.py:1-153)."""
from __future__ import annotations

from collections.abc import Iterable
from dataclasses import dataclass

import torch
from torch import nn

from tinyvllm._validation import _check_positive_int
from tinyvllm.batch import PreparedBatch, StepResult
from tinyvllm.runtime.runner import ModelRunner
from tinyvllm.sampling import Sampler


@dataclass(frozen=True, slots=True)
class ExecutorCapabilities:
    """Model geometry and execution limits the scheduler must respect."""

    vocab_size: int | None = None
    max_model_len: int | None = None
    kv_block_size: int | None = None
    kv_num_blocks: int | None = None
    max_batch_size: int | None = None

    def __post_init__(self) -> None:
        for name in ("vocab_size", "max_model_len", "kv_block_size", "kv_num_blocks",
                     "max_batch_size"):
            value = getattr(self, name)
            if value is not None:
                _check_positive_int(name, value)

    def validate_configuration(self, *, max_model_len: int, block_size: int,
                               num_blocks: int, max_batch_size: int) -> None:
        if self.max_model_len is not None and max_model_len > self.max_model_len:
            raise ValueError("scheduler max_model_len exceeds executor capacity")
        if self.max_batch_size is not None and max_batch_size > self.max_batch_size:
            raise ValueError("scheduler maximum step batch exceeds executor capacity")
        for name, actual, expected in (("block_size", block_size, self.kv_block_size),
                                       ("num_blocks", num_blocks, self.kv_num_blocks)):
            if expected is not None and actual != expected:
                raise ValueError(f"scheduler {name} does not match executor")

    def validate_token_ids(self, token_ids: Iterable[int]) -> None:
        if self.vocab_size is not None and any(t >= self.vocab_size for t in token_ids):
            raise ValueError("token ID is out of vocabulary range")


class PendingStep:
    """A launched step whose sampled token ids are on their way to the host."""

    __slots__ = ("plan_id", "sample_request_ids", "_host", "_rows", "_event", "_result")

    def __init__(self, plan_id: int, sample_request_ids: tuple[int, ...],
                 host: torch.Tensor | None, rows: int, event) -> None:
        self.plan_id = plan_id
        self.sample_request_ids = sample_request_ids
        self._host, self._rows, self._event = host, rows, event
        self._result: StepResult | None = None

    def ready(self) -> bool:
        return self._result is not None or self._event is None or self._event.query()

    def result(self) -> StepResult:
        """Wait for the step's sampled ids (the step's one device->host sync)."""
        if self._result is None:
            tokens = ()
            if self._event is not None:
                self._event.synchronize()
                tokens = tuple(self._host[:self._rows].tolist())
            self._result = StepResult(self.plan_id, self.sample_request_ids, tokens)
            self._host = self._event = None
        return self._result


class Executor:
    """Runs one PreparedBatch: forward, sample, and hand tokens back to the CPU."""

    def __init__(self, model: nn.Module, *, block_size: int, num_blocks: int,
                 max_model_len: int | None = None, sampler: Sampler | None = None,
                 max_num_seqs: int = 64, attention_backend: str = "hip",
                 enforce_eager: bool = False,
                 graph_sizes: tuple[int, ...] | None = None,
                 kv_cache_dtype: torch.dtype | None = None,
                 kv_scales: tuple[float, float] = (1.0, 1.0),
                 kv_cache_layout: str = "auto",
                 prefill_graph_tokens: int | None = None) -> None:
        self.runner = ModelRunner(model, block_size=block_size, num_blocks=num_blocks,
                                  max_model_len=max_model_len, max_num_seqs=max_num_seqs,
                                  attention_backend=attention_backend,
                                  enforce_eager=enforce_eager, graph_sizes=graph_sizes,
                                  kv_cache_dtype=kv_cache_dtype, kv_scales=kv_scales,
                                  kv_cache_layout=kv_cache_layout,
                                  prefill_graph_tokens=prefill_graph_tokens)
        self.capabilities = ExecutorCapabilities(
            vocab_size=model.config.vocab_size,
            max_model_len=self.runner.max_model_len,
            kv_block_size=block_size,
            kv_num_blocks=num_blocks,
            max_batch_size=(self.runner.decode_inputs.capacity
                            if self.runner.decode_inputs is not None else None),
        )
        self.sampler = Sampler() if sampler is None else sampler
        self._host: list[torch.Tensor | None] = [None, None]
        self._in_flight: list[PendingStep | None] = [None, None]
        self._turn = 0

    @torch.inference_mode()
    def execute(self, batch: PreparedBatch) -> StepResult:
        return self.launch(batch).result()

    @torch.inference_mode()
    def launch(self, batch: PreparedBatch) -> PendingStep:
        """Enqueue the step and return at once; its sampled ids travel to a
        pinned host buffer behind it on the stream. Until ``result()`` the
        host is free to build the next batch, whose ``input_token_sources``
        may name this step's sampled rows (they never leave the device)."""
        counters = self.sampler.counters(batch.sampling_params, batch.sample_request_ids)
        out = self.runner.run_and_sample(batch, counters)
        if out is None:
            return PendingStep(batch.plan_id, batch.sample_request_ids, None, 0, None)
        tokens = out[1]
        rows = tokens.numel()
        # Two host buffers alternate; a step two launches back must be read
        # before its buffer is reused.
        index = self._turn
        self._turn ^= 1
        previous = self._in_flight[index]
        if previous is not None:
            previous.result()
        host = self._host[index]
        if host is None or host.numel() < rows:
            host = torch.empty(max(rows, 64), dtype=torch.long, pin_memory=True)
            self._host[index] = host
        host[:rows].copy_(tokens, non_blocking=True)
        event = torch.cuda.Event()
        event.record()
        pending = PendingStep(batch.plan_id, batch.sample_request_ids, host, rows, event)
        self._in_flight[index] = pending
        return pending

    def release(self, request_id: int) -> None:
        self.sampler.release(request_id)

    def clear(self) -> None:
        try:
            self.runner.clear()
        finally:
            self.sampler.clear()
