"""Step plans and the flat CPU batch handed to the executor
(reference: tinyvllm/batch.py:1-288).

``PreparedBatch`` keeps the reference's field names: it is the contract
between the CPU scheduler and the GPU runner.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum, auto
from typing import Protocol

import numpy as np

from tinyvllm._validation import _check_positive_int
from tinyvllm.request import RequestState, SamplingParams, WorkClass


class StepMode(Enum):
    PREFILL_ONLY = auto()
    DECODE_ONLY = auto()
    MIXED = auto()


@dataclass(frozen=True, slots=True)
class WorkItem:
    request_id: int
    request_slot: int
    work_class: WorkClass
    token_start: int
    query_len: int
    context_len_before: int
    should_sample: bool

    @property
    def token_end(self) -> int:
        return self.token_start + self.query_len

    @property
    def context_len_after(self) -> int:
        return self.context_len_before + self.query_len


@dataclass(frozen=True, slots=True)
class StepPlan:
    """Ordered work of one step: decode items first, then prefill items."""

    plan_id: int
    items: tuple[WorkItem, ...]
    mode: StepMode = field(init=False)
    num_decode_items: int = field(init=False)
    num_prefill_items: int = field(init=False)
    num_query_tokens: int = field(init=False)
    num_samples: int = field(init=False)

    def __post_init__(self) -> None:
        items = tuple(self.items)
        object.__setattr__(self, "items", items)
        if not items:
            raise ValueError("StepPlan must contain at least one item")
        decode = 0
        seen_prefill = False
        for item in items:
            if item.work_class is WorkClass.PREFILL:
                seen_prefill = True
            elif item.work_class is WorkClass.DECODE:
                if seen_prefill:
                    raise ValueError("decode items must precede prefill items")
                decode += 1
            else:
                raise ValueError(f"unsupported work class: {item.work_class}")
        prefill = len(items) - decode
        mode = (StepMode.PREFILL_ONLY if decode == 0 else
                StepMode.DECODE_ONLY if prefill == 0 else StepMode.MIXED)
        object.__setattr__(self, "mode", mode)
        object.__setattr__(self, "num_decode_items", decode)
        object.__setattr__(self, "num_prefill_items", prefill)
        object.__setattr__(self, "num_query_tokens", sum(i.query_len for i in items))
        object.__setattr__(self, "num_samples", sum(i.should_sample for i in items))


@dataclass(frozen=True, slots=True)
class PreparedBatch:
    """One step's flat CPU metadata. Sequence fields are tuples of ints or
    1-D int64 numpy arrays (BatchBuilder emits arrays for the block-table
    ids and the slot mapping)."""

    plan_id: int
    mode: StepMode
    input_ids: tuple[int, ...]
    positions: tuple[int, ...]
    q_offsets: tuple[int, ...]
    context_lens_before: tuple[int, ...]
    query_lens: tuple[int, ...]
    context_lens_after: tuple[int, ...]
    sample_token_indices: tuple[int, ...]
    sample_request_ids: tuple[int, ...]
    sampling_params: tuple[SamplingParams, ...]
    kv_block_size: int
    kv_num_blocks: int
    kv_block_table_ids: tuple[int, ...] | np.ndarray
    kv_block_table_offsets: tuple[int, ...]
    kv_slot_mapping: tuple[int, ...] | np.ndarray
    request_ids: tuple[int, ...]
    # Pipelined steps (beyond the reference): per input token, -1 = the id in
    # input_ids, j >= 0 = row j of the previous launched step's sampled tokens,
    # still on the device when this batch is built. None = all from input_ids.
    input_token_sources: tuple[int, ...] | np.ndarray | None = None
    # Device-resident block tables (beyond the reference): per item, its
    # request slot (unique among active requests) and its table epoch
    # (equal epochs: the table only grew since). None: upload whole tables.
    request_slots: tuple[int, ...] | None = None
    kv_table_epochs: tuple[int, ...] | None = None

    @property
    def num_items(self) -> int:
        return len(self.query_lens)

    @property
    def num_query_tokens(self) -> int:
        return len(self.input_ids)

    @property
    def num_samples(self) -> int:
        return len(self.sample_token_indices)


@dataclass(frozen=True, slots=True)
class StepResult:
    """Ordered executor output for one dispatched plan."""

    plan_id: int
    sample_request_ids: tuple[int, ...]
    sampled_token_ids: tuple[int, ...]

    def __post_init__(self) -> None:
        object.__setattr__(self, "sample_request_ids", tuple(self.sample_request_ids))
        object.__setattr__(self, "sampled_token_ids", tuple(self.sampled_token_ids))
        if len(self.sample_request_ids) != len(self.sampled_token_ids):
            raise ValueError("sample request and token counts do not match")


class KVPlan(Protocol):
    """What BatchBuilder needs from the block manager's per-step plan."""

    plan_id: int
    request_ids: tuple[int, ...]
    block_size: int
    num_blocks: int

    def append_metadata(self, request_id: int, start: int,
                        count: int) -> tuple[np.ndarray, np.ndarray]:
        """(block ids of the request's table, slots of positions [start, start+count))."""
        ...


class BatchBuilder:
    """Flattens a StepPlan into a PreparedBatch (reference batch.py:164-288).

    The block-table ids and the slot mapping - the large, per-step fields -
    are int64 numpy arrays; every other field is a tuple."""

    def __init__(self, *, max_model_len: int) -> None:
        _check_positive_int("max_model_len", max_model_len)
        self.max_model_len = max_model_len

    def prepare(self, plan: StepPlan, requests: tuple[RequestState, ...], *,
                kv: KVPlan, pending_rows: dict[int, int] | None = None) -> PreparedBatch:
        """``pending_rows``: request -> row among the previous launched step's
        samples, for requests whose newest token (a negative placeholder) is
        still on the device; such inputs become ``input_token_sources``."""
        if len(requests) != len(plan.items):
            raise ValueError("requests must align with plan items")
        if kv.plan_id != plan.plan_id:
            raise ValueError("KV plan_id does not match step plan")
        if tuple(kv.request_ids) != tuple(i.request_id for i in plan.items):
            raise ValueError("KV requests must match all plan items in order")
        input_ids: list[int] = []
        positions: list[int] = []
        q_offsets = [0]
        before_l: list[int] = []
        query_l: list[int] = []
        after_l: list[int] = []
        sample_idx: list[int] = []
        sample_rid: list[int] = []
        params: list[SamplingParams] = []
        tables: list[np.ndarray] = []
        table_off = [0]
        epoch_of = getattr(kv, "table_epoch", None)
        slots: list[np.ndarray] = []
        rids: list[int] = []
        sources: list[int] | None = None
        for item, request in zip(plan.items, requests):
            if request.request_id != item.request_id:
                raise ValueError("request order does not match plan")
            after = item.context_len_after
            if after > self.max_model_len:
                raise ValueError("planned context exceeds max_model_len")
            if item.context_len_before != item.token_start:
                raise ValueError("context length must match append start")
            tokens = request.token_slice(item.token_start, item.token_end)
            if len(tokens) != item.query_len:
                raise RuntimeError("token slice length does not match query_len")
            if tokens and tokens[-1] < 0:  # the previous step's sample, unresolved
                row = (pending_rows or {}).get(request.request_id)
                if row is None or min(tokens[:-1], default=0) < 0:
                    raise ValueError("unresolved input token without a pending sample row")
                if sources is None:
                    sources = [-1] * len(input_ids)
                sources.extend([-1] * (len(tokens) - 1) + [row])
                tokens = tokens[:-1] + [0]
            elif sources is not None:
                sources.extend([-1] * len(tokens))
            table, slot_map = kv.append_metadata(item.request_id, item.token_start,
                                                 item.query_len)
            rids.append(request.request_id)
            tables.append(table)
            table_off.append(table_off[-1] + len(table))
            slots.append(slot_map)
            input_ids.extend(tokens)
            positions.extend(range(item.context_len_before, after))
            q_offsets.append(len(input_ids))
            before_l.append(item.context_len_before)
            query_l.append(item.query_len)
            after_l.append(after)
            if item.should_sample:
                sample_idx.append(q_offsets[-1] - 1)
                sample_rid.append(item.request_id)
                params.append(request.sampling)
        return PreparedBatch(
            plan_id=plan.plan_id, mode=plan.mode,
            input_ids=tuple(input_ids), positions=tuple(positions),
            q_offsets=tuple(q_offsets), context_lens_before=tuple(before_l),
            query_lens=tuple(query_l), context_lens_after=tuple(after_l),
            sample_token_indices=tuple(sample_idx), sample_request_ids=tuple(sample_rid),
            sampling_params=tuple(params), kv_block_size=kv.block_size,
            kv_num_blocks=kv.num_blocks,
            kv_block_table_ids=np.concatenate(tables) if tables else np.zeros(0, np.int64),
            kv_block_table_offsets=tuple(table_off),
            kv_slot_mapping=np.concatenate(slots) if slots else np.zeros(0, np.int64),
            request_ids=tuple(rids),
            input_token_sources=None if sources is None else tuple(sources),
            request_slots=tuple(i.request_slot for i in plan.items),
            kv_table_epochs=None if epoch_of is None else tuple(
                epoch_of(i.request_id) for i in plan.items),
        )
