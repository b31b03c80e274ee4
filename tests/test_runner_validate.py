"""The runner's CPU batch checks reject every malformed batch before any
transfer (reference runner.py:101-193), including prefix-sharing rules."""
import dataclasses

import numpy as np
import pytest

from tinyvllm.batch import PreparedBatch, StepMode
from tinyvllm.request import SamplingParams
from tinyvllm.runtime.runner import ModelRunner


class _Cache:
    block_size = 4
    num_blocks = 32


def _runner():
    r = ModelRunner.__new__(ModelRunner)
    r.vocab_size, r.max_model_len = 100, 64
    return r


def _batch(tables, befores, qlens):
    ids, pos, qoff, after, slots, toff = [], [], [0], [], [], [0]
    for table, b, q in zip(tables, befores, qlens):
        ids += [7] * q
        pos += list(range(b, b + q))
        qoff.append(len(ids))
        after.append(b + q)
        toff.append(toff[-1] + len(table))
        slots += [table[p // 4] * 4 + p % 4 for p in range(b, b + q)]
    n = len(tables)
    return PreparedBatch(
        plan_id=0, mode=StepMode.MIXED, input_ids=tuple(ids), positions=tuple(pos),
        q_offsets=tuple(qoff), context_lens_before=tuple(befores), query_lens=tuple(qlens),
        context_lens_after=tuple(after), sample_token_indices=tuple(q - 1 for q in qoff[1:]),
        sample_request_ids=tuple(range(n)), sampling_params=(SamplingParams(),) * n,
        kv_block_size=4, kv_num_blocks=32,
        kv_block_table_ids=np.array([b for t in tables for b in t], dtype=np.int64),
        kv_block_table_offsets=tuple(toff), kv_slot_mapping=np.array(slots, dtype=np.int64),
        request_ids=tuple(range(n)))


def test_valid_batch_with_shared_read_only_prefix_passes():
    # Rows 0 and 1 share full prefix blocks 3, 9 and write only their own tails.
    b = _batch([[3, 9, 5], [3, 9, 6]], befores=[8, 8], qlens=[3, 2])
    _runner()._validate(b, _Cache)


@pytest.mark.parametrize("tables,befores,qlens,message", [
    ([[3, 3]], [0], [6], "alias"),                    # a row reuses its own block
    ([[3, 9], [3, 10]], [0, 4], [6, 2], "read-only"),  # row 0 writes shared block 3
    ([[3, 9, 5], [4, 9]], [8, 4], [1, 2], "read-only"),  # row 1 writes into row 0's block 9
    ([[3, 40]], [0], [6], "out of range"),
])
def test_malformed_tables_are_rejected(tables, befores, qlens, message):
    with pytest.raises(ValueError, match=message):
        _runner()._validate(_batch(tables, befores, qlens), _Cache)


def test_wrong_slots_and_positions_are_rejected():
    b = _batch([[3, 9]], befores=[4], qlens=[2])
    bad = dataclasses.replace(b, kv_slot_mapping=np.array([36, 38]))
    with pytest.raises(ValueError, match="slots"):
        _runner()._validate(bad, _Cache)
    bad = dataclasses.replace(b, positions=(4, 6))
    with pytest.raises(ValueError, match="positions"):
        _runner()._validate(bad, _Cache)
    bad = dataclasses.replace(b, input_ids=(7, 100))
    with pytest.raises(ValueError, match="vocabulary"):
        _runner()._validate(bad, _Cache)


def test_token_sources_must_name_rows_of_the_previous_step():
    b = _batch([[3, 9], [4, 10]], befores=[6, 5], qlens=[1, 2])
    r = _runner()
    r._prev_count = 2
    r._validate(dataclasses.replace(b, input_token_sources=(1, 0, -1)), _Cache)
    for sources, message in (((2, -1, -1), "previous step"), ((0, -2, -1), "previous step"),
                             ((0, 1), "one entry per token")):
        with pytest.raises(ValueError, match=message):
            r._validate(dataclasses.replace(b, input_token_sources=sources), _Cache)
    r._prev_count = 0  # nothing launched before: no source is valid
    with pytest.raises(ValueError, match="previous step"):
        r._validate(dataclasses.replace(b, input_token_sources=(0, -1, -1)), _Cache)


def test_batch_builder_turns_pending_tokens_into_sources():
    """A decode row whose newest token is still a placeholder gets input id 0
    and a source naming its row among the previous step's samples; prompt
    tokens keep source -1; a placeholder without a known row is an error."""
    from tinyvllm.batch import BatchBuilder, StepPlan, WorkItem
    from tinyvllm.request import RequestState, WorkClass
    from tinyvllm.scheduler import PENDING_TOKEN

    class _KV:
        plan_id, request_ids, block_size, num_blocks = 5, (1, 2), 4, 32

        def append_metadata(self, rid, start, count):
            table = np.array([3, 9] if rid == 1 else [4], dtype=np.int64)
            pos = np.arange(start, start + count)
            return table, table[pos // 4] * 4 + pos % 4

    dec = RequestState(request_id=1, submit_seq=0, prompt_token_ids=[11, 12, 13, 14, 15],
                       sampling=SamplingParams(), arrival_ns=0,
                       output_token_ids=[21])
    dec.output_token_ids.append(PENDING_TOKEN)  # sampled by the launched step, row 3
    pre = RequestState(request_id=2, submit_seq=1, prompt_token_ids=[31, 32, 33],
                       sampling=SamplingParams(), arrival_ns=0)
    plan = StepPlan(plan_id=5, items=(
        WorkItem(1, 0, WorkClass.DECODE, 6, 1, 6, True),
        WorkItem(2, 1, WorkClass.PREFILL, 0, 3, 0, True)))
    batch = BatchBuilder(max_model_len=64).prepare(plan, (dec, pre), kv=_KV(),
                                                   pending_rows={1: 3})
    assert batch.input_ids == (0, 31, 32, 33)
    assert batch.input_token_sources == (3, -1, -1, -1)
    with pytest.raises(ValueError, match="pending sample row"):
        BatchBuilder(max_model_len=64).prepare(plan, (dec, pre), kv=_KV())
