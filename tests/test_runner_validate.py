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
