"""Which steps replay a captured prefill graph, and in which (token, item)
bucket (host logic of tinyvllm/runtime/prefill_graphs.py; no GPU)."""
from helpers import ManualBatches

from tinyvllm.runtime.prefill_graphs import DECODE_CONTEXT_BOUND, PrefillInputs


def _inputs(max_tokens=2048, max_items=16, pitch_pages=64):
    inputs = PrefillInputs.__new__(PrefillInputs)  # bucket logic only: no buffers
    inputs.max_tokens, inputs.max_items = max_tokens, max_items
    inputs.table_capacity = max_items * pitch_pages
    return inputs


def _batch(prompts, items, done=None, num_blocks=1024):
    mb = ManualBatches(prompts, block_size=16, num_blocks=num_blocks)
    if done:
        for seq, n in done.items():
            mb.done[seq] = n
    return mb.step(items)


def test_prefill_buckets_round_up():
    p = [[1] * 700] * 3
    assert _inputs().buckets_for(_batch(p, [(0, 37, True), (1, 5, True)])) == (64, 2)
    assert _inputs().buckets_for(_batch(p, [(0, 600, True)])) == (768, 1)
    assert _inputs().buckets_for(_batch(p, [(0, 2, True), (1, 3, True), (2, 4, True)])) == (32, 4)
    # the bucket ceiling follows max_tokens (the cache's slot count caps it)
    assert _inputs(max_tokens=512).buckets_for(_batch(p, [(0, 600, True)])) is None
    assert _inputs(max_tokens=600).buckets_for(_batch(p, [(0, 500, True)])) == (512, 1)


def test_decode_only_and_long_decode_rows_stay_off_the_prefill_graphs():
    p = [[1] * 2000] * 3
    # every item a single token: a decode step (it has graphs of its own)
    assert _inputs().buckets_for(_batch(p, [(0, 1, True), (1, 1, True)],
                                        done={0: 100, 1: 100})) is None
    # a decode row of short context rides along in the prefill kernel
    short = _batch(p, [(0, 1, True), (1, 64, True)], done={0: DECODE_CONTEXT_BOUND - 1})
    assert _inputs().buckets_for(short) == (128, 2)
    # beyond the bound the split-K decode kernel is faster: eager
    long = _batch(p, [(0, 1, True), (1, 64, True)], done={0: DECODE_CONTEXT_BOUND})
    assert _inputs().buckets_for(long) is None


def test_item_and_table_limits():
    p = [[1] * 40] * 20
    many = _batch(p, [(s, 2, True) for s in range(17)])
    assert _inputs().buckets_for(many) is None            # 17 items > 16
    assert _inputs().buckets_for(_batch(p, [(s, 2, True) for s in range(16)])) == (32, 16)
    assert _inputs(max_items=4).buckets_for(_batch(p, [(s, 2, True) for s in range(5)])) is None
    # block tables beyond the packed capacity
    assert _inputs(max_items=1, pitch_pages=2).buckets_for(_batch(p, [(0, 40, True)])) is None
    assert _inputs(max_items=1, pitch_pages=3).buckets_for(_batch(p, [(0, 40, True)])) == (64, 1)
