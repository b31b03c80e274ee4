"""The host KV ledger (BlockPool, StepKV journal, BlockManager, PrefixCache)
on the CPU: holder counts, reuse order, journal undo, slot arithmetic and
prefix indexing, each against a brute-force or closed-form expectation."""
import numpy as np
import pytest

from tinyvllm.cache import BlockAppend, BlockManager, BlockPool, BlockRef, StepKV
from tinyvllm.prefix_cache import block_digests


def test_pool_hands_out_blank_blocks_then_the_oldest_idle_ones():
    pool = BlockPool(num_blocks=4)
    a = pool.allocate(4)
    assert sorted(a) == [0, 1, 2, 3] and pool.free_block_count == 0
    refs = [pool.ref(b) for b in a]
    pool.label(b"x", refs[2])
    pool.label(b"y", refs[0])
    for r in (refs[2], refs[0], refs[1], refs[3]):  # 2 then 0 go idle (labelled)
        pool.drop(r)
    assert pool.free_block_count == 4 and pool.cached_block_count == 2
    # Blank blocks (1, 3) first, then idle blocks oldest-released first (2, 0).
    order = [pool.allocate(1)[0] for _ in range(4)]
    assert set(order[:2]) == {1, 3}
    assert order[2:] == [2, 0]
    assert pool.evictions == 2 and pool.cached_block_count == 0
    assert pool.find(b"x") is None
    with pytest.raises(RuntimeError, match="stale"):
        pool.hold(refs[2])  # generation moved on with the reuse


def test_holding_an_idle_block_takes_it_out_of_the_free_count():
    pool = BlockPool(num_blocks=3)
    (b,) = pool.allocate(1)
    ref = pool.ref(b)
    assert pool.label(b"k", ref) == ref
    pool.drop(ref)
    assert pool.is_idle(ref) and pool.free_block_count == 3
    pool.hold(ref)
    assert not pool.is_idle(ref) and pool.free_block_count == 2
    assert pool.held(ref) == 1
    # Its old heap entry is stale: allocating everything skips it.
    assert sorted(pool.allocate(2)) == [x for x in range(3) if x != b]
    pool.drop(ref)
    assert pool.allocate(1) == [b] and pool.evictions == 1


def test_label_returns_the_block_already_holding_the_contents():
    pool = BlockPool(num_blocks=2)
    x, y = (pool.ref(b) for b in pool.allocate(2))
    assert pool.label(b"d", x) == x
    assert pool.label(b"d", y) == x
    with pytest.raises(RuntimeError, match="another prefix"):
        pool.label(b"e", x)


def _slots(ids, start, end, bs):
    return [int(ids[p // bs]) * bs + p % bs for p in range(start, end)]


def test_stage_slots_follow_the_table_closed_form_and_undo_restores_the_pool():
    bs = 4
    m = BlockManager(block_size=bs, num_blocks=16, enable_prefix_caching=False)
    step = m.stage(0, [BlockAppend(7, 0, 10), BlockAppend(9, 0, 3)])
    assert isinstance(step, StepKV) and step.request_ids == (7, 9)
    assert m.free_block_count == 16 - 3 - 1
    ids, slots = step.append_metadata(7, 0, 10)
    assert len(ids) == 3 and list(slots) == _slots(ids, 0, 10, bs)
    step.undo()
    assert m.free_block_count == 16 and m.block_table(7) == ()
    with pytest.raises(RuntimeError):
        step.append_metadata(7, 0, 10)
    # Real step, then growth across a block boundary.
    step = m.stage(1, [BlockAppend(7, 0, 10)])
    step.go_live()
    step.writes_done()
    assert m.valid_token_count(7) == 10 and m.table_length(7) == 3
    step = m.stage(2, [BlockAppend(7, 10, 5)])
    ids, slots = step.append_metadata(7, 10, 5)
    assert len(ids) == 4 and list(slots) == _slots(ids, 10, 15, bs)
    step.go_live()
    step.writes_done()
    with pytest.raises(ValueError, match="starts at"):
        m.stage(3, [BlockAppend(7, 14, 1)])
    m.release_request(7)
    assert m.free_block_count == 16


def test_stage_refuses_when_the_pool_is_short_and_keeps_nothing():
    m = BlockManager(block_size=4, num_blocks=3, enable_prefix_caching=False)
    assert m.stage(0, [BlockAppend(1, 0, 8), BlockAppend(2, 0, 5)]) is None
    assert m.free_block_count == 3
    assert m.stage(0, [BlockAppend(1, 0, 12)]) is not None


def test_prefix_blocks_are_indexed_shared_and_swapped_to_one_copy():
    bs = 4
    m = BlockManager(block_size=bs, num_blocks=32)
    prompt = list(range(100, 111))  # 11 tokens: 2 reusable blocks
    cache = m.prefix_cache
    assert cache.lookup(1, prompt) == ()
    for rid in (1, 2):  # two requests compute the same prefix independently
        step = m.stage(rid, [BlockAppend(rid, 0, len(prompt))])
        step.go_live()
        step.writes_done()
        m.publish_blocks(rid, lambda a, b: prompt[a:b], len(prompt))
    t1, t2 = m.block_table(1), m.block_table(2)
    assert t1[:2] == t2[:2]          # request 2's copies were swapped out
    assert t1[2] != t2[2]            # the partial block stays private
    assert m.free_block_count == 32 - 4
    hit = cache.lookup(3, prompt + [5, 6])
    assert hit == t1[:2]
    # The next chunk completes block 2 (13 tokens: 3 reusable blocks).
    assert cache.chunk_digest(3, prompt + [5, 6], len(hit) * bs, 8) == \
        block_digests(prompt + [5, 6], bs)[2]
    assert cache.chunk_digest(3, prompt + [5, 6], 12, 8) is None
    step = m.stage(10, [BlockAppend(3, 8, 5, prefix=hit)])
    step.go_live()
    step.writes_done()
    assert cache.hits == 1 and cache.hit_tokens == 8
    assert m.block_table(3)[:2] == hit
    for rid in (1, 2, 3):
        m.release_request(rid)
    assert m.free_block_count == 32 and m.pool.cached_block_count == 2


def test_digests_chain_over_the_whole_prefix():
    a = block_digests([1, 2, 3, 4, 5, 6, 7, 8], 4)
    b = block_digests([9, 2, 3, 4, 5, 6, 7, 8], 4)
    assert len(a) == 2 and a[0] != b[0] and a[1] != b[1]  # same second block, other prefix
    assert block_digests([5, 6, 7, 8], 4, parent=a[0]) == a[1:]


def test_teardown_releases_every_table_and_forgets_prefixes():
    m = BlockManager(block_size=4, num_blocks=8)
    step = m.stage(0, [BlockAppend(1, 0, 9)])
    step.go_live()
    step.writes_done()
    m.publish_blocks(1, lambda a, b: list(range(a, b)), 9)
    live = m.stage(1, [BlockAppend(1, 9, 4)])
    live.go_live()
    m.teardown()
    assert live.phase == StepKV.FAILED
    assert m.free_block_count == 8 and m.pool.cached_block_count == 0
    assert m.block_table(1) == () and isinstance(BlockRef(0, 0), BlockRef)
    assert np.all(m.pool._holders == 0)


def test_table_epochs_change_only_when_an_entry_may_be_replaced():
    """Growth keeps a request's table epoch (readers append), a prefix swap
    or a new request gets a new one (readers re-read the whole table)."""
    bs = 4
    m = BlockManager(block_size=bs, num_blocks=32)
    prompt = list(range(200, 209))  # 9 tokens: 2 full blocks
    epochs = {}
    for rid in (1, 2):
        step = m.stage(rid, [BlockAppend(rid, 0, len(prompt))])
        epochs[rid] = step.table_epoch(rid)
        step.go_live()
        step.writes_done()
    assert epochs[1] != epochs[2]
    step = m.stage(5, [BlockAppend(1, 9, 4)])  # growth into a new block
    assert step.table_epoch(1) == epochs[1]
    step.go_live()
    step.writes_done()
    m.publish_blocks(1, lambda a, b: (prompt + [0] * 8)[a:b], len(prompt))
    m.publish_blocks(2, lambda a, b: prompt[a:b], len(prompt))  # swaps to 1's blocks
    step = m.stage(6, [BlockAppend(1, 13, 1), BlockAppend(2, 9, 1)])
    assert step.table_epoch(1) == epochs[1]      # request 1 kept its own blocks
    assert step.table_epoch(2) != epochs[2]      # request 2's entries were replaced
    step.undo()
