"""The host KV ledger under seeded random step sequences (CPU): requests
arrive (some attaching cached prefixes), grow by chunks and single decode
tokens, publish full blocks, finish; steps are committed or undone, and some
are refused for want of blocks. After every operation: each request's write
slots equal the oracle's closed form over its table
(``slot = table[p // bs] * bs + p % bs``), tables never share a block
except cached prefix blocks, every block is free, cached or held (no leak),
a refused step leaves the ledger exactly as it was, an undone one leaves
the tables and the free count as they were (evicted cache entries stay
evicted, as in the reference), and releasing everything returns the pool to
full."""
import random

import numpy as np
import pytest

from oracle import paged_kv as OK
from tinyvllm.cache import BlockAppend, BlockManager


def _snapshot(m: BlockManager, rids):
    return (m.free_block_count,
            {r: (m.block_table(r), m.valid_token_count(r)) for r in rids})


def _unchanged(m: BlockManager, rids, before, cached_before) -> None:
    """Free count and tables as before. A staged allocation may have evicted
    idle cached blocks; like the reference's rollback (cache.py:125-134),
    undo returns them blank and does not restore their cache entries."""
    assert _snapshot(m, rids) == before
    assert m.pool.cached_block_count <= cached_before


def _check(m: BlockManager, live: dict, num_blocks: int) -> None:
    owners: dict[int, set] = {}
    for rid in live:
        table = [ref.block_id for ref in m.block_table(rid)]
        assert len(table) == m.blocks_for(m.valid_token_count(rid)), rid
        assert len(set(table)) == len(table), rid
        for b in table:
            owners.setdefault(b, set()).add(rid)
    # A block in several tables is a shared cached prefix block, held once
    # per table; every block is either held by a table or idle (blank or
    # cached), which is what the free count counts.
    for b, rids in owners.items():
        assert m.pool.held(m.pool.ref(b)) == len(rids), b
    assert len(owners) + m.free_block_count == num_blocks


@pytest.mark.parametrize("seed", range(12))
@pytest.mark.parametrize("prefix_caching", [False, True])
def test_random_step_sequences_keep_the_ledger_consistent(seed, prefix_caching):
    r = random.Random(seed)
    bs = r.choice([1, 2, 4, 16])
    num_blocks = r.choice([24, 64, 200])
    m = BlockManager(block_size=bs, num_blocks=num_blocks,
                     enable_prefix_caching=prefix_caching)
    # A few shared prompt heads so prefix hits happen.
    heads = [[r.randrange(1000) for _ in range(r.randint(1, 4) * bs)] for _ in range(3)]
    live: dict[int, list[int]] = {}   # request -> token ids known so far
    next_rid = 0
    for plan in range(300):
        op = r.random()
        if op < 0.15 and live:
            rid = r.choice(list(live))
            m.release_request(rid)
            del live[rid]
        else:
            appends, tokens_of = [], {}
            for rid in r.sample(list(live), min(len(live), r.randint(0, 4))):
                have = m.valid_token_count(rid)
                n = 1 if r.random() < 0.6 else r.randint(1, 3 * bs)
                appends.append(BlockAppend(rid, have, n))
                tokens_of[rid] = live[rid] + [r.randrange(1000) for _ in range(n)]
            if r.random() < 0.5 or not appends:
                rid, next_rid = next_rid, next_rid + 1
                prompt = list(r.choice(heads)) + [r.randrange(1000)
                                                  for _ in range(r.randint(1, 3 * bs))]
                hit = m.prefix_cache.lookup(rid, prompt) if prefix_caching else ()
                start = len(hit) * bs
                appends.append(BlockAppend(rid, start, r.randint(1, len(prompt) - start)
                                           if len(prompt) > start else 1, prefix=hit))
                tokens_of[rid] = prompt + [r.randrange(1000)] * max(
                    0, start + appends[-1].query_len - len(prompt))
            known = set(live)
            before = _snapshot(m, known)
            cached_before = m.pool.cached_block_count
            step = m.stage(plan, appends)
            if step is None:  # refused: nothing changed
                assert _snapshot(m, known) == before
                assert m.pool.cached_block_count == cached_before
                continue
            # Write slots: the oracle's closed form over the staged table,
            # unique and inside the pool.
            slots_all = []
            for a in appends:
                ids, slots = step.append_metadata(a.request_id, a.token_start, a.query_len)
                expect = OK.slot_mapping(ids, a.token_start, a.token_start + a.query_len, bs)
                assert np.array_equal(slots, expect), (plan, a)
                assert len(ids) == m.blocks_for(a.token_start + a.query_len)
                slots_all.extend(slots.tolist())
            assert len(set(slots_all)) == len(slots_all)
            assert all(0 <= s < num_blocks * bs for s in slots_all)
            if r.random() < 0.2:
                step.undo()
                _unchanged(m, known, before, cached_before)
                continue
            step.go_live()
            step.writes_done()
            for a in appends:
                live[a.request_id] = tokens_of[a.request_id]
                assert m.valid_token_count(a.request_id) == a.token_start + a.query_len
            if prefix_caching:
                for a in appends:
                    toks = live[a.request_id]
                    m.publish_blocks(a.request_id, lambda x, y, t=toks: t[x:y],
                                     min(len(toks), m.valid_token_count(a.request_id)))
        _check(m, live, num_blocks)
    if prefix_caching:
        assert m.prefix_cache.hits > 0  # the sequence exercised shared prefixes
    for rid in list(live):
        m.release_request(rid)
    assert m.free_block_count == num_blocks
