"""Pins for oracle/paged_kv.py: closed form, brute force, bit copies, sentinel."""
import numpy as np
import torch

from oracle import paged_kv as O


def test_slot_closed_form_matches_brute_force():
    rng = np.random.default_rng(0)
    for block_size in (1, 3, 16, 32):
        pool = rng.permutation(64)
        table = pool[:10]
        # Brute force: enumerate the physical pool in block order and assign
        # logical positions by walking the table.
        physical = {}
        pos = 0
        for block in table:
            for off in range(block_size):
                physical[pos] = int(block) * block_size + off
                pos += 1
        for p in range(len(table) * block_size):
            assert O.slot_for_position(table, p, block_size) == physical[p]


def test_read_slots_in_logical_order():
    table = [7, 2, 5]
    slots = O.read_slots(table, 40, 16)
    assert slots.tolist() == [7 * 16 + i for i in range(16)] + \
        [2 * 16 + i for i in range(16)] + [5 * 16 + i for i in range(8)]


def test_write_is_bitwise_and_sentinel_skips():
    g = torch.Generator().manual_seed(1)
    kc = torch.full((64, 2, 8), -7.0).to(torch.bfloat16)
    vc = torch.full((64, 2, 8), 3.0).to(torch.bfloat16)
    k = torch.randn(5, 2, 8, generator=g).to(torch.bfloat16)
    v = torch.randn(5, 2, 8, generator=g).to(torch.bfloat16)
    slots = torch.tensor([9, -1, 0, 63, 17])
    O.kv_write(kc, vc, slots, k, v)
    for t, s in enumerate(slots.tolist()):
        if s >= 0:
            assert torch.equal(kc[s].view(torch.int16), k[t].view(torch.int16))
            assert torch.equal(vc[s].view(torch.int16), v[t].view(torch.int16))
    untouched = [i for i in range(64) if i not in (9, 0, 63, 17)]
    assert (kc[untouched].float() == -7.0).all() and (vc[untouched].float() == 3.0).all()
    rk, rv = O.kv_read(kc, vc, torch.tensor([17, 9]))
    assert torch.equal(rk[0], k[4]) and torch.equal(rv[1], v[0])
