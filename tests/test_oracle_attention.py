"""Pins for oracle/attention.py against float64 loops, torch SDPA and closed forms."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as A
from oracle import paged_kv as PK
from helpers import paged_decode_case


def _dense(case, r):
    table = case["blocks"][case["offsets"][r]:case["offsets"][r + 1]]
    slots = PK.read_slots(table, int(case["lengths"][r]), case["block_size"])
    return case["k"].index_select(0, slots), case["v"].index_select(0, slots)


@pytest.mark.parametrize("heads,kv_heads", [(4, 2), (2, 2), (4, 1)])
def test_decode_matches_float64_textbook(heads, kv_heads):
    case = paged_decode_case(seed=3, batch=3, heads=heads, kv_heads=kv_heads, head_dim=8,
                             block_size=4, pool_blocks=32, lengths=[5, 1, 9],
                             dtype=torch.float32)
    out = torch.zeros_like(case["q"])
    A.decode_attention(case["q"], case["k"], case["v"], case["rows"], case["blocks"],
                       case["offsets"], case["lengths"], 4, case["scale"], out)
    for r in range(3):
        k, v = _dense(case, r)
        ref = A.textbook_attention_f64(case["q"][r:r + 1], k, v, case["scale"])
        assert torch.allclose(out[r:r + 1].double(), ref, atol=1e-6, rtol=1e-5)


def test_decode_matches_torch_sdpa_gqa():
    case = paged_decode_case(seed=4, batch=4, heads=16, kv_heads=8, pool_blocks=256,
                             min_len=1, max_len=300, dtype=torch.float32)
    out = torch.zeros_like(case["q"])
    A.decode_attention(case["q"], case["k"], case["v"], case["rows"], case["blocks"],
                       case["offsets"], case["lengths"], 16, case["scale"], out)
    for r in range(4):
        k, v = _dense(case, r)
        ref = F.scaled_dot_product_attention(
            case["q"][r:r + 1].transpose(0, 1).unsqueeze(0), k.transpose(0, 1).unsqueeze(0),
            v.transpose(0, 1).unsqueeze(0), scale=case["scale"], enable_gqa=True,
        ).squeeze(0).transpose(0, 1)
        assert torch.allclose(out[r:r + 1], ref, atol=1e-5, rtol=1e-4)


def test_decode_special_cases():
    case = paged_decode_case(seed=5, batch=3, heads=2, kv_heads=1, head_dim=16,
                             block_size=4, pool_blocks=16, lengths=[1, 6, 0],
                             dtype=torch.float32)
    # Row 1: identical keys -> uniform weights -> mean of V.
    table = case["blocks"][case["offsets"][1]:case["offsets"][2]]
    slots = PK.read_slots(table, 6, 4)
    case["k"][slots] = case["k"][slots[0]].clone()
    out = torch.full_like(case["q"], 99.0)
    A.decode_attention(case["q"], case["k"], case["v"], case["rows"], case["blocks"],
                       case["offsets"], case["lengths"], 4, case["scale"], out)
    s0 = PK.read_slots(case["blocks"][0:1], 1, 4)[0]
    assert torch.allclose(out[0], case["v"][s0].expand(2, 16))          # L = 1 -> V
    assert torch.allclose(out[1], case["v"][slots].mean(0).expand(2, 16), atol=1e-6)
    assert (out[2] == 0).all()                                           # L = 0 -> 0


def test_decode_dominant_key_selects_its_value():
    case = paged_decode_case(seed=6, batch=1, heads=1, kv_heads=1, head_dim=8,
                             block_size=4, pool_blocks=8, lengths=[11], dtype=torch.float32)
    table = case["blocks"][0:3]
    slots = PK.read_slots(table, 11, 4)
    case["k"][slots[7]] = case["q"][0] * 1e4
    out = torch.zeros_like(case["q"])
    A.decode_attention(case["q"], case["k"], case["v"], case["rows"], case["blocks"],
                       case["offsets"], case["lengths"], 4, 1.0, out)
    assert torch.allclose(out[0, 0], case["v"][slots[7], 0], atol=1e-6)


def test_prefill_matches_textbook_lower_right_causal():
    g = torch.Generator().manual_seed(7)
    ctx, qlen, hq, hkv, d, bs = 11, 4, 4, 2, 8, 4
    k = torch.randn(64, hkv, d, generator=g)
    v = torch.randn(64, hkv, d, generator=g)
    q = torch.randn(qlen, hq, d, generator=g)
    blocks = torch.tensor([5, 1, 12])
    out = torch.zeros_like(q)
    A.prefill_attention(q, k, v, torch.tensor([0, qlen]), blocks, torch.tensor([0, 3]),
                        torch.tensor([ctx]), bs, d ** -0.5, out)
    slots = PK.read_slots(blocks, ctx, bs)
    ref = A.textbook_attention_f64(q, k[slots], v[slots], d ** -0.5,
                                   causal_offset=ctx - qlen)
    assert torch.allclose(out.double(), ref, atol=1e-6)
    # The last query sees the whole context: equals decode attention.
    dec = torch.zeros(1, hq, d)
    A.decode_attention(q[-1:], k, v, torch.tensor([0]), blocks, torch.tensor([0, 3]),
                       torch.tensor([ctx]), bs, d ** -0.5, dec)
    assert torch.allclose(dec[0], out[-1], atol=1e-6)
