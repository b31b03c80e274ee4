"""The FP8 E4M3 KV layout's oracle, pinned against the format's definition.

The layout has no reference counterpart; ``oracle/paged_kv.py`` defines it as
nearest-even E4M3 of clamp(x / scale, +-448). The oracle's quantiser uses
torch's float8_e4m3fn cast; these tests check that cast against a brute-force
nearest-value search over the closed-form code table, ties to the even code,
and check the decode table against the textbook definition."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_kv as OK


def test_e4m3_closed_form_matches_torch_decode():
    table = OK.e4m3_table()
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    finite = np.isfinite(table)
    assert np.array_equal(np.isnan(table), np.isnan(codes))
    assert np.array_equal(table[finite], codes[finite])
    # Landmarks of the format: max 448, min normal 2^-6, min subnormal 2^-9.
    assert np.nanmax(table) == 448.0 and table[0x7E] == 448.0
    assert table[0x08] == 2.0 ** -6 and table[0x01] == 2.0 ** -9
    assert np.isnan(table[0x7F]) and np.isnan(table[0xFF]) and not np.isinf(table).any()


def _brute_force(x: np.ndarray) -> np.ndarray:
    """Nearest finite E4M3 code of each (already clamped) float32 value; ties
    go to the code with the even mantissa; signed zero keeps its sign."""
    table = OK.e4m3_table()
    codes = np.array([c for c in range(256) if np.isfinite(table[c])])
    values = table[codes]
    out = np.empty(x.shape, dtype=np.uint8)
    for i, v in enumerate(x.astype(np.float64)):
        d = np.abs(values - v)
        best = np.flatnonzero(d == d.min())
        if len(best) > 1:  # a tie: +-0 (the sign of v) or a midpoint (even code)
            if values[best[0]] == 0.0:
                out[i] = 0x80 if np.signbit(v) else 0x00
                continue
            best = [b for b in best if codes[b] % 2 == 0]
        out[i] = codes[best[0]]
    return out


def test_quantize_is_nearest_even_with_saturation():
    g = torch.Generator().manual_seed(3)
    table = OK.e4m3_table()
    finite = np.unique(table[np.isfinite(table)])
    mids = (finite[1:] + finite[:-1]) / 2
    x = torch.cat([
        torch.randn(3000, generator=g) * 0.01, torch.randn(3000, generator=g) * 3,
        torch.randn(1000, generator=g) * 300, torch.tensor(mids), torch.tensor(-mids),
        torch.tensor([448.0, 449.0, 464.0, 1e6, -1e6, 0.0, -0.0, 2.0 ** -10, 3 * 2.0 ** -11]),
    ]).float()
    got = OK.fp8_quantize(x, 1.0).numpy()
    want = _brute_force(np.clip(x.numpy(), -448.0, 448.0))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("scale", [1.0, 0.25, 3.0])
def test_scaled_round_trip_error_bound(scale):
    """|dequant(quant(x)) - x| <= half an E4M3 step (relative 2^-4 for normal
    values, 2^-10 * scale absolute below the normal range)."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(20000, generator=g) * 4 * scale
    y = OK.fp8_dequantize(OK.fp8_quantize(x, scale), scale)
    err = (y - x).abs()
    bound = torch.maximum(x.abs() * 2.0 ** -4, torch.full_like(x, 2.0 ** -10 * scale))
    assert (err <= bound * 1.0001).all()
    # scale folds exactly out of power-of-two scalings
    if scale == 0.25:
        assert torch.equal(OK.fp8_quantize(x, scale), OK.fp8_quantize(x * 4, 1.0))


def test_cpu_cache_read_dequantises():
    from tinyvllm.paged_kv import PagedKVCache

    cache = PagedKVCache(num_layers=1, num_blocks=2, block_size=4, num_kv_heads=2,
                         head_dim=8, device="cpu", dtype=torch.float8_e4m3fn,
                         k_scale=0.5, v_scale=2.0)
    g = torch.Generator().manual_seed(1)
    k = torch.randn(8, 2, 8, generator=g)
    v = torch.randn(8, 2, 8, generator=g)
    cache.key[0].view(torch.uint8).copy_(OK.fp8_quantize(k, 0.5))
    cache.value[0].view(torch.uint8).copy_(OK.fp8_quantize(v, 2.0))
    slots = torch.tensor([5, 0, 7])
    rk, rv = cache.read(0, slots)
    assert rk.dtype == torch.float32
    assert torch.equal(rk, OK.fp8_dequantize(OK.fp8_quantize(k, 0.5), 0.5)[slots])
    assert torch.equal(rv, OK.fp8_dequantize(OK.fp8_quantize(v, 2.0), 2.0)[slots])
    with pytest.raises(ValueError, match="FP8 cache only"):
        PagedKVCache(num_layers=1, num_blocks=1, block_size=4, num_kv_heads=1, head_dim=8,
                     device="cpu", dtype=torch.bfloat16, k_scale=2.0)
    with pytest.raises(ValueError, match="positive finite"):
        PagedKVCache(num_layers=1, num_blocks=1, block_size=4, num_kv_heads=1, head_dim=8,
                     device="cpu", dtype=torch.float8_e4m3fn, v_scale=0.0)
