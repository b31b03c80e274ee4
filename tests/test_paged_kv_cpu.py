"""PagedKVCache storage layouts on the CPU: both keep the reference's
[layers, slots, kv_heads, head_dim] view (reference paged_kv.py:53-65); the
default stores each KV head's slots contiguously underneath."""
import pytest
import torch

from tinyvllm.paged_kv import PagedKVCache


def _cache(layout, **kw):
    return PagedKVCache(num_layers=3, num_blocks=4, block_size=8, num_kv_heads=2,
                        head_dim=16, device="cpu", dtype=torch.bfloat16, layout=layout, **kw)


def test_views_keep_the_reference_shape():
    hm, tm = _cache("head_major"), _cache("token_major")
    for cache in (hm, tm):
        assert cache.key.shape == cache.value.shape == (3, 32, 2, 16)
    # head-major: a head's 32 slots are one contiguous [32, 16] block
    assert hm.key[1].stride() == (16, 32 * 16, 1)
    assert hm.key[1][:, 1].is_contiguous()
    assert tm.key[1].stride() == (2 * 16, 16, 1) and tm.key.is_contiguous()
    assert hm.key.untyped_storage().data_ptr() != hm.value.untyped_storage().data_ptr()
    assert PagedKVCache(num_layers=1, num_blocks=1, block_size=4, num_kv_heads=1,
                        head_dim=8, device="cpu", dtype=torch.float16).layout == "token_major"


def test_read_gathers_the_same_rows_in_both_layouts():
    g = torch.Generator().manual_seed(0)
    values = torch.randn(3, 32, 2, 16, generator=g).to(torch.bfloat16)
    slots = torch.tensor([31, 0, 7, 8, 8])
    rows = []
    for layout in ("head_major", "token_major"):
        cache = _cache(layout)
        cache.key.copy_(values)
        cache.value.copy_(-values)
        k, v = cache.read(2, slots)
        assert torch.equal(k, values[2, slots]) and torch.equal(v, -values[2, slots])
        rows.append(k)
    assert torch.equal(rows[0], rows[1])


def test_unknown_layout_is_rejected():
    with pytest.raises(ValueError, match="layout"):
        _cache("slot_major")


def test_auto_layout_follows_the_decode_parallelism():
    from tinyvllm.paged_kv import resolve_layout

    assert resolve_layout("auto", 64, 8) == "token_major"   # 8B bs64: 512 pairs
    assert resolve_layout("auto", 16, 8) == "head_major"    # 32B, 16 long rows
    assert resolve_layout("auto", 31, 8) == "head_major"
    assert resolve_layout("auto", 32, 8) == "token_major"
    assert resolve_layout("head_major", 64, 8) == "head_major"
    with pytest.raises(ValueError, match="layout"):
        resolve_layout("slot_major", 1, 1)
