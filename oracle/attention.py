"""Paged attention restated on the CPU in fp32 (test infrastructure only).

Reference: tinyvllm/runtime/attention.py:102-151 (SDPAAttention._attend:
gather each row's K/V in logical order with PagedKVCache.read, then
F.scaled_dot_product_attention with enable_gqa; fresh rows use is_causal,
chunked rows the lower-right causal mask of :176-214) and
tinyvllm/kernels/paged_decode.cu:92-466 (decode rows; zero-length rows give
zeros, :130-135).

The softmax is computed in fp32 from the stored (bf16/fp16) values and the
result is rounded once to the storage type.
"""
from __future__ import annotations

import torch

from oracle.paged_kv import read_slots


def _attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
            allowed: torch.Tensor | None) -> torch.Tensor:
    """q [Lq, Hq, D], k/v [Lk, Hkv, D] (fp32) -> [Lq, Hq, D] fp32, GQA by
    repeating each KV head over its Hq/Hkv query heads."""
    group = q.shape[1] // k.shape[1]
    k = k.repeat_interleave(group, dim=1)
    v = v.repeat_interleave(group, dim=1)
    scores = torch.einsum("qhd,khd->hqk", q, k) * scale
    if allowed is not None:
        scores = scores.masked_fill(~allowed[None], float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    return torch.einsum("hqk,khd->qhd", probs, v)


def decode_attention(q, key_cache, value_cache, rows, blocks, offsets, lengths,
                     block_size: int, scale: float, output: torch.Tensor) -> None:
    """Fill output[rows[r]] with single-query paged attention (in place)."""
    for r in range(rows.numel()):
        row, length = int(rows[r]), int(lengths[r])
        if length == 0:
            output[row].zero_()
            continue
        table = blocks[int(offsets[r]):int(offsets[r + 1])]
        slots = read_slots(table, length, block_size)
        k = key_cache.index_select(0, slots).float()
        v = value_cache.index_select(0, slots).float()
        out = _attend(q[row:row + 1].float(), k, v, scale, None)
        output[row] = out[0].to(output.dtype)


def prefill_attention(q, key_cache, value_cache, q_offsets, blocks, block_offsets,
                      context_lens, block_size: int, scale: float,
                      output: torch.Tensor) -> None:
    """Chunked prefill: item i's queries q[q_offsets[i]:q_offsets[i+1]] are
    the last tokens of its context; query j sees t <= ctx - qlen + j."""
    for i in range(context_lens.numel()):
        start, end = int(q_offsets[i]), int(q_offsets[i + 1])
        qlen, ctx = end - start, int(context_lens[i])
        if qlen <= 0:
            continue
        table = blocks[int(block_offsets[i]):int(block_offsets[i + 1])]
        slots = read_slots(table, ctx, block_size)
        k = key_cache.index_select(0, slots).float()
        v = value_cache.index_select(0, slots).float()
        qpos = torch.arange(ctx - qlen, ctx)[:, None]
        allowed = torch.arange(ctx)[None, :] <= qpos
        out = _attend(q[start:end].float(), k, v, scale, allowed)
        output[start:end] = out.to(output.dtype)


def textbook_attention_f64(q, k, v, scale: float, causal_offset: int | None = None):
    """Loop-form softmax attention in float64 for tiny inputs (the pin).

    q [Lq, Hq, D], k/v [Lk, Hkv, D]; when causal_offset is given, query j
    sees keys t <= causal_offset + j."""
    lq, hq, d = q.shape
    lk, hkv, _ = k.shape
    group = hq // hkv
    out = torch.zeros(lq, hq, d, dtype=torch.float64)
    q, k, v = q.double(), k.double(), v.double()
    for j in range(lq):
        for h in range(hq):
            kh = h // group
            limit = lk if causal_offset is None else min(lk, causal_offset + j + 1)
            s = [float(scale * sum(q[j, h, x] * k[t, kh, x] for x in range(d)))
                 for t in range(limit)]
            m = max(s)
            e = [pow(2.718281828459045, si - m) for si in s]
            z = sum(e)
            for x in range(d):
                out[j, h, x] = sum(e[t] * float(v[t, kh, x]) for t in range(limit)) / z
    return out
