"""Paged decode and chunked prefill against the oracle over seeded random
configurations: GQA groups 1-32, head dims 32-256 (128 on the MFMA
kernels; 32, 36, 64, 96 and 256, and groups above 16, on the general
kernel, 36 through its unvectorised loads), page sizes 1-32
(powers of two and not), bf16 / fp16 queries, bf16 / fp16 / FP8 E4M3
caches, both storage layouts, ragged lengths with empty rows, query rows
picked out of a larger token axis and max_context_len hints above the
longest row; and the fused decode step (QK-norm, RoPE, KV write and
attention in one launch) over the same kind of draw; and sampling (greedy
rows exact, temperature / top-k / top-p draws inside the oracle's kept set)
over vocab sizes around the scan spans, three logit dtypes and tied maxima.
Each configuration comes from its own seed and is printed in
the test id; the bar is the one every attention test uses (max abs 2e-2,
mean relative 1e-3), with empty rows exactly zero. TVLLM_RANDOM_CASES=k
multiplies every case count by k for a longer sweep."""
import math
import os
import random

import pytest
import torch

from helpers import assert_bf16_close
from oracle import attention as OA
from test_gpu_fp8 import _fp8_cache
from test_gpu_kernels import _Cache

pytestmark = pytest.mark.gpu

_SCALE = max(1, int(os.environ.get("TVLLM_RANDOM_CASES", "1")))
DECODE_CASES = 36 * _SCALE
PREFILL_CASES = 26 * _SCALE


def _decode_config(seed: int) -> dict:
    r = random.Random(1000 + seed)
    kv_heads = r.choice([1, 2, 4, 8])
    group = r.choice([1, 2, 3, 4, 5, 8, 16, 20, 32])
    head_dim = r.choice([128, 128, 128, 64, 256, 32, 96, 36])
    cache = r.choice(["same", "same", "fp8"])
    block_size = r.choice([16, 16, 16, 1, 2, 5, 8, 32])
    longest = r.choice([1, 17, 300, 2500, 6000])
    batch = r.randint(1, 12 if longest <= 2500 else 5)
    lengths = [r.randint(0, longest) for _ in range(batch)]
    lengths[r.randrange(batch)] = longest
    if batch > 2 and r.random() < 0.5:
        lengths[r.randrange(batch)] = 0
    return dict(kv_heads=kv_heads, heads=kv_heads * group, head_dim=head_dim, cache=cache,
                block_size=block_size, lengths=lengths,
                dtype=r.choice([torch.bfloat16, torch.float16]),
                layout=r.choice(["head_major", "token_major"]),
                hint=r.choice([None, longest, 2 * longest + 31]),
                extra_rows=r.randint(0, 5), scales=r.choice([(1.0, 1.0), (0.5, 2.0)]))


def _decode_id(seed: int) -> str:
    c = _decode_config(seed)
    return (f"s{seed}-h{c['heads']}kv{c['kv_heads']}-d{c['head_dim']}-bs{c['block_size']}-"
            f"{str(c['dtype'])[6:]}-{c['cache']}-{c['layout']}-L{max(c['lengths'])}x"
            f"{len(c['lengths'])}")


def _tables(g, lengths, block_size):
    pages = [math.ceil(n / block_size) for n in lengths]
    pool = sum(pages) + 3
    perm = torch.randperm(pool, generator=g)
    blocks, offsets = [], [0]
    for p in pages:
        blocks += perm[offsets[-1]:offsets[-1] + p].tolist()
        offsets.append(offsets[-1] + p)
    return pool, torch.tensor(blocks, dtype=torch.long), torch.tensor(offsets, dtype=torch.long)


@pytest.mark.parametrize("seed", range(DECODE_CASES), ids=_decode_id)
def test_decode_random_configuration(device, seed):
    from tinyvllm.kernels.paged_decode import paged_decode_attention
    from tinyvllm.runtime.contracts import SingleQueryMetadata

    c = _decode_config(seed)
    g = torch.Generator().manual_seed(seed)
    bs, d, dt = c["block_size"], c["head_dim"], c["dtype"]
    batch = len(c["lengths"])
    pool, blocks, offsets = _tables(g, c["lengths"], bs)
    k = torch.randn(pool * bs, c["kv_heads"], d, generator=g)
    v = torch.randn(pool * bs, c["kv_heads"], d, generator=g)
    tokens = batch + c["extra_rows"]
    q = torch.randn(tokens, c["heads"], d, generator=g).to(dt)
    rows = torch.randperm(tokens, generator=g)[:batch]
    lengths = torch.tensor(c["lengths"], dtype=torch.long)
    if c["cache"] == "fp8":
        ks, vs = c["scales"]
        cache, kd, vd = _fp8_cache(k * ks, v * vs, bs, device, ks, vs, c["layout"])
    else:
        kd, vd = k.to(dt), v.to(dt)
        cache = _Cache(kd.to(device), vd.to(device), bs, layout=c["layout"])
    meta = SingleQueryMetadata(rows.to(device), blocks.to(device), offsets.to(device),
                               lengths.to(device), c["hint"])
    scale = d ** -0.5
    out = torch.full(q.shape, 7.0, dtype=dt, device=device)
    paged_decode_attention(q.to(device), cache, 0, meta, out, scale=scale)
    torch.cuda.synchronize()
    expect = torch.full(q.shape, 7.0, dtype=dt)
    OA.decode_attention(q, kd, vd, rows, blocks, offsets, lengths, bs, scale, expect)
    out = out.cpu()
    for i, n in enumerate(c["lengths"]):
        if n == 0:
            assert (out[rows[i]] == 0).all(), f"empty row {i} not zero"
    untouched = torch.ones(tokens, dtype=torch.bool)
    untouched[rows] = False
    assert (out[untouched] == 7.0).all(), "rows outside query_rows were written"
    assert_bf16_close(out, expect)


def _prefill_config(seed: int) -> dict:
    r = random.Random(2000 + seed)
    kv_heads = r.choice([1, 2, 4, 8])
    group = r.choice([1, 2, 4, 8, 16, 24])
    head_dim = r.choice([128, 128, 128, 64, 256, 32, 96, 36])
    items = []
    for _ in range(r.randint(1, 6)):
        q_len = r.choice([1, r.randint(2, 40), r.randint(41, 300), 512])
        history = r.choice([0, 0, r.randint(1, 200), r.randint(200, 3000)])
        items.append((history + q_len, q_len))
    return dict(kv_heads=kv_heads, heads=kv_heads * group, items=items, head_dim=head_dim,
                block_size=r.choice([16, 16, 1, 4, 5, 8, 12, 32]),
                cache=r.choice(["bf16", "bf16", "fp16", "fp8"]),
                layout=r.choice(["head_major", "token_major"]))


def _prefill_id(seed: int) -> str:
    c = _prefill_config(seed)
    return (f"s{seed}-h{c['heads']}kv{c['kv_heads']}-d{c['head_dim']}-bs{c['block_size']}-"
            f"{c['cache']}-{c['layout']}-{len(c['items'])}items-q{sum(q for _, q in c['items'])}")


@pytest.mark.parametrize("seed", range(PREFILL_CASES), ids=_prefill_id)
def test_prefill_random_configuration(device, seed):
    from tinyvllm.kernels.paged_prefill import paged_prefill_attention
    from tinyvllm.runtime.contracts import MultiQueryMetadata

    c = _prefill_config(seed)
    g = torch.Generator().manual_seed(seed)
    bs, d = c["block_size"], c["head_dim"]
    contexts = [ctx for ctx, _ in c["items"]]
    pool, blocks, boffsets = _tables(g, contexts, bs)
    k = torch.randn(pool * bs, c["kv_heads"], d, generator=g)
    v = torch.randn(pool * bs, c["kv_heads"], d, generator=g)
    dt = torch.float16 if c["cache"] == "fp16" else torch.bfloat16
    q_offsets = torch.tensor([0] + [sum(q for _, q in c["items"][:i + 1])
                                    for i in range(len(c["items"]))], dtype=torch.long)
    q = torch.randn(int(q_offsets[-1]), c["heads"], d, generator=g).to(dt)
    if c["cache"] == "fp8":
        cache, kd, vd = _fp8_cache(k * 0.5, v, bs, device, 0.5, 1.0, c["layout"])
    else:
        kd, vd = k.to(dt), v.to(dt)
        cache = _Cache(kd.to(device), vd.to(device), bs, layout=c["layout"])
    context = torch.tensor(contexts, dtype=torch.long)
    meta = MultiQueryMetadata(q_offsets.to(device), blocks.to(device), boffsets.to(device),
                              context.to(device), max_query_len=max(q for _, q in c["items"]))
    out = torch.zeros(q.shape, dtype=dt, device=device)
    paged_prefill_attention(q.to(device), cache, 0, meta, out, scale=d ** -0.5)
    torch.cuda.synchronize()
    expect = torch.zeros_like(q)
    OA.prefill_attention(q, kd, vd, q_offsets, blocks, boffsets, context, bs, d ** -0.5,
                         expect)
    assert_bf16_close(out.cpu(), expect)


FUSED_CASES = 12 * _SCALE


def _fused_config(seed: int) -> dict:
    r = random.Random(3000 + seed)
    kv_heads = r.choice([1, 2, 4, 8])
    longest = r.choice([1, 40, 900, 3000, 12000])
    batch = r.randint(1, 10 if longest <= 3000 else 3)
    lengths = [r.randint(0, longest) for _ in range(batch)]
    lengths[r.randrange(batch)] = longest
    return dict(kv_heads=kv_heads, heads=kv_heads * r.choice([1, 2, 4, 5, 8, 16]),
                lengths=lengths, block_size=r.choice([16, 16, 8, 32, 5]),
                fp8=r.random() < 0.3, layout=r.choice(["head_major", "token_major"]),
                hint=r.choice([None, longest, 4 * longest + 7]))


def _fused_id(seed: int) -> str:
    c = _fused_config(seed)
    return (f"s{seed}-h{c['heads']}kv{c['kv_heads']}-bs{c['block_size']}-"
            f"{'fp8' if c['fp8'] else 'bf16'}-{c['layout']}-L{max(c['lengths'])}x"
            f"{len(c['lengths'])}")


@pytest.mark.parametrize("seed", range(FUSED_CASES), ids=_fused_id)
def test_fused_decode_step_random_configuration(device, seed):
    """The fused decode step (QK-norm + RoPE + the new token's K/V write +
    attention) against the unfused kernels (cache bytes bit-identical) and
    the oracle of the whole step (attention output at the bar)."""
    from oracle import paged_kv as OK
    from oracle import pointwise as OP
    from tinyvllm.kernels.paged_decode import paged_decode_qk_norm_rope
    from tinyvllm.kernels.pointwise import qk_norm_rope_store
    from tinyvllm.runtime.contracts import SingleQueryMetadata

    c = _fused_config(seed)
    g = torch.Generator().manual_seed(seed)
    bs, d, heads, hkv = c["block_size"], 128, c["heads"], c["kv_heads"]
    lengths = c["lengths"]
    rows = len(lengths)
    pool, blocks, offsets = _tables(g, [max(n, 1) for n in lengths], bs)
    slots = [int(blocks[offsets[r] + (n - 1) // bs]) * bs + (n - 1) % bs if n > 0 else -1
             for r, n in enumerate(lengths)]
    ks, vs = (0.5, 0.25) if c["fp8"] else (1.0, 1.0)
    k_init = torch.randn(pool * bs, hkv, d, generator=g) * ks
    v_init = torch.randn(pool * bs, hkv, d, generator=g) * vs
    qkv = torch.randn(rows, (heads + 2 * hkv) * d, generator=g).to(torch.bfloat16)
    qw = (1 + 0.05 * torch.randn(d, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.05 * torch.randn(d, generator=g)).to(torch.bfloat16)
    cos, sin = OP.rope_tables(torch.tensor([max(n - 1, 0) for n in lengths]), d, 1e6,
                              torch.bfloat16)

    def cache():
        if c["fp8"]:
            return _fp8_cache(k_init, v_init, bs, device, ks, vs, c["layout"])[0]
        return _Cache(k_init.to(torch.bfloat16).to(device), v_init.to(torch.bfloat16).to(device),
                      bs, layout=c["layout"])

    G = lambda t: t.to(device)  # noqa: E731
    gqkv = G(qkv)
    q = gqkv[:, :heads * d].view(rows, heads, d)
    k = gqkv[:, heads * d:(heads + hkv) * d].view(rows, hkv, d)
    v = gqkv[:, (heads + hkv) * d:].view(rows, hkv, d)
    gslots = G(torch.tensor(slots))
    meta = SingleQueryMetadata(G(torch.arange(rows)), G(blocks), G(offsets),
                               G(torch.tensor(lengths)), c["hint"])
    cache_a = cache()
    qk_norm_rope_store(q, k, v, G(qw), G(kw), G(cos), G(sin), 1e-6, 1e-6,
                       cache_a.key[0], cache_a.value[0], gslots, k_scale=ks, v_scale=vs)
    cache_b = cache()
    out = torch.full((rows, heads, d), 7.0, dtype=torch.bfloat16, device=device)
    paged_decode_qk_norm_rope(q, k, v, G(qw), G(kw), G(cos), G(sin), 1e-6, 1e-6,
                              cache_b, 0, meta, gslots, out, scale=d ** -0.5)
    torch.cuda.synchronize()
    for name in ("key", "value"):
        a = getattr(cache_a, name)[0].cpu().view(torch.uint8)
        b = getattr(cache_b, name)[0].cpu().view(torch.uint8)
        assert torch.equal(a, b), f"{name} cache bytes differ from the unfused write"
    # The oracle of the whole step attends over the cache as the step left it
    # (its new rows are the unfused kernels' bytes, pinned above).
    if c["fp8"]:
        kd = OK.fp8_dequantize(cache_b.key[0].cpu().view(torch.uint8), ks)
        vd = OK.fp8_dequantize(cache_b.value[0].cpu().view(torch.uint8), vs)
    else:
        kd, vd = cache_b.key[0].cpu(), cache_b.value[0].cpu()
    q_ref, _ = OP.qk_norm_rope(qkv[:, :heads * d].view(rows, heads, d),
                               qkv[:, heads * d:(heads + hkv) * d].view(rows, hkv, d),
                               qw, kw, cos, sin)
    expect = torch.zeros(rows, heads, d, dtype=torch.bfloat16)
    OA.decode_attention(q_ref, kd, vd, torch.arange(rows), blocks, offsets,
                        torch.tensor(lengths), bs, d ** -0.5, expect)
    assert_bf16_close(out.cpu(), expect)
    for r, n in enumerate(lengths):
        if n == 0:
            assert (out[r].cpu() == 0).all()


SAMPLING_CASES = 16 * _SCALE


def _sampling_config(seed: int) -> dict:
    r = random.Random(5000 + seed)
    vocab = r.choice([1, 7, 1000, 8191, 8192, 8193, 32000, 151936, 151939])
    rows = r.randint(1, 8)
    return dict(vocab=vocab, rows=rows, dtype=r.choice(["bf16", "fp16", "fp32"]),
                scale=r.choice([0.5, 2.0, 8.0]),
                temperature=[r.choice([0.0, 0.0, 0.3, 1.0, 1.7]) for _ in range(rows)],
                top_k=[r.choice([0, 0, 1, 5, 50, vocab]) for _ in range(rows)],
                top_p=[r.choice([1.0, 1.0, 0.95, 0.5, 0.01]) for _ in range(rows)])


def _sampling_id(seed: int) -> str:
    c = _sampling_config(seed)
    return f"s{seed}-V{c['vocab']}-R{c['rows']}-{c['dtype']}-x{c['scale']}"


@pytest.mark.parametrize("seed", range(SAMPLING_CASES), ids=_sampling_id)
def test_sampling_random_configuration(device, seed):
    """Greedy rows (temperature 0) equal the first index of the maximum;
    every other row's draws, over several noise counters, stay inside the
    oracle's float64 top-k / top-p kept set."""
    from oracle import sampling as OS
    from tinyvllm.kernels.sampling import argmax, sample

    c = _sampling_config(seed)
    g = torch.Generator().manual_seed(seed)
    dt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[c["dtype"]]
    rows, vocab = c["rows"], c["vocab"]
    logits = (c["scale"] * torch.randn(rows, vocab, generator=g)).to(dt)
    if vocab > 3:  # a tied maximum resolves to its first index
        logits[0, vocab // 2] = logits[0, vocab - 1] = logits[0].float().max() + 1
    gl = logits.to(device)
    greedy = OS.greedy(logits)
    assert torch.equal(argmax(gl).cpu(), greedy)
    temp = torch.tensor(c["temperature"], dtype=torch.float32)
    top_k = torch.tensor(c["top_k"], dtype=torch.long)
    top_p = torch.tensor(c["top_p"], dtype=torch.float32)
    kept = [None if c["temperature"][i] == 0 else
            OS.kept_set(logits[i], c["temperature"][i], c["top_k"][i], c["top_p"][i])
            for i in range(rows)]
    seeds = torch.arange(rows, dtype=torch.long) * 7919 + seed
    for step in range(8):
        counters = torch.full((rows,), step, dtype=torch.long)
        drawn = sample(gl, *(t.to(device) for t in (temp, top_k, top_p, seeds, counters))).cpu()
        for i in range(rows):
            if kept[i] is None:
                assert int(drawn[i]) == int(greedy[i]), (step, i)
            else:
                assert bool(kept[i][int(drawn[i])]), (step, i, int(drawn[i]))


@pytest.mark.parametrize("head_dim,group", [(128, 4), (64, 4), (128, 32), (36, 2)],
                         ids=["mfma", "rows-d64", "rows-group32", "scalar-d36"])
def test_decode_padded_rows_with_one_past_the_end_offsets(device, head_dim, group):
    """The engine's decode graphs pad a batch with rows of length 0 whose
    table offset is one past the end of the block tables (the reference's
    padding). Every decode kernel path must return zeros for them without
    reading a table entry, and the real rows must still match the oracle."""
    from tinyvllm.kernels.paged_decode import paged_decode_attention
    from tinyvllm.runtime.contracts import SingleQueryMetadata

    g = torch.Generator().manual_seed(77)
    kv_heads, bs = 2, 16
    lengths = [40, 0, 300, 0]
    pool, blocks, csr = _tables(g, lengths, bs)
    offsets = csr.clone()
    for i, n in enumerate(lengths):
        if n == 0:
            offsets[i] = blocks.numel()  # one past the end
    k = torch.randn(pool * bs, kv_heads, head_dim, generator=g).to(torch.bfloat16)
    v = torch.randn(pool * bs, kv_heads, head_dim, generator=g).to(torch.bfloat16)
    q = torch.randn(len(lengths), kv_heads * group, head_dim, generator=g).to(torch.bfloat16)
    cache = _Cache(k.to(device), v.to(device), bs)
    rows = torch.arange(len(lengths))
    lens = torch.tensor(lengths)
    meta = SingleQueryMetadata(rows.to(device), blocks.to(device), offsets.to(device),
                               lens.to(device), 512)
    out = torch.full(q.shape, 7.0, dtype=q.dtype, device=device)
    paged_decode_attention(q.to(device), cache, 0, meta, out, scale=head_dim ** -0.5)
    torch.cuda.synchronize()
    expect = torch.zeros_like(q)
    OA.decode_attention(q, k, v, rows, blocks, csr, lens, bs, head_dim ** -0.5, expect)
    out = out.cpu()
    assert (out[1] == 0).all() and (out[3] == 0).all()
    assert_bf16_close(out, expect)
