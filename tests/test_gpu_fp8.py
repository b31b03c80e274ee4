"""FP8 E4M3 KV-cache layout on the GPU kernels (no reference counterpart).

Bit-exact: every byte the KV writers store equals the oracle's
``fp8_quantize`` of the row the bf16 path writes (store_kv, the fused
QK-norm/RoPE write, the fused decode step). Attention over an FP8 cache is
compared with the oracle's attention over the dequantised cache (the kernels
widen E4M3 to bf16 exactly and fold the scales into the softmax scale and
the output), to the same bf16 tolerance as the 16-bit cache."""
from __future__ import annotations

import math

import pytest
import torch

from helpers import assert_bf16_close, paged_decode_case
from oracle import attention as OA
from oracle import paged_kv as OK
from oracle import pointwise as OP
from test_gpu_kernels import _Cache

pytestmark = pytest.mark.gpu
F8 = torch.float8_e4m3fn


def _fp8_cache(k, v, bs, device, k_scale=1.0, v_scale=1.0, layout="head_major"):
    """GPU FP8 cache holding the oracle's quantisation of k/v (and the CPU
    dequantised copies the oracle attends over)."""
    kq, vq = OK.fp8_quantize(k, k_scale), OK.fp8_quantize(v, v_scale)
    cache = _Cache(kq.view(F8).to(device), vq.view(F8).to(device), bs, k_scale, v_scale,
                   layout=layout)
    return cache, OK.fp8_dequantize(kq, k_scale), OK.fp8_dequantize(vq, v_scale)


@pytest.mark.parametrize("layout", ["head_major", "token_major"])
@pytest.mark.parametrize("strided", [False, True])
@pytest.mark.parametrize("scales", [(1.0, 1.0), (0.25, 3.0)])
def test_store_kv_fp8_bit_exact(device, strided, scales, layout):
    from tinyvllm.kernels.kv_store import store_kv

    g = torch.Generator().manual_seed(12)
    tokens, hkv, d, total = 200, 8, 128, 4096
    qkv = (torch.randn(tokens, (16 + 2 * hkv) * d, generator=g) * 20).to(torch.bfloat16)
    if strided:
        k = qkv[:, 16 * d:(16 + hkv) * d].view(tokens, hkv, d)
        v = qkv[:, (16 + hkv) * d:].view(tokens, hkv, d)
    else:
        k = qkv[:, :hkv * d].reshape(tokens, hkv, d).contiguous()
        v = qkv[:, hkv * d:2 * hkv * d].reshape(tokens, hkv, d).contiguous()
    slots = torch.randperm(total, generator=g)[:tokens]
    slots[::9] = -1
    sentinel = 0x5A
    kc = torch.full((total, hkv, d), sentinel, dtype=torch.uint8)
    vc = kc.clone()
    ek, ev = kc.clone(), vc.clone()
    keep = slots >= 0
    ek[slots[keep]] = OK.fp8_quantize(k.contiguous()[keep], scales[0])
    ev[slots[keep]] = OK.fp8_quantize(v.contiguous()[keep], scales[1])
    cache = _Cache(kc.view(F8).to(device), vc.view(F8).to(device), 16, *scales, layout=layout)
    dq = qkv.to(device)
    if strided:
        dk = dq[:, 16 * d:(16 + hkv) * d].view(tokens, hkv, d)
        dv = dq[:, (16 + hkv) * d:].view(tokens, hkv, d)
    else:
        dk, dv = k.to(device), v.to(device)
    store_kv(cache, 0, slots.to(device), dk, dv)
    torch.cuda.synchronize()
    assert torch.equal(cache.key[0].cpu().view(torch.uint8), ek)
    assert torch.equal(cache.value[0].cpu().view(torch.uint8), ev)


def test_qk_norm_rope_store_fp8_bit_exact(device):
    from tinyvllm.kernels.pointwise import qk_norm_rope, qk_norm_rope_store

    g = torch.Generator().manual_seed(13)
    t, hq, hkv, d = 96, 16, 8, 128
    qkv = torch.randn(t, (hq + 2 * hkv) * d, generator=g).to(torch.bfloat16)
    qw = (1 + 0.05 * torch.randn(d, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.05 * torch.randn(d, generator=g)).to(torch.bfloat16)
    pos = torch.randint(0, 2048, (t,), generator=g)
    cos, sin = OP.rope_tables(pos, d, 1e6, torch.bfloat16)
    dq = qkv.to(device)
    q = dq[:, :hq * d].view(t, hq, d)
    k = dq[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    v = dq[:, (hq + hkv) * d:].view(t, hkv, d)
    args = tuple(x.to(device) for x in (qw, kw, cos, sin))
    slots = torch.randperm(1024, generator=g)[:t]
    slots[3] = -1
    kc = torch.full((1024, hkv, d), 0x11, dtype=torch.uint8, device=device).view(F8)
    vc = torch.full((1024, hkv, d), 0x22, dtype=torch.uint8, device=device).view(F8)
    oq, ok = qk_norm_rope(q, k, *args)
    fq, _ = qk_norm_rope_store(q, k, v, *args, 1e-6, 1e-6, kc, vc, slots.to(device),
                               k_scale=0.5, v_scale=2.0)
    torch.cuda.synchronize()
    assert torch.equal(fq, oq)
    ek = torch.full((1024, hkv, d), 0x11, dtype=torch.uint8)
    ev = torch.full((1024, hkv, d), 0x22, dtype=torch.uint8)
    keep = slots >= 0
    ek[slots[keep]] = OK.fp8_quantize(ok.cpu()[keep], 0.5)
    ev[slots[keep]] = OK.fp8_quantize(qkv[:, (hq + hkv) * d:].view(t, hkv, d)[keep], 2.0)
    assert torch.equal(kc.cpu().view(torch.uint8), ek)
    assert torch.equal(vc.cpu().view(torch.uint8), ev)


def _decode(case, device, k_scale, v_scale, max_ctx, dtype=torch.bfloat16,
            layout="head_major"):
    from tinyvllm.kernels.paged_decode import paged_decode_attention
    from tinyvllm.runtime.contracts import SingleQueryMetadata

    cache, kd, vd = _fp8_cache(case["k"].float() * k_scale, case["v"].float() * v_scale,
                               case["block_size"], device, k_scale, v_scale, layout)
    q = case["q"].to(dtype)
    meta = SingleQueryMetadata(*(case[n].to(device) for n in ("rows", "blocks", "offsets",
                                                              "lengths")), max_ctx)
    out = torch.full(q.shape, 7.0, dtype=dtype, device=device)
    paged_decode_attention(q.to(device), cache, 0, meta, out, scale=case["scale"])
    torch.cuda.synchronize()
    expect = torch.full(q.shape, 7.0, dtype=dtype)
    OA.decode_attention(q, kd, vd, case["rows"], case["blocks"], case["offsets"],
                        case["lengths"], case["block_size"], case["scale"], expect)
    return out.cpu(), expect


@pytest.mark.parametrize("heads,kv_heads,lengths,max_ctx,scales", [
    (16, 8, None, 1024, (1.0, 1.0)),                       # C1 shapes
    (32, 8, [2049] * 64, 4096, (0.5, 2.0)),                # 8B bs64: in-workgroup splits
    (64, 8, [20000, 5, 0, 9000], 32768, (1.0, 0.25)),      # workgroup splits + merge
    (8, 8, [300, 1, 77], 1024, (1.0, 1.0)),                # group 1
    (16, 4, [513, 2], 1024, (1.0, 1.0)),                   # group 4
    (64, 4, [3000, 40], 4096, (2.0, 1.0)),                 # group 16
    (8, 1, [700, 33, 1], 1024, (1.0, 1.0)),                # group 8, MQA
])
def test_decode_fp8_cache_matches_oracle(device, heads, kv_heads, lengths, max_ctx, scales):
    pool = 1024 if lengths is None else sum(max(1, -(-n // 16)) for n in lengths) + 8
    case = paged_decode_case(seed=heads + kv_heads, batch=8 if lengths is None else len(lengths),
                             heads=heads, kv_heads=kv_heads, pool_blocks=pool, lengths=lengths)
    out, expect = _decode(case, device, *scales, max_ctx)
    if lengths is not None:
        for r, n in enumerate(lengths):
            if n == 0:
                assert (out[r] == 0).all()
    assert_bf16_close(out, expect)


@pytest.mark.parametrize("head_dim,heads,kv_heads,lengths,scales", [
    (64, 8, 2, [20000, 0, 300], (1.0, 0.25)),
    (256, 4, 2, [9000, 1], (0.5, 2.0)),
])
def test_decode_fp8_general_kernel_splits(device, head_dim, heads, kv_heads, lengths, scales):
    """The general kernel over an FP8 cache with its keys split over
    workgroups (few rows, long contexts)."""
    pool = sum(max(1, -(-n // 16)) for n in lengths) + 8
    case = paged_decode_case(seed=head_dim, batch=len(lengths), heads=heads,
                             kv_heads=kv_heads, head_dim=head_dim, pool_blocks=pool,
                             lengths=lengths)
    out, expect = _decode(case, device, *scales, max(lengths))
    for r, n in enumerate(lengths):
        if n == 0:
            assert (out[r] == 0).all()
    assert_bf16_close(out, expect)


def test_decode_fp8_cache_fp16_queries(device):
    case = paged_decode_case(seed=5, batch=6, heads=32, kv_heads=8, pool_blocks=1024)
    out, expect = _decode(case, device, 1.0, 1.0, 1024, dtype=torch.float16)
    assert_bf16_close(out.float(), expect.float())


def test_decode_fp8_token_major_cache(device):
    """The reference's contiguous [slots, heads, dim] layout through the same
    kernel (its 128-byte head rows at a 1 KiB stride)."""
    case = paged_decode_case(seed=6, batch=8, heads=32, kv_heads=8, pool_blocks=1024)
    out, expect = _decode(case, device, 0.5, 2.0, 1024, layout="token_major")
    assert_bf16_close(out, expect)


@pytest.mark.parametrize("lengths,heads,kv_heads,max_ctx", [
    ([2049, 1, 700, 0, 16, 17], 32, 8, 4096),
    ([5000, 33, 1], 64, 8, 32768),
])
def test_decode_fused_fp8_write_matches_unfused(device, lengths, heads, kv_heads, max_ctx):
    """The fused decode step's FP8 K/V bytes equal qk_norm_rope_store's FP8
    bytes (bit-exact); outputs match the unfused path and the oracle."""
    from tinyvllm.kernels.paged_decode import paged_decode_attention, paged_decode_qk_norm_rope
    from tinyvllm.kernels.pointwise import qk_norm_rope_store
    from tinyvllm.runtime.contracts import SingleQueryMetadata

    g = torch.Generator().manual_seed(sum(lengths) % 997)
    bs, d, ks, vs = 16, 128, 0.5, 0.25
    rows = len(lengths)
    pages = [max(1, -(-n // bs)) for n in lengths]
    pool = sum(pages) + 4
    perm = torch.randperm(pool, generator=g)
    blocks, offsets = [], [0]
    for p in pages:
        blocks += perm[offsets[-1]:offsets[-1] + p].tolist()
        offsets.append(offsets[-1] + p)
    slots = [blocks[offsets[r] + (n - 1) // bs] * bs + (n - 1) % bs if n > 0 else -1
             for r, n in enumerate(lengths)]
    kc = OK.fp8_quantize(torch.randn(pool * bs, kv_heads, d, generator=g) * ks, ks)
    vc = OK.fp8_quantize(torch.randn(pool * bs, kv_heads, d, generator=g) * vs, vs)
    qkv = torch.randn(rows, (heads + 2 * kv_heads) * d, generator=g).to(torch.bfloat16)
    qw = (1 + 0.05 * torch.randn(d, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.05 * torch.randn(d, generator=g)).to(torch.bfloat16)
    cos, sin = OP.rope_tables(torch.tensor([max(n - 1, 0) for n in lengths]), d, 1e6,
                              torch.bfloat16)
    G = lambda t: t.to(device)  # noqa: E731
    gqkv = G(qkv)
    q = gqkv[:, :heads * d].view(rows, heads, d)
    k = gqkv[:, heads * d:(heads + kv_heads) * d].view(rows, kv_heads, d)
    v = gqkv[:, (heads + kv_heads) * d:].view(rows, kv_heads, d)
    meta = SingleQueryMetadata(G(torch.arange(rows)), G(torch.tensor(blocks)),
                               G(torch.tensor(offsets)), G(torch.tensor(lengths)), max_ctx)
    gslots = G(torch.tensor(slots))
    args = (G(qw), G(kw), G(cos), G(sin))
    scale = d ** -0.5

    cache_a = _Cache(G(kc).view(F8), G(vc).view(F8), bs, ks, vs)
    q_rot, _ = qk_norm_rope_store(q, k, v, *args, 1e-6, 1e-6, cache_a.key[0],
                                  cache_a.value[0], gslots, k_scale=ks, v_scale=vs)
    out_a = torch.zeros(rows, heads, d, dtype=torch.bfloat16, device=device)
    paged_decode_attention(q_rot, cache_a, 0, meta, out_a, scale=scale)
    cache_b = _Cache(G(kc).view(F8), G(vc).view(F8), bs, ks, vs)
    out_b = torch.zeros(rows, heads, d, dtype=torch.bfloat16, device=device)
    paged_decode_qk_norm_rope(q, k, v, *args, 1e-6, 1e-6, cache_b, 0, meta, gslots, out_b,
                              scale=scale)
    torch.cuda.synchronize()
    assert torch.equal(cache_a.key[0].cpu().view(torch.uint8),
                       cache_b.key[0].cpu().view(torch.uint8))
    assert torch.equal(cache_a.value[0].cpu().view(torch.uint8),
                       cache_b.value[0].cpu().view(torch.uint8))
    assert_bf16_close(out_b.cpu(), out_a.cpu())
    # oracle of the whole step over the dequantised cache
    q_ref, k_ref = OP.qk_norm_rope(qkv[:, :heads * d].view(rows, heads, d),
                                   qkv[:, heads * d:(heads + kv_heads) * d].view(rows, kv_heads, d),
                                   qw, kw, cos, sin)
    kq, vq = kc.clone(), vc.clone()
    for r, sl in enumerate(slots):
        if sl >= 0:
            kq[sl] = OK.fp8_quantize(k_ref[r], ks)
            vq[sl] = OK.fp8_quantize(qkv[r, (heads + kv_heads) * d:].view(kv_heads, d), vs)
    assert torch.equal(cache_b.key[0].cpu().view(torch.uint8), kq)
    expect = torch.zeros(rows, heads, d, dtype=torch.bfloat16)
    OA.decode_attention(q_ref, OK.fp8_dequantize(kq, ks), OK.fp8_dequantize(vq, vs),
                        torch.arange(rows), torch.tensor(blocks), torch.tensor(offsets),
                        torch.tensor(lengths), bs, scale, expect)
    assert_bf16_close(out_b.cpu(), expect)


@pytest.mark.parametrize("bs,layout", [(16, "head_major"), (12, "head_major"),
                                       (16, "token_major")])
def test_prefill_fp8_cache_matches_oracle(device, bs, layout):
    from tinyvllm.kernels.paged_prefill import paged_prefill_attention
    from tinyvllm.runtime.contracts import MultiQueryMetadata

    g = torch.Generator().manual_seed(41)
    heads, kv_heads, d, pool = 32, 8, 128, 12288 // bs
    items = [(70, 70), (600, 128), (513, 1), (1024, 512)]
    ks, vs = 0.5, 0.25  # unit-variance K/V stored as 2x and 4x their values
    cache_cpu_k = torch.randn(pool * bs, kv_heads, d, generator=g)
    cache_cpu_v = torch.randn(pool * bs, kv_heads, d, generator=g)
    cache, kd, vd = _fp8_cache(cache_cpu_k, cache_cpu_v, bs, device, ks, vs, layout)
    perm = torch.randperm(pool, generator=g).tolist()
    blocks, boff, qoff = [], [0], [0]
    for ctx, ql in items:
        n = math.ceil(ctx / bs)
        blocks += perm[boff[-1]:boff[-1] + n]
        boff.append(boff[-1] + n)
        qoff.append(qoff[-1] + ql)
    q = torch.randn(qoff[-1], heads, d, generator=g).to(torch.bfloat16)
    meta_cpu = [torch.tensor(x) for x in (qoff, blocks, boff, [c for c, _ in items])]
    expect = torch.zeros_like(q)
    OA.prefill_attention(q, kd, vd, *meta_cpu, bs, d ** -0.5, expect)
    meta = MultiQueryMetadata(*(t.to(device) for t in meta_cpu),
                              max_query_len=max(ql for _, ql in items))
    out = torch.zeros(q.shape, dtype=q.dtype, device=device)
    paged_prefill_attention(q.to(device), cache, 0, meta, out, scale=d ** -0.5)
    torch.cuda.synchronize()
    assert_bf16_close(out.cpu(), expect)
