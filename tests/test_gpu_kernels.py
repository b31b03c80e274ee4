"""HIP kernels vs the CPU oracle on identical seeded inputs (C1/C2 recipes).

Integer/byte work (KV writes, slot indexing, argmax indices) must be
bit-exact; floating-point outputs must meet max abs err <= 2e-2 and mean
relative (L1) error <= 1e-3 against the oracle rounded to the same dtype.
"""
import math

import pytest
import torch

from helpers import assert_bf16_close, paged_decode_case
from oracle import attention as OA
from oracle import paged_kv as OK
from oracle import pointwise as OP

pytestmark = pytest.mark.gpu


def _Cache(k, v, block_size, k_scale=1.0, v_scale=1.0, layout="head_major"):
    """A one-layer PagedKVCache holding the values of the given [slots,
    kv_heads, dim] K/V, stored head-major (the cache's default: each head's
    slots contiguous, ``key`` a [slots, heads, dim] view of that storage) or,
    with ``layout="token_major"``, in the given tensors themselves."""
    from tinyvllm.paged_kv import PagedKVCache

    if layout == "head_major":
        k, v = (t.transpose(0, 1).contiguous().transpose(0, 1) for t in (k, v))
    cache = PagedKVCache.__new__(PagedKVCache)
    cache.layout = layout
    cache.key, cache.value = k[None], v[None]
    cache.num_layers, cache.block_size = 1, block_size
    cache.num_slots, cache.num_kv_heads, cache.head_dim = k.shape
    cache.num_blocks = cache.num_slots // block_size
    cache.device, cache.dtype = k.device, k.dtype
    cache.fp8 = k.dtype == torch.float8_e4m3fn
    cache.k_scale, cache.v_scale = float(k_scale), float(v_scale)
    return cache


# ------------------------------------------------------------------ store_kv --

@pytest.mark.parametrize("layout", ["head_major", "token_major"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("strided", [False, True])
def test_store_kv_bit_exact_with_padding(device, dtype, strided, layout):
    from tinyvllm.kernels.kv_store import store_kv

    g = torch.Generator().manual_seed(11)
    tokens, hkv, d, slots_total = 256, 8, 128, 16384
    qkv = torch.randn(tokens, (16 + 2 * hkv) * d, generator=g).to(dtype)
    if strided:  # K/V as views of a packed QKV projection output
        k = qkv[:, 16 * d:(16 + hkv) * d].view(tokens, hkv, d)
        v = qkv[:, (16 + hkv) * d:].view(tokens, hkv, d)
    else:
        k = qkv[:, :hkv * d].reshape(tokens, hkv, d).contiguous()
        v = qkv[:, hkv * d:2 * hkv * d].reshape(tokens, hkv, d).contiguous()
    slots = torch.randperm(slots_total, generator=g)[:tokens]
    slots[::7] = -1
    kc = torch.full((slots_total, hkv, d), 1.5).to(dtype)
    vc = torch.full((slots_total, hkv, d), -2.5).to(dtype)
    ek, ev = kc.clone(), vc.clone()
    OK.kv_write(ek, ev, slots, k.contiguous(), v.contiguous())
    cache = _Cache(kc.to(device), vc.to(device), 16, layout=layout)
    if strided:
        dq = qkv.to(device)
        dk = dq[:, 16 * d:(16 + hkv) * d].view(tokens, hkv, d)
        dv = dq[:, (16 + hkv) * d:].view(tokens, hkv, d)
    else:
        dk, dv = k.to(device), v.to(device)
    store_kv(cache, 0, slots.to(device), dk, dv)
    torch.cuda.synchronize()
    assert torch.equal(cache.key[0].cpu().view(torch.int16), ek.view(torch.int16))
    assert torch.equal(cache.value[0].cpu().view(torch.int16), ev.view(torch.int16))


# -------------------------------------------------------------- paged decode --

def _run_decode(case, device, max_context_len=None, layout="head_major"):
    from tinyvllm.kernels.paged_decode import paged_decode_attention
    from tinyvllm.runtime.contracts import SingleQueryMetadata

    cache = _Cache(case["k"].to(device), case["v"].to(device), case["block_size"],
                   layout=layout)
    meta = SingleQueryMetadata(
        case["rows"].to(device), case["blocks"].to(device), case["offsets"].to(device),
        case["lengths"].to(device), max_context_len,
    )
    q = case["q"].to(device)
    out = torch.full_like(q, 7.0)
    paged_decode_attention(q, cache, 0, meta, out, scale=case["scale"])
    torch.cuda.synchronize()
    expect = torch.full_like(case["q"], 7.0)
    OA.decode_attention(case["q"], case["k"], case["v"], case["rows"], case["blocks"],
                        case["offsets"], case["lengths"], case["block_size"],
                        case["scale"], expect)
    return out.cpu(), expect


@pytest.mark.parametrize("layout", ["head_major", "token_major"])
def test_decode_c1_qwen3_0p6b_shapes(device, layout):
    case = paged_decode_case(seed=0, batch=8, heads=16, kv_heads=8)
    out, expect = _run_decode(case, device, max_context_len=1024, layout=layout)
    assert_bf16_close(out, expect)


@pytest.mark.parametrize("heads,kv_heads", [(8, 8), (16, 8), (32, 8), (40, 8), (64, 8), (64, 4)])
@pytest.mark.parametrize("max_ctx", [None, 2048])
def test_decode_gqa_groups_and_splits(device, heads, kv_heads, max_ctx):
    case = paged_decode_case(seed=heads + kv_heads, batch=5, heads=heads, kv_heads=kv_heads,
                             pool_blocks=512, min_len=1, max_len=1500)
    out, expect = _run_decode(case, device, max_context_len=max_ctx)
    assert_bf16_close(out, expect)


def test_decode_edge_lengths_and_padding_rows(device):
    lengths = [0, 1, 15, 16, 17, 63, 64, 65, 0, 1000]
    case = paged_decode_case(seed=9, batch=len(lengths), heads=32, kv_heads=8,
                             pool_blocks=256, lengths=lengths)
    out, expect = _run_decode(case, device, max_context_len=1024)
    assert (out[0] == 0).all() and (out[8] == 0).all()
    assert_bf16_close(out, expect)


def test_decode_selected_rows_and_strided_q(device):
    """query_rows picks rows of a larger token axis; Q is a strided view."""
    case = paged_decode_case(seed=12, batch=4, heads=32, kv_heads=8, pool_blocks=256,
                             max_len=700)
    wide = torch.randn(10, 48, 128).to(torch.bfloat16)
    q = wide[:, :32]
    rows = torch.tensor([7, 2, 9, 0])
    from tinyvllm.kernels.paged_decode import paged_decode_attention
    from tinyvllm.runtime.contracts import SingleQueryMetadata

    cache = _Cache(case["k"].to(device), case["v"].to(device), 16)
    meta = SingleQueryMetadata(rows.to(device), case["blocks"].to(device),
                               case["offsets"].to(device), case["lengths"].to(device), 800)
    out = torch.full((10, 32, 128), 3.0, dtype=torch.bfloat16, device=device)
    paged_decode_attention(q.to(device), cache, 0, meta, out, scale=case["scale"])
    expect = torch.full((10, 32, 128), 3.0).to(torch.bfloat16)
    OA.decode_attention(q, case["k"], case["v"], rows, case["blocks"], case["offsets"],
                        case["lengths"], 16, case["scale"], expect)
    assert_bf16_close(out.cpu(), expect)


@pytest.mark.parametrize("layout", ["head_major", "token_major"])
@pytest.mark.parametrize("head_dim,block_size", [(64, 16), (128, 5), (256, 8)])
def test_decode_generic_shapes(device, head_dim, block_size, layout):
    case = paged_decode_case(seed=head_dim + block_size, batch=3, heads=4, kv_heads=2,
                             head_dim=head_dim, block_size=block_size, pool_blocks=300,
                             max_len=400)
    out, expect = _run_decode(case, device, layout=layout)
    assert_bf16_close(out, expect)


@pytest.mark.parametrize("head_dim,heads,kv_heads,lengths", [
    (64, 8, 2, [0, 20000, 1, 4097]),   # 64 splits; an empty row and a 1-token row
    (256, 4, 1, [12000, 300]),         # most splits of the short row hold no key
    (32, 16, 4, [9000]),
    (128, 64, 2, [15000, 0, 700]),     # GQA group 32: the general kernel at head dim 128
])
def test_decode_general_kernel_splits_long_contexts(device, head_dim, heads, kv_heads, lengths):
    """Few rows with long contexts on the general kernel (head dims other
    than 128, groups above 16): the keys split over workgroups, whose
    partials a second launch merges."""
    from tinyvllm.kernels.paged_decode import decode_split_plan, decode_workspace_bytes

    pool = sum(-(-n // 16) for n in lengths) + 8
    case = paged_decode_case(seed=head_dim + heads, batch=len(lengths), heads=heads,
                             kv_heads=kv_heads, head_dim=head_dim, pool_blocks=pool,
                             lengths=lengths)
    max_ctx = max(lengths)
    plan = decode_split_plan(len(lengths), heads, kv_heads, head_dim, max_ctx, 16)
    assert plan >> 32 == 1 and plan & 0xFFFF > 1, plan  # general kernel, split
    assert decode_workspace_bytes(len(lengths), heads, kv_heads, head_dim, max_ctx, 16) > 0
    out, expect = _run_decode(case, device, max_context_len=max_ctx)
    for r, n in enumerate(lengths):
        if n == 0:
            assert (out[r] == 0).all()
    assert_bf16_close(out, expect)


@pytest.mark.parametrize("head_dim,heads", [(128, 32), (64, 32), (256, 8)])
def test_decode_rows_longer_than_max_context_len(device, head_dim, heads):
    """max_context_len only sizes the split plan: rows longer than it still
    attend all their keys (both kernels)."""
    lengths = [9000, 300, 4100]
    case = paged_decode_case(seed=head_dim + 1, batch=3, heads=heads, kv_heads=8,
                             head_dim=head_dim, pool_blocks=sum(-(-n // 16) for n in lengths) + 4,
                             lengths=lengths)
    out, expect = _run_decode(case, device, max_context_len=1024)
    assert_bf16_close(out, expect)


def test_decode_fp16(device):
    case = paged_decode_case(seed=21, batch=6, heads=32, kv_heads=8, pool_blocks=512,
                             dtype=torch.float16)
    out, expect = _run_decode(case, device, max_context_len=1024)
    assert_bf16_close(out, expect)


# ------------------------------------------------------------- prefill attn --

PREFILL_ITEMS = {
    # (context, query_len): fresh prompt, chunk with history, short tail, 1-token;
    # the query lengths and the grid select 128 or 256 queries per workgroup.
    "q512": [(70, 70), (600, 128), (513, 1), (300, 45), (1024, 512)],
    "q100": [(100, 100), (700, 99), (65, 1), (129, 64)],
    "q50": [(50, 50), (333, 17), (64, 64), (1, 1)],
    # eight items x 64 heads: enough workgroups for the four-wave kernel
    "q128x8": [(300, 128), (129, 128), (700, 99), (65, 1), (128, 128), (900, 64),
               (2000, 7), (128, 33)],
}


@pytest.mark.parametrize("heads,kv_heads,items,bs,layout", [
    (16, 8, "q512", 16, "head_major"), (32, 8, "q512", 16, "head_major"),
    (32, 8, "q100", 16, "head_major"), (64, 8, "q50", 16, "head_major"),
    (32, 4, "q100", 8, "head_major"), (16, 16, "q50", 32, "head_major"),
    (32, 8, "q512", 12, "head_major"), (16, 8, "q100", 2, "head_major"),
    (64, 8, "q128x8", 16, "head_major"), (64, 8, "q128x8", 12, "head_major"),
    (32, 8, "q512", 16, "token_major"), (32, 8, "q512", 12, "token_major")])
def test_prefill_chunks_with_history(device, heads, kv_heads, items, bs, layout):
    from tinyvllm.kernels.paged_prefill import paged_prefill_attention
    from tinyvllm.runtime.contracts import MultiQueryMetadata

    g = torch.Generator().manual_seed(31)
    d, pool = 128, 12288 // bs
    items = PREFILL_ITEMS[items]
    k = torch.randn(pool * bs, kv_heads, d, generator=g).to(torch.bfloat16)
    v = torch.randn(pool * bs, kv_heads, d, generator=g).to(torch.bfloat16)
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
    OA.prefill_attention(q, k, v, *meta_cpu, bs, d ** -0.5, expect)
    cache = _Cache(k.to(device), v.to(device), bs, layout=layout)
    meta = MultiQueryMetadata(*(t.to(device) for t in meta_cpu),
                              max_query_len=max(ql for _, ql in items))
    out = torch.zeros(q.shape, dtype=q.dtype, device=device)
    paged_prefill_attention(q.to(device), cache, 0, meta, out, scale=d ** -0.5)
    torch.cuda.synchronize()
    assert_bf16_close(out.cpu(), expect)


def test_prefill_v_beyond_fp16_range_takes_the_exact_path(device):
    """P.V runs on fp16 MFMAs with V converted from bf16; V values of 65536
    or more (or inf/NaN) reach the outputs as fp16 infinities, and a wave
    whose accumulators end non-finite makes the call recompute on bf16
    MFMAs. Every case matches the oracle (a missed recompute would leave
    infinities or NaNs in the output), and the fallback guard is back to
    zero after each. 65280 is the largest bf16 below 65536 (exact in fp16);
    65536 is the smallest that overflows; a value in the last pages is seen
    only by the chunk's last queries."""
    from helpers import assert_within_ulp
    from tinyvllm.kernels import paged_prefill as PP
    from tinyvllm.kernels.paged_prefill import paged_prefill_attention
    from tinyvllm.runtime.contracts import MultiQueryMetadata

    g = torch.Generator().manual_seed(41)
    heads, kv_heads, d, bs, pool = 16, 8, 128, 16, 128
    items = [(700, 300), (64, 64)]
    k = torch.randn(pool * bs, kv_heads, d, generator=g).to(torch.bfloat16)
    perm = torch.randperm(pool, generator=g).tolist()
    blocks, boff, qoff = [], [0], [0]
    for ctx, ql in items:
        n = math.ceil(ctx / bs)
        blocks += perm[boff[-1]:boff[-1] + n]
        boff.append(boff[-1] + n)
        qoff.append(qoff[-1] + ql)
    q = torch.randn(qoff[-1], heads, d, generator=g).to(torch.bfloat16)
    meta_cpu = [torch.tensor(x) for x in (qoff, blocks, boff, [c for c, _ in items])]
    meta = MultiQueryMetadata(*(t.to(device) for t in meta_cpu),
                              max_query_len=max(ql for _, ql in items))
    first_rows = torch.tensor(blocks[:3]) * bs + 5     # item 0, keys 5, 21, 37
    late_row = torch.tensor([blocks[boff[1] - 1] * bs + (700 - 1) % bs])  # key 699
    for case in ("large", "none", "65536_late", "65280", "-65536_first"):
        v = torch.randn(pool * bs, kv_heads, d, generator=g)
        if case == "large":  # a few values fp16 cannot hold, in the first item's pages
            v[first_rows, 2, 7] = 3.0e5
            v[first_rows[:1], 5, 100] = -70000.0
        elif case == "65536_late":
            v[late_row, 3, 64] = 65536.0
        elif case == "65280":
            v[first_rows, 1, 0] = 65280.0
            v[late_row, 6, 127] = -65280.0
        elif case == "-65536_first":
            v[first_rows[:1], 0, 1] = -65536.0
        v = v.to(torch.bfloat16)
        expect = torch.zeros_like(q)
        OA.prefill_attention(q, k, v, *meta_cpu, bs, d ** -0.5, expect)
        cache = _Cache(k.to(device), v.to(device), bs)
        out = torch.zeros(q.shape, dtype=q.dtype, device=device)
        paged_prefill_attention(q.to(device), cache, 0, meta, out, scale=d ** -0.5)
        torch.cuda.synchronize()
        print(f"prefill V case {case}", flush=True)
        assert_within_ulp(out.cpu(), expect, ulps=2.0)
        guard = PP._GUARDS[(out.device, torch.cuda.current_stream(out.device).cuda_stream)]
        assert int(guard.count_nonzero()) == 0


# ----------------------------------------------------------------- pointwise --

def _c2_inputs(dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(2)
    t = 256
    return dict(
        x=torch.randn(t, 1024, generator=g).to(dtype),
        res=torch.randn(t, 1024, generator=g).to(dtype),
        w=(1 + 0.02 * torch.randn(1024, generator=g)).to(dtype),
        qkv=torch.randn(t, (16 + 16) * 128, generator=g).to(dtype),
        qw=(1 + 0.02 * torch.randn(128, generator=g)).to(dtype),
        kw=(1 + 0.02 * torch.randn(128, generator=g)).to(dtype),
        pos=torch.randint(0, 2048, (t,), generator=g),
        gu=torch.randn(t, 6144, generator=g).to(dtype),
        slots=torch.randperm(16384, generator=g)[:t],
    )


@pytest.mark.parametrize("width", [1024, 4096, 5120, 128, 100, 20000])
def test_rms_norm_and_add(device, width):
    from tinyvllm.kernels.pointwise import add_rms_norm, rms_norm

    g = torch.Generator().manual_seed(width)
    x = torch.randn(37, width, generator=g).to(torch.bfloat16)
    r = torch.randn(37, width, generator=g).to(torch.bfloat16)
    w = (1 + 0.02 * torch.randn(width, generator=g)).to(torch.bfloat16)
    y = rms_norm(x.to(device), w.to(device))
    assert_bf16_close(y.cpu(), OP.rms_norm(x, w))
    y2, merged = add_rms_norm(x.to(device), r.to(device), w.to(device))
    ey, em = OP.add_rms_norm(x, r, w)
    assert torch.equal(merged.cpu(), em)  # the rounded sum is exact
    assert_bf16_close(y2.cpu(), ey)


@pytest.mark.parametrize("splits,tokens,width", [(4, 64, 4096), (8, 200, 1024),
                                                (1, 5, 5120), (3, 33, 8192)])
def test_add_rms_norm_partials(device, splits, tokens, width):
    """x = round(sequential fp32 sum of the split-K partials), then add+RMSNorm:
    the rounded residual sum is bit-exact, the normed output within bf16."""
    from tinyvllm.kernels.pointwise import add_rms_norm_partials

    g = torch.Generator().manual_seed(splits * 1000 + tokens)
    parts = torch.randn(splits, tokens, width, generator=g)
    r = torch.randn(tokens, width, generator=g).to(torch.bfloat16)
    w = (1 + 0.02 * torch.randn(width, generator=g)).to(torch.bfloat16)
    x = parts[0].clone()
    for p in range(1, splits):
        x = x + parts[p]
    x = x.to(torch.bfloat16)
    y, merged = add_rms_norm_partials(parts.to(device), r.to(device), w.to(device))
    ey, em = OP.add_rms_norm(x, r, w)
    assert torch.equal(merged.cpu(), em)
    assert_bf16_close(y.cpu(), ey)


# (in, out) -> slices at rows (1, 64, 200, 512, 600): the shapes of the
# Qwen3 attention-output and MLP-down projections (0.6B, 8B, 32B).
SPLIT_K_SHAPES = {
    (3072, 1024): (8, 8, 2, 2, 1),    # 0.6B down
    (4096, 4096): (4, 4, 4, 4, 1),    # 8B o_proj
    (12288, 4096): (4, 4, 8, 8, 1),   # 8B down
    (8192, 5120): (4, 4, 8, 8, 1),    # 32B o_proj
    (25600, 5120): (4, 4, 8, 8, 1),   # 32B down
}
SPLIT_K_ROWS = (1, 64, 200, 512, 600)


@pytest.mark.parametrize("shape", list(SPLIT_K_SHAPES), ids=lambda s: f"{s[0]}x{s[1]}")
def test_split_k_projection_matches_oracle_linear(device, shape):
    """SplitKLinear (torch.bmm over reduction slices, fp32 partials) summed by
    RMSNorm.add equals the oracle's fp32-accumulated linear (one rounding)
    followed by the oracle's add+RMSNorm, at the bf16 bar. A different fp32
    summation order may flip one rounding of the projection or of the
    residual sum, so magnitudes are chosen where one bf16 ulp fits inside
    max abs 2e-2: projection and residual ~N(0, 0.25) (sums below 4, ulp <=
    1/64) and norm weights 0.25 * (1 + N(0, 0.02)) (normed values below 2)."""
    from oracle import model as OM
    from tinyvllm.layers import RMSNorm, SplitKLinear, SplitKPartials

    k, n = shape
    g = torch.Generator().manual_seed(k + n)
    w = (torch.randn(n, k, generator=g) * (0.5 / math.sqrt(k))).to(torch.bfloat16)
    nw = (0.25 * (1 + 0.02 * torch.randn(n, generator=g))).to(torch.bfloat16)
    lin = SplitKLinear(k, n, device=device, dtype=torch.bfloat16)
    norm = RMSNorm(n, device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(w)
        norm.weight.copy_(nw)
    for rows, expect_splits in zip(SPLIT_K_ROWS, SPLIT_K_SHAPES[shape]):
        print(f"split-K {k}x{n} rows={rows}", flush=True)
        assert lin.splits_for(rows) == expect_splits
        x = torch.randn(rows, k, generator=g).to(torch.bfloat16)
        res = (0.5 * torch.randn(rows, n, generator=g)).to(torch.bfloat16)
        y = lin(x.to(device))
        assert isinstance(y, SplitKPartials) == (expect_splits > 1)
        if expect_splits > 1:
            assert y.partials.shape == (expect_splits, rows, n)
        ref = OM.linear(x, w)
        dense = y.materialize() if isinstance(y, SplitKPartials) else y
        assert_bf16_close(dense.cpu(), ref)
        out, merged = norm.add(y, res.to(device))
        eo, em = OP.add_rms_norm(ref, res, nw)
        assert_bf16_close(merged.cpu(), em)
        assert_bf16_close(out.cpu(), eo)


def test_split_k_linear_falls_back_for_strided_input(device):
    """A non-contiguous input takes F.linear (no split-K view of its rows)."""
    from tinyvllm.layers import SplitKLinear

    lin = SplitKLinear(4096, 4096, device=device, dtype=torch.bfloat16)
    torch.nn.init.normal_(lin.weight, std=0.02)
    base = torch.randn(64, 8192, device=device, dtype=torch.bfloat16)
    x = base[:, ::2]
    y = lin(x)
    assert isinstance(y, torch.Tensor)
    assert torch.equal(y, torch.nn.functional.linear(x, lin.weight))


def test_rms_norm_3d_strided_and_fp32(device):
    from tinyvllm.kernels.pointwise import rms_norm

    base = torch.randn(9, 6, 128)
    x = base[:, 1:5]  # [9, 4, 128] with head stride 128, token stride 768
    w = 1 + 0.02 * torch.randn(128)
    y = rms_norm(x.to(device), w.to(device))
    assert torch.allclose(y.cpu(), OP.rms_norm(x, w), atol=1e-5, rtol=1e-5)
    xb, wb = x.to(torch.bfloat16), w.to(torch.bfloat16)
    assert_bf16_close(rms_norm(xb.to(device), wb.to(device)).cpu(), OP.rms_norm(xb, wb))


def test_silu_and_mul_c2(device):
    from tinyvllm.kernels.pointwise import silu_and_mul

    c = _c2_inputs()
    y = silu_and_mul(c["gu"].to(device))
    assert_bf16_close(y.cpu(), OP.silu_and_mul(c["gu"]))
    odd = torch.randn(5, 2 * 37).to(torch.bfloat16)
    assert_bf16_close(silu_and_mul(odd.to(device)).cpu(), OP.silu_and_mul(odd))


@pytest.mark.parametrize("head_dim", [64, 256])
def test_qk_norm_rope_other_head_dims(device, head_dim):
    """Head dims other than 128 take the one-pair-per-lane kernel: outputs
    against the oracle, the fused KV write bit-exact."""
    from tinyvllm.kernels.pointwise import qk_norm_rope_store

    g = torch.Generator().manual_seed(head_dim)
    t, hq, hkv, d = 40, 4, 2, head_dim
    qkv = torch.randn(t, (hq + 2 * hkv) * d, generator=g).to(torch.bfloat16)
    q = qkv[:, :hq * d].view(t, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
    qw = (1 + 0.02 * torch.randn(d, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.02 * torch.randn(d, generator=g)).to(torch.bfloat16)
    cos, sin = OP.rope_tables(torch.randint(0, 4096, (t,), generator=g), d, 1e6, torch.bfloat16)
    eq, ek = OP.qk_norm_rope(q, k, qw, kw, cos, sin)
    slots = torch.randperm(256, generator=g)[:t]
    slots[3] = -1
    dq = qkv.to(device)
    gq = dq[:, :hq * d].view(t, hq, d)
    gk = dq[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    gv = dq[:, (hq + hkv) * d:].view(t, hkv, d)
    kc = torch.zeros(256, hkv, d, dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    oq, ok = qk_norm_rope_store(gq, gk, gv, *(x.to(device) for x in (qw, kw, cos, sin)),
                                1e-6, 1e-6, kc, vc, slots.to(device), key_out=True)
    assert_bf16_close(oq.cpu(), eq)
    assert_bf16_close(ok.cpu(), ek)
    ekc, evc = torch.zeros(256, hkv, d).to(torch.bfloat16), torch.zeros(256, hkv, d).to(torch.bfloat16)
    OK.kv_write(ekc, evc, slots, ok.cpu(), v.contiguous())
    assert torch.equal(kc.cpu(), ekc) and torch.equal(vc.cpu(), evc)


def test_qk_norm_rope_vector_and_scalar_kernels_agree_bitwise(device):
    """head_dim 128 with 8-byte aligned rows runs 16 lanes per row; the same
    rows one element off alignment run one RoPE pair per lane. Both sum the
    squares in the same order, so every output bit and every cache byte
    agree."""
    from tinyvllm.kernels.pointwise import qk_norm_rope_store

    g = torch.Generator().manual_seed(128)
    t, hq, hkv, d = 64, 8, 4, 128
    width = (hq + 2 * hkv) * d
    base = torch.randn(t, width, generator=g).to(torch.bfloat16).to(device)
    qw = (1 + 0.05 * torch.randn(d, generator=g)).to(torch.bfloat16).to(device)
    kw = (1 + 0.05 * torch.randn(d, generator=g)).to(torch.bfloat16).to(device)
    cos, sin = (x.to(device) for x in OP.rope_tables(
        torch.randint(0, 8192, (t,), generator=g), d, 1e6, torch.bfloat16))
    slots = torch.randperm(512, generator=g)[:t].to(device)
    outs = []
    for shift in (0, 1):  # shift 1: the same values, rows 2 bytes past alignment
        buf = torch.zeros(t, width + 1, dtype=torch.bfloat16, device=device)
        buf[:, shift:shift + width] = base
        qkv = buf[:, shift:shift + width]
        q = qkv[:, :hq * d].view(t, hq, d)
        k = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
        v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
        assert (q.data_ptr() % 8 == 0) == (shift == 0)
        kc = torch.zeros(512, hkv, d, dtype=torch.bfloat16, device=device)
        vc = torch.zeros_like(kc)
        oq, ok = qk_norm_rope_store(q, k, v, qw, kw, cos, sin, 1e-6, 1e-6, kc, vc, slots,
                                    key_out=True)
        outs.append((oq, ok, kc, vc))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("layout", ["head_major", "token_major"])
def test_qk_norm_rope_c2_and_fused_kv_write(device, layout):
    from tinyvllm.kernels.pointwise import qk_norm_rope, qk_norm_rope_store

    c = _c2_inputs()
    t, hq, hkv, d = 256, 16, 8, 128
    qkv = c["qkv"]
    q = qkv[:, :hq * d].view(t, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
    cos, sin = OP.rope_tables(c["pos"], d, 1e6, torch.bfloat16)
    eq, ek = OP.qk_norm_rope(q, k, c["qw"], c["kw"], cos, sin)
    dq = qkv.to(device)
    gq = dq[:, :hq * d].view(t, hq, d)
    gk = dq[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    gv = dq[:, (hq + hkv) * d:].view(t, hkv, d)
    args = (c["qw"].to(device), c["kw"].to(device), cos.to(device), sin.to(device))
    oq, ok = qk_norm_rope(gq, gk, *args)
    assert_bf16_close(oq.cpu(), eq)
    assert_bf16_close(ok.cpu(), ek)
    # Fused write: same Q bits, and the cache holds exactly the K/V rows the
    # unfused path produces (bit-exact), untouched elsewhere and at slot -1.
    slots = c["slots"].clone()
    slots[5] = -1
    cache = _Cache(torch.full((16384, hkv, d), 9.0, dtype=torch.bfloat16, device=device),
                   torch.full((16384, hkv, d), -9.0, dtype=torch.bfloat16, device=device),
                   16, layout=layout)
    kc, vc = cache.key[0], cache.value[0]
    fq, fk = qk_norm_rope_store(gq, gk, gv, *args, 1e-6, 1e-6, kc, vc, slots.to(device),
                                key_out=True)
    assert torch.equal(fq, oq) and torch.equal(fk, ok)
    ekc = torch.full((16384, hkv, d), 9.0).to(torch.bfloat16)
    evc = torch.full((16384, hkv, d), -9.0).to(torch.bfloat16)
    OK.kv_write(ekc, evc, slots, ok.cpu(), v.contiguous())
    assert torch.equal(kc.cpu().view(torch.int16), ekc.view(torch.int16))
    assert torch.equal(vc.cpu().view(torch.int16), evc.view(torch.int16))


# ------------------------------------------------------------------ sampling --

def test_argmax_exact_with_ties_and_nan(device):
    from tinyvllm.kernels.sampling import argmax

    g = torch.Generator().manual_seed(4)
    logits = torch.randn(64, 151936, generator=g).to(torch.bfloat16)
    logits[3, 100] = logits[3, 90000] = 50.0      # tie -> lower index
    logits[5, 151935] = 60.0                       # last element
    assert torch.equal(argmax(logits.to(device)).cpu(), logits.float().argmax(-1))
    odd = torch.randn(3, 1001).float()
    odd[1, 7] = float("nan")
    assert argmax(odd.to(device)).cpu().tolist() == [int(odd[0].argmax()), 7, int(odd[2].argmax())]


def test_sample_greedy_rows_and_degenerate_filters(device):
    from tinyvllm.kernels.sampling import sample

    g = torch.Generator().manual_seed(5)
    rows, vocab = 6, 50000
    logits = torch.randn(rows, vocab, generator=g).to(torch.bfloat16)
    temp = torch.tensor([0.0, 0.8, 1.0, 0.5, 1.2, 0.9])
    top_k = torch.tensor([0, 1, 0, 0, 1, 0])
    top_p = torch.tensor([1.0, 1.0, 1e-7, 1.0, 0.3, 1e-6])
    seeds = torch.arange(rows) * 17
    counters = torch.zeros(rows, dtype=torch.long)
    out = sample(*(x.to(device) for x in (logits, temp, top_k, top_p, seeds, counters))).cpu()
    best = logits.float().argmax(-1)
    for r in (0, 1, 2, 4, 5):  # greedy, top-k 1, tiny top-p all reduce to argmax
        assert out[r] == best[r], r


@pytest.mark.parametrize("dtype,vocab", [(torch.bfloat16, 151936), (torch.float32, 151939),
                                         (torch.float16, 16387)])
def test_sample_greedy_split_scan_matches_argmax(device, dtype, vocab):
    """Greedy rows scanned in spans over many workgroups (the workspace
    path) agree with torch's argmax and with the one-workgroup scan: ties
    across spans keep the lower index, a NaN anywhere wins, the last element
    and a vocabulary tail that is not a whole vector count."""
    from tinyvllm.kernels._extension import check, dtype_code, load_kernels, stream_of
    from tinyvllm.kernels.sampling import sample

    g = torch.Generator().manual_seed(8)
    rows = 9
    logits = torch.randn(rows, vocab, generator=g).to(dtype)
    logits[1, 100] = logits[1, vocab - 30] = 40.0   # tie in different spans
    logits[2, vocab - 1] = 50.0                     # last element (the tail)
    logits[3, 16383] = logits[3, 16384] = 45.0      # tie across a span boundary
    logits[4, vocab // 2] = float("nan")            # NaN in a middle span
    logits[5, 7] = float("nan")
    logits[5, vocab - 2] = float("nan")             # first NaN wins
    logits[6] = 0.0                                 # all equal -> index 0
    expect = logits.float().argmax(-1)
    expect[4], expect[5] = vocab // 2, 7
    zeros_f = torch.zeros(rows, device=device)
    zeros_l = torch.zeros(rows, dtype=torch.long, device=device)
    ones_f = torch.ones(rows, device=device)
    dl = logits.to(device)
    out = sample(dl, zeros_f, zeros_l, ones_f, zeros_l, zeros_l).cpu()
    assert out.tolist() == expect.tolist()
    single = torch.empty(rows, dtype=torch.long, device=device)
    lib = load_kernels()
    check(lib.tvllm_sample(dl.data_ptr(), rows, vocab, dl.stride(0), zeros_f.data_ptr(),
                           zeros_l.data_ptr(), ones_f.data_ptr(), zeros_l.data_ptr(),
                           zeros_l.data_ptr(), single.data_ptr(), None, 0,
                           dtype_code(dtype), stream_of(device)))
    assert single.cpu().tolist() == expect.tolist()


def test_sample_stays_in_kept_set_and_follows_softmax(device):
    from oracle.sampling import kept_set
    from tinyvllm.kernels.sampling import sample

    g = torch.Generator().manual_seed(6)
    vocab = 4096
    row = (torch.randn(vocab, generator=g) * 3).to(torch.bfloat16)
    cases = [(1.0, 0, 0.9), (0.7, 50, 1.0), (1.3, 200, 0.8), (1.0, 0, 1.0)]
    n = 256
    for temp, k, p in cases:
        keep = kept_set(row.float(), temp, k, p)
        logits = row[None].expand(n, vocab).contiguous()
        out = sample(logits.to(device), torch.full((n,), temp).to(device),
                     torch.full((n,), k).to(device), torch.full((n,), p).to(device),
                     torch.full((n,), 1234).to(device), torch.arange(n).to(device)).cpu()
        assert keep[out.numpy()].all(), (temp, k, p)
    # Frequencies over a 3-token distribution (temperature 1, no filters).
    probs = torch.tensor([0.5, 0.3, 0.2])
    n = 8192
    logits = torch.log(probs)[None].expand(n, 3).contiguous()
    out = sample(logits.to(device), torch.ones(n, device=device),
                 torch.zeros(n, dtype=torch.long, device=device),
                 torch.ones(n, device=device), torch.full((n,), 99, device=device),
                 torch.arange(n, device=device)).cpu()
    freq = torch.bincount(out, minlength=3).float() / n
    assert torch.allclose(freq, probs, atol=0.03), freq


@pytest.mark.parametrize("rows,heads,ctx,max_ctx", [
    (64, 32, 2049, 4096),   # the benchmark shape: 2 splits, 4-wave workgroups
    (4, 64, 20000, 32768),  # long context, few rows: workgroup-level splits + merge
])
def test_decode_benchmark_and_long_context_shapes(device, rows, heads, ctx, max_ctx):
    pages = -(-ctx // 16)
    case = paged_decode_case(seed=rows + ctx, batch=rows, heads=heads, kv_heads=8,
                             pool_blocks=rows * pages + 8, lengths=[ctx] * rows)
    out, expect = _run_decode(case, device, max_context_len=max_ctx)
    assert_bf16_close(out, expect)


@pytest.mark.parametrize("lengths,heads,kv_heads", [
    # workgroup-level splits with one span for all rows: empty and tiny rows
    # next to long ones (their spare workgroups exit early)
    ([0, 5, 30000, 17, 9000, 0], 64, 8),
    ([20000, 1, 20000, 333], 32, 8),
])
def test_decode_mixed_long_context_splits(device, lengths, heads, kv_heads):
    pool = sum(-(-n // 16) for n in lengths) + 8
    case = paged_decode_case(seed=sum(lengths) % 997, batch=len(lengths), heads=heads,
                             kv_heads=kv_heads, pool_blocks=pool, lengths=lengths)
    out, expect = _run_decode(case, device, max_context_len=32768)
    for r, n in enumerate(lengths):
        if n == 0:
            assert (out[r] == 0).all()
    assert_bf16_close(out, expect)


def test_decode_many_rows_long_context_splits(device):
    """80 rows with workgroup-level splits (MQA: one KV head, few units)."""
    g = torch.Generator().manual_seed(77)
    lengths = torch.randint(1, 3000, (80,), generator=g).tolist()
    lengths[3] = 0
    pool = sum(-(-n // 16) for n in lengths) + 8
    case = paged_decode_case(seed=78, batch=80, heads=8, kv_heads=1, pool_blocks=pool,
                             lengths=lengths)
    out, expect = _run_decode(case, device, max_context_len=4096)
    assert (out[3] == 0).all()
    assert_bf16_close(out, expect)



@pytest.mark.parametrize("heads,kv_heads,lengths,max_ctx,layout", [
    (32, 8, [2049, 1, 700, 0, 16, 17], 4096, "head_major"),  # a workgroup per row, padding
    (64, 8, [5000, 33, 1], 32768, "head_major"),   # group 8; workgroup-level splits
    (16, 8, [30000, 2], 32768, "head_major"),      # the new token in the last workgroup
    (32, 8, [2049, 1, 700, 0, 16, 17], 4096, "token_major"),
])
def test_decode_fused_qk_norm_rope_kv_write(device, heads, kv_heads, lengths, max_ctx,
                                            layout):
    """Fused decode step == qk_norm_rope_store + paged_decode: the cache after
    the step is bit-identical (rotated K, copied V, slot -1 untouched) and the
    attention output matches the unfused path and the oracle."""
    from tinyvllm.kernels.paged_decode import paged_decode_attention, paged_decode_qk_norm_rope
    from tinyvllm.kernels.pointwise import qk_norm_rope_store
    from tinyvllm.runtime.contracts import SingleQueryMetadata

    g = torch.Generator().manual_seed(sum(lengths) % 1009 + heads)
    bs, d = 16, 128
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
    kc = torch.randn(pool * bs, kv_heads, d, generator=g).to(torch.bfloat16)
    vc = torch.randn(pool * bs, kv_heads, d, generator=g).to(torch.bfloat16)
    width = (heads + 2 * kv_heads) * d
    qkv = torch.randn(rows, width, generator=g).to(torch.bfloat16)
    qw = (1 + 0.05 * torch.randn(d, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.05 * torch.randn(d, generator=g)).to(torch.bfloat16)
    pos = torch.tensor([max(n - 1, 0) for n in lengths])
    cos, sin = OP.rope_tables(pos, d, 1e6, torch.bfloat16)
    G = lambda t: t.to(device)  # noqa: E731
    gqkv = G(qkv)
    q = gqkv[:, :heads * d].view(rows, heads, d)
    k = gqkv[:, heads * d:(heads + kv_heads) * d].view(rows, kv_heads, d)
    v = gqkv[:, (heads + kv_heads) * d:].view(rows, kv_heads, d)
    meta = SingleQueryMetadata(G(torch.arange(rows)), G(torch.tensor(blocks)),
                               G(torch.tensor(offsets)), G(torch.tensor(lengths)), max_ctx)
    gslots = G(torch.tensor(slots))
    scale = d ** -0.5

    cache_a = _Cache(G(kc), G(vc), bs, layout=layout)
    q_rot, _ = qk_norm_rope_store(q, k, v, G(qw), G(kw), G(cos), G(sin), 1e-6, 1e-6,
                                  cache_a.key[0], cache_a.value[0], gslots)
    out_a = torch.zeros(rows, heads, d, dtype=torch.bfloat16, device=device)
    paged_decode_attention(q_rot, cache_a, 0, meta, out_a, scale=scale)

    cache_b = _Cache(G(kc), G(vc), bs, layout=layout)
    out_b = torch.zeros(rows, heads, d, dtype=torch.bfloat16, device=device)
    paged_decode_qk_norm_rope(q, k, v, G(qw), G(kw), G(cos), G(sin), 1e-6, 1e-6,
                              cache_b, 0, meta, gslots, out_b, scale=scale)
    torch.cuda.synchronize()
    assert torch.equal(cache_a.key[0].cpu(), cache_b.key[0].cpu())
    assert torch.equal(cache_a.value[0].cpu(), cache_b.value[0].cpu())
    assert_bf16_close(out_b.cpu(), out_a.cpu())
    # and against the oracle of the whole step
    q_ref, k_ref = OP.qk_norm_rope(qkv[:, :heads * d].view(rows, heads, d),
                                   qkv[:, heads * d:(heads + kv_heads) * d].view(rows, kv_heads, d),
                                   qw, kw, cos, sin)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    for r, sl in enumerate(slots):
        if sl >= 0:
            kc_ref[sl] = k_ref[r]
            vc_ref[sl] = qkv[r, (heads + kv_heads) * d:].view(kv_heads, d)
    expect = torch.zeros(rows, heads, d, dtype=torch.bfloat16)
    OA.decode_attention(q_ref, kc_ref, vc_ref, torch.arange(rows), torch.tensor(blocks),
                        torch.tensor(offsets), torch.tensor(lengths), bs, scale, expect)
    assert_bf16_close(out_b.cpu(), expect)
    for r, n in enumerate(lengths):
        if n == 0:
            assert (out_b[r].cpu() == 0).all()


def test_decode_shared_prefix_pages_long_context(device):
    """C5 layout: every row's table starts with the same 256 read-only pages
    (a 4096-token prefix shared through the prefix cache), then private pages;
    contexts up to 31k tokens, so the rows run workgroup-level splits over
    shared pages. Two rows with the same query and the same table must give
    bit-identical outputs wherever they sit in the batch."""
    g = torch.Generator().manual_seed(91)
    bs, prefix_pages, heads, kv_heads = 16, 256, 64, 8
    lengths = [20000, 4096, 31000, 4100, 16500, 4096]
    pool = prefix_pages + sum(-(-n // bs) - prefix_pages for n in lengths) + 4
    perm = torch.randperm(pool, generator=g).tolist()
    shared, rest = perm[:prefix_pages], perm[prefix_pages:]
    blocks, offsets = [], [0]
    for n in lengths:
        own = -(-n // bs) - prefix_pages
        blocks += shared + rest[:own]
        rest = rest[own:]
        offsets.append(len(blocks))
    k = torch.randn(pool * bs, kv_heads, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(pool * bs, kv_heads, 128, generator=g).to(torch.bfloat16)
    q = torch.randn(len(lengths), heads, 128, generator=g).to(torch.bfloat16)
    q[5] = q[1]   # rows 1 and 5: same query, same (prefix-only) table
    case = dict(q=q, k=k, v=v, rows=torch.arange(len(lengths)),
                blocks=torch.tensor(blocks), offsets=torch.tensor(offsets),
                lengths=torch.tensor(lengths), block_size=bs, scale=128 ** -0.5)
    out, expect = _run_decode(case, device, max_context_len=32768)
    assert_bf16_close(out, expect)
    assert torch.equal(out[1].view(torch.int16), out[5].view(torch.int16))



def test_decode_split_merge_reuses_its_workspace(device):
    """Workgroup-level splits write partials to the workspace and a second
    kernel merges them. Repeated calls on one workspace (eager and in a
    replayed graph) give identical outputs, equal to the oracle's."""
    from tinyvllm.kernels.paged_decode import decode_workspace_bytes, paged_decode_attention
    from tinyvllm.runtime.contracts import SingleQueryMetadata

    lengths = [1000, 3, 0, 777]
    pool = sum(-(-n // 16) for n in lengths) + 8
    case = paged_decode_case(seed=91, batch=4, heads=16, kv_heads=8, pool_blocks=pool,
                             lengths=lengths)
    need = decode_workspace_bytes(4, 16, 8, 128, 1024, case["block_size"])
    assert need > 0  # this shape splits over workgroups
    ws = torch.empty(need, dtype=torch.uint8, device=device)
    cache = _Cache(case["k"].to(device), case["v"].to(device), case["block_size"])
    meta = SingleQueryMetadata(case["rows"].to(device), case["blocks"].to(device),
                               case["offsets"].to(device), case["lengths"].to(device), 1024)
    q = case["q"].to(device)
    outs = []
    for _ in range(3):
        out = torch.full_like(q, 7.0)
        paged_decode_attention(q, cache, 0, meta, out, scale=case["scale"], workspace=ws)
        torch.cuda.synchronize()
        outs.append(out.cpu())
    expect = torch.full_like(case["q"], 7.0)
    OA.decode_attention(case["q"], case["k"], case["v"], case["rows"], case["blocks"],
                        case["offsets"], case["lengths"], case["block_size"], case["scale"],
                        expect)
    assert_bf16_close(outs[0], expect)
    assert all(torch.equal(o, outs[0]) for o in outs[1:])
    graph_out = torch.full_like(q, 7.0)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        paged_decode_attention(q, cache, 0, meta, graph_out, scale=case["scale"], workspace=ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged_decode_attention(q, cache, 0, meta, graph_out, scale=case["scale"], workspace=ws)
    for _ in range(3):
        graph_out.fill_(7.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(graph_out.cpu(), outs[0])


@pytest.mark.parametrize("layout,fp8", [("head_major", False), ("token_major", False),
                                       ("token_major", True)])
@pytest.mark.parametrize("heads,kv_heads,lengths,max_ctx", [
    (32, 8, [2049, 1, 700, 0, 16, 17], 4096),   # group 4, a padding row
    (16, 8, [300, 77, 1], 1024),                 # group 2
    (64, 8, [5000, 33], 32768),                  # group 8, workgroup-level splits
])
def test_decode_fused_from_qkv_partials(device, heads, kv_heads, lengths, max_ctx, layout,
                                        fp8):
    """The fused decode kernel fed the qkv projection as four fp32 split-K
    partials equals the same kernel fed their in-order sum rounded to bf16:
    the cache bits written and the attention output are identical."""
    from tinyvllm.kernels.paged_decode import (paged_decode_qk_norm_rope,
                                               paged_decode_qk_norm_rope_partials)
    from tinyvllm.runtime.contracts import SingleQueryMetadata

    g = torch.Generator().manual_seed(sum(lengths) % 997 + heads)
    bs, d = 16, 128
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
    kc = torch.randn(pool * bs, kv_heads, d, generator=g).to(torch.bfloat16)
    vc = torch.randn(pool * bs, kv_heads, d, generator=g).to(torch.bfloat16)
    width = (heads + 2 * kv_heads) * d
    parts = torch.randn(4, rows, width, generator=g) * 0.5
    summed = (((parts[0] + parts[1]) + parts[2]) + parts[3]).to(torch.bfloat16)
    qw = (1 + 0.05 * torch.randn(d, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.05 * torch.randn(d, generator=g)).to(torch.bfloat16)
    pos = torch.tensor([max(n - 1, 0) for n in lengths])
    cos, sin = OP.rope_tables(pos, d, 1e6, torch.bfloat16)
    G = lambda t: t.to(device)  # noqa: E731
    meta = SingleQueryMetadata(G(torch.arange(rows)), G(torch.tensor(blocks)),
                               G(torch.tensor(offsets)), G(torch.tensor(lengths)), max_ctx)
    gslots = G(torch.tensor(slots))
    args = (G(qw), G(kw), G(cos), G(sin), 1e-6, 1e-6)
    gs = G(summed)
    q = gs[:, :heads * d].view(rows, heads, d)
    k = gs[:, heads * d:(heads + kv_heads) * d].view(rows, kv_heads, d)
    v = gs[:, (heads + kv_heads) * d:].view(rows, kv_heads, d)
    if fp8:  # an FP8 E4M3 cache (scales 0.5 / 2): the same quantised writes
        kc, vc = (OK.fp8_quantize(t.float(), sc).view(torch.float8_e4m3fn)
                  for t, sc in ((kc, 0.5), (vc, 2.0)))
    scales = (0.5, 2.0) if fp8 else (1.0, 1.0)
    cache_a = _Cache(G(kc), G(vc), bs, *scales, layout=layout)
    out_a = torch.zeros(rows, heads, d, dtype=torch.bfloat16, device=device)
    paged_decode_qk_norm_rope(q, k, v, *args, cache_a, 0, meta, gslots, out_a, scale=d ** -0.5)
    cache_b = _Cache(G(kc), G(vc), bs, *scales, layout=layout)
    out_b = torch.full((rows, heads, d), 5.0, dtype=torch.bfloat16, device=device)
    paged_decode_qk_norm_rope_partials(G(parts), heads, *args, cache_b, 0, meta, gslots, out_b,
                                       scale=d ** -0.5)
    torch.cuda.synchronize()
    bits = torch.uint8 if fp8 else torch.int16
    assert torch.equal(cache_a.key[0].cpu().view(bits), cache_b.key[0].cpu().view(bits))
    assert torch.equal(cache_a.value[0].cpu().view(bits), cache_b.value[0].cpu().view(bits))
    assert torch.equal(out_a.cpu(), out_b.cpu())


def test_qkv_decode_partials_rule_and_values(device):
    """PackedLinear.decode_partials: four fp32 slices whose sum is the
    projection (within fp32 rounding), only at decode batch sizes."""
    from tinyvllm.layers import PackedLinear

    torch.manual_seed(0)
    small = PackedLinear(1024, (2048, 1024, 1024), device=device, dtype=torch.bfloat16)
    wide = PackedLinear(4096, (4096, 1024, 1024), device=device, dtype=torch.bfloat16)
    x = torch.randn(32, 1024, device=device, dtype=torch.bfloat16)
    parts = small.decode_partials(x)
    assert parts.shape == (4, 32, 4096) and parts.dtype == torch.float32
    ref = x.float() @ small.weight.float().t()
    assert (parts.sum(0) - ref).abs().max().item() < 1e-3
    assert small.decode_partials(torch.randn(65, 1024, device=device,
                                             dtype=torch.bfloat16)) is None
    assert small.decode_partials(x[:16]) is None                 # 16 rows: one GEMM
    assert wide.decode_partials(torch.randn(64, 4096, device=device,
                                            dtype=torch.bfloat16)) is None
    wider = PackedLinear(5120, (8192, 1024, 1024), device=device, dtype=torch.bfloat16)
    assert wider.decode_partials(torch.randn(64, 5120, device=device,
                                             dtype=torch.bfloat16)).shape == (4, 64, 10240)
    assert wider.decode_partials(torch.randn(32, 5120, device=device,
                                             dtype=torch.bfloat16)) is None
