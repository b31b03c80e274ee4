"""The pointwise kernels against the oracle over seeded random
configurations: RMSNorm (2-D and strided 3-D rows, bf16 / fp16 / fp32, any
width), add+RMSNorm, the split-K partial sums with add+RMSNorm, SiLU*up
(strided inputs, odd half widths), QK-norm + RoPE with the fused KV write
(head dims 64 / 128 / 256, Q/K/V strided views of one packed projection,
padding slots -1, both cache layouts) and the slot-mapped KV store. The KV
bytes, the rounded residual sums and the slots left alone are bit-exact;
normed and rotated values meet the bar (max abs 2e-2, mean relative 1e-3).
Each configuration comes from its own seed and is printed in the test id."""
import random

import pytest
import torch

from helpers import assert_bf16_close
from oracle import paged_kv as OK
from oracle import pointwise as OP
from test_gpu_kernels import _Cache

pytestmark = pytest.mark.gpu

CASES = 40
KINDS = ("rms", "add", "partials", "silu", "rope", "store")
DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def _config(seed: int) -> dict:
    r = random.Random(4000 + seed)
    kind = KINDS[seed % len(KINDS)]
    c = dict(kind=kind, tokens=r.choice([1, 2, 7, 64, 129, 300]))
    if kind in ("rms", "add", "silu"):
        c["width"] = r.choice([2, 64, 100, 128, 1024, 3072, 4096, 5120, 8192, 20000])
        if kind == "silu" and c["width"] % 2:
            c["width"] += 1
        c["dtype"] = r.choice(["bf16", "fp16", "fp32"] if kind != "add" else ["bf16", "fp16"])
        c["strided"] = r.random() < 0.5
        c["heads"] = r.choice([1, 1, 4]) if kind != "add" else 1
    elif kind == "partials":
        c["width"] = r.choice([8, 128, 1024, 4096, 5120, 8192])
        c["splits"] = r.choice([1, 2, 3, 4, 8])
        c["dtype"] = r.choice(["bf16", "fp16"])
    else:  # rope, store
        c["kv_heads"] = r.choice([1, 2, 4, 8])
        c["heads"] = c["kv_heads"] * r.choice([1, 2, 4, 8])
        c["head_dim"] = r.choice([128, 128, 64, 256]) if kind == "rope" else 128
        c["dtype"] = r.choice(["bf16", "fp16"])
        c["layout"] = r.choice(["head_major", "token_major"])
    return c


def _id(seed: int) -> str:
    c = _config(seed)
    return f"s{seed}-" + "-".join(f"{k}{v}" for k, v in c.items() if k != "kind") + f"-{c['kind']}"


@pytest.mark.parametrize("seed", range(CASES), ids=_id)
def test_pointwise_random_configuration(device, seed):
    from tinyvllm.kernels import pointwise as KP
    from tinyvllm.kernels.kv_store import store_kv

    c = _config(seed)
    g = torch.Generator().manual_seed(seed)
    dt = DTYPES[c["dtype"]]
    t = c["tokens"]
    G = lambda x: x.to(device)  # noqa: E731

    if c["kind"] in ("rms", "silu"):
        heads, w = c["heads"], c["width"]
        pad = 24 if c["strided"] else 0
        wide = torch.randn(t, heads, w + pad, generator=g).to(dt)
        x = wide[..., :w] if heads > 1 else wide[:, 0, :w]
        gx = G(wide)[..., :w] if heads > 1 else G(wide)[:, 0, :w]
        if c["kind"] == "rms":
            weight = (1 + 0.02 * torch.randn(w, generator=g)).to(dt)
            assert_bf16_close(KP.rms_norm(gx, G(weight)).cpu(), OP.rms_norm(x, weight))
        else:
            assert_bf16_close(KP.silu_and_mul(gx).cpu(), OP.silu_and_mul(x))
        return

    if c["kind"] == "add":
        w = c["width"]
        x = torch.randn(t, w, generator=g).to(dt)
        res = torch.randn(t, w, generator=g).to(dt)
        weight = (1 + 0.02 * torch.randn(w, generator=g)).to(dt)
        if c["strided"]:
            gx = G(torch.cat([x, x[:, :8]], 1))[:, :w]
        else:
            gx = G(x)
        y, merged = KP.add_rms_norm(gx, G(res), G(weight))
        ey, em = OP.add_rms_norm(x, res, weight)
        assert torch.equal(merged.cpu(), em)  # one rounding of an exact sum
        assert_bf16_close(y.cpu(), ey)
        return

    if c["kind"] == "partials":
        s, w = c["splits"], c["width"]
        parts = torch.randn(s, t, w, generator=g)
        res = torch.randn(t, w, generator=g).to(dt)
        weight = (1 + 0.02 * torch.randn(w, generator=g)).to(dt)
        x = parts[0].clone()
        for p in range(1, s):  # the kernel's summation order
            x = x + parts[p]
        y, merged = KP.add_rms_norm_partials(G(parts), G(res), G(weight))
        ey, em = OP.add_rms_norm(x.to(dt), res, weight)
        assert torch.equal(merged.cpu(), em)
        assert_bf16_close(y.cpu(), ey)
        return

    # rope / store: Q, K, V are strided views of one packed projection.
    hq, hkv, d = c["heads"], c["kv_heads"], c["head_dim"]
    qkv = torch.randn(t, (hq + 2 * hkv) * d, generator=g).to(dt)
    q = qkv[:, :hq * d].view(t, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
    gqkv = G(qkv)
    gq = gqkv[:, :hq * d].view(t, hq, d)
    gk = gqkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    gv = gqkv[:, (hq + hkv) * d:].view(t, hkv, d)
    num_slots = 16 * (t + 7)
    slots = torch.randperm(num_slots, generator=g)[:t]
    slots[torch.rand(t, generator=g) < 0.2] = -1
    kc = torch.full((num_slots, hkv, d), 1.5).to(dt)
    vc = torch.full((num_slots, hkv, d), -2.5).to(dt)
    cache = _Cache(G(kc), G(vc), 16, layout=c["layout"])
    if c["kind"] == "store":
        store_kv(cache, 0, G(slots), gk, gv)
        OK.kv_write(kc, vc, slots, k.contiguous(), v.contiguous())
        torch.cuda.synchronize()
        assert torch.equal(cache.key[0].cpu().view(torch.int16), kc.view(torch.int16))
        assert torch.equal(cache.value[0].cpu().view(torch.int16), vc.view(torch.int16))
        return
    qw = (1 + 0.05 * torch.randn(d, generator=g)).to(dt)
    kw = (1 + 0.05 * torch.randn(d, generator=g)).to(dt)
    cos, sin = OP.rope_tables(torch.randint(0, 40960, (t,), generator=g), d, 1e6, dt)
    q_out, k_out = KP.qk_norm_rope_store(gq, gk, gv, G(qw), G(kw), G(cos), G(sin), 1e-6, 1e-6,
                                         cache.key[0], cache.value[0], G(slots), key_out=True)
    eq, ek = OP.qk_norm_rope(q, k, qw, kw, cos, sin)
    assert_bf16_close(q_out.cpu(), eq)
    assert_bf16_close(k_out.cpu(), ek)
    # The cache holds exactly the kernel's rotated K and the V rows.
    OK.kv_write(kc, vc, slots, k_out.cpu(), v.contiguous())
    torch.cuda.synchronize()
    assert torch.equal(cache.key[0].cpu().view(torch.int16), kc.view(torch.int16))
    assert torch.equal(cache.value[0].cpu().view(torch.int16), vc.view(torch.int16))
