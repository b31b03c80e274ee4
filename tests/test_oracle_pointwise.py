"""Pins for oracle/pointwise.py: transformers' fp32 Qwen3 modules and closed forms."""
import torch
from transformers.models.qwen3 import modeling_qwen3 as hf

from oracle import pointwise as P


def test_rms_norm_matches_transformers_fp32():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(7, 64, generator=g)
    w = 1 + 0.02 * torch.randn(64, generator=g)
    mod = hf.Qwen3RMSNorm(64, eps=1e-6)
    mod.weight.data.copy_(w)
    assert torch.allclose(P.rms_norm(x, w, 1e-6), mod(x), atol=1e-6, rtol=1e-6)


def test_rms_norm_closed_forms_bf16():
    # Constant row c with unit weight: x * rsqrt(c^2 + eps) -> sign(c) (rounded).
    for c in (0.5, -3.0, 7.25):
        x = torch.full((2, 128), c).to(torch.bfloat16)
        y = P.rms_norm(x, torch.ones(128, dtype=torch.bfloat16), 0.0)
        assert (y.float() == (1.0 if c > 0 else -1.0)).all()
    # Rounding sequence: y = r(r(x * inv) * w) differs from r(x * inv * w).
    x = torch.tensor([[1.0, 3.0]]).to(torch.bfloat16)
    w = torch.tensor([1.0078125, 1.0078125]).to(torch.bfloat16)
    inv = torch.rsqrt(torch.tensor(5.0))
    expect = (x.float() * inv).to(torch.bfloat16).float() * w.float()
    assert torch.equal(P.rms_norm(x, w, 0.0), expect.to(torch.bfloat16))


def test_add_rms_norm_rounds_the_sum_first():
    x = torch.tensor([[1.0, 256.0]]).to(torch.bfloat16)
    r = torch.tensor([[1.0 / 512, 1.0]]).to(torch.bfloat16)
    y, merged = P.add_rms_norm(x, r, torch.ones(2, dtype=torch.bfloat16), 0.0)
    assert merged.float().tolist() == [[1.0, 256.0]]  # 1 + 2^-9 and 257 round in bf16
    assert torch.equal(y, P.rms_norm(merged, torch.ones(2, dtype=torch.bfloat16), 0.0))


def test_silu_and_mul_closed_forms():
    x = torch.tensor([[0.0, 2.0, 5.0, 3.0]])
    out = P.silu_and_mul(x)
    assert out[0, 0] == 0.0  # g = 0 -> 0
    assert torch.allclose(out[0, 1], (2.0 / (1 + torch.exp(torch.tensor(-2.0))) * 3.0))
    xb = torch.randn(4, 16).to(torch.bfloat16)
    g, u = xb[:, :8].float(), xb[:, 8:].float()
    expect = (torch.nn.functional.silu(g).to(torch.bfloat16).float() * u).to(torch.bfloat16)
    assert torch.equal(P.silu_and_mul(xb), expect)


def test_rope_tables_match_transformers_and_the_max_position_form():
    cfg = hf.Qwen3Config(head_dim=128, rope_theta=1e6, max_position_embeddings=2048,
                         hidden_size=256, num_attention_heads=2)
    rot = hf.Qwen3RotaryEmbedding(cfg)
    pos = torch.tensor([0, 1, 5, 1000, 2047])
    cos_hf, sin_hf = rot(torch.zeros(1, dtype=torch.float32), pos[None])
    cos, sin = P.rope_tables(pos, 128, 1e6, torch.float32)
    assert torch.allclose(cos[:, 0], cos_hf[0, :, :64], atol=1e-6)
    assert torch.allclose(sin[:, 0], sin_hf[0, :, :64], atol=1e-6)
    c2, s2 = P.rope_tables_from_max(pos, 128, 1e6, 2048, torch.bfloat16)
    c1, s1 = P.rope_tables(pos, 128, 1e6, torch.bfloat16)
    assert torch.equal(c1, c2) and torch.equal(s1, s2)


def test_qk_norm_rope_matches_transformers_fp32():
    g = torch.Generator().manual_seed(2)
    t, hq, hkv, d = 5, 4, 2, 64
    q = torch.randn(t, hq, d, generator=g)
    k = torch.randn(t, hkv, d, generator=g)
    qw = 1 + 0.02 * torch.randn(d, generator=g)
    kw = 1 + 0.02 * torch.randn(d, generator=g)
    pos = torch.tensor([0, 3, 17, 100, 999])
    cos, sin = P.rope_tables(pos, d, 1e6, torch.float32)
    oq, ok = P.qk_norm_rope(q, k, qw, kw, cos, sin)
    qn, kn = hf.Qwen3RMSNorm(d), hf.Qwen3RMSNorm(d)
    qn.weight.data.copy_(qw)
    kn.weight.data.copy_(kw)
    full_cos = torch.cat([cos, cos], -1)[:, 0][None]  # [1, T, D]
    full_sin = torch.cat([sin, sin], -1)[:, 0][None]
    eq, ek = hf.apply_rotary_pos_emb(qn(q).transpose(0, 1)[None], kn(k).transpose(0, 1)[None],
                                     full_cos, full_sin)
    assert torch.allclose(oq, eq[0].transpose(0, 1), atol=1e-5)
    assert torch.allclose(ok, ek[0].transpose(0, 1), atol=1e-5)


def test_rope_position_zero_is_identity_after_norm():
    q = torch.randn(1, 2, 128).to(torch.bfloat16)
    w = torch.ones(128, dtype=torch.bfloat16)
    cos, sin = P.rope_tables(torch.tensor([0]), 128, 1e6, torch.bfloat16)
    oq, _ = P.qk_norm_rope(q, q[:, :1], w, w, cos, sin)
    assert torch.equal(oq, P.rms_norm(q, w))
