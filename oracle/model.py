"""Qwen3 forward restated on the CPU (test infrastructure only).

Follows the reference op order (tinyvllm/models/qwen3.py:263-303 attention,
:386-412 decoder layer, :458-494 model, :703-717 logits) with the oracle's
pointwise ops and fp32-softmax attention. Weights are a flat dict named like
the reference's parameters (qkv_proj packed q|k|v, gate_up_proj packed
gate|up). Linear layers multiply in fp32 and round to the storage dtype,
like a bf16 F.linear with fp32 accumulation.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from oracle import paged_kv as KV
from oracle import pointwise as P


@dataclass(frozen=True)
class TinyQwen3:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    rope_theta: float = 1_000_000.0
    rms_norm_eps: float = 1e-6
    tie_word_embeddings: bool = True
    max_position_embeddings: int = 4096


def random_weights(cfg: TinyQwen3, seed: int, dtype: torch.dtype,
                   std: float = 0.02) -> dict[str, torch.Tensor]:
    """N(0, std) matrices, norm weights 1 + N(0, std) (CPU, given dtype)."""
    g = torch.Generator().manual_seed(seed)

    def mat(*shape):
        return (torch.randn(*shape, generator=g) * std).to(dtype)

    def norm(n):
        return (1.0 + torch.randn(n, generator=g) * std).to(dtype)

    q = cfg.num_attention_heads * cfg.head_dim
    kv = cfg.num_key_value_heads * cfg.head_dim
    w = {"model.embed_tokens.weight": mat(cfg.vocab_size, cfg.hidden_size),
         "model.norm.weight": norm(cfg.hidden_size)}
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}"
        w[f"{p}.input_layernorm.weight"] = norm(cfg.hidden_size)
        w[f"{p}.post_attention_layernorm.weight"] = norm(cfg.hidden_size)
        w[f"{p}.self_attn.qkv_proj.weight"] = mat(q + 2 * kv, cfg.hidden_size)
        w[f"{p}.self_attn.o_proj.weight"] = mat(cfg.hidden_size, q)
        w[f"{p}.self_attn.q_norm.weight"] = norm(cfg.head_dim)
        w[f"{p}.self_attn.k_norm.weight"] = norm(cfg.head_dim)
        w[f"{p}.mlp.gate_up_proj.weight"] = mat(2 * cfg.intermediate_size, cfg.hidden_size)
        w[f"{p}.mlp.down_proj.weight"] = mat(cfg.hidden_size, cfg.intermediate_size)
    if not cfg.tie_word_embeddings:
        w["lm_head.weight"] = mat(cfg.vocab_size, cfg.hidden_size)
    return w


def linear(x: torch.Tensor, w: torch.Tensor, k_slices: int = 1) -> torch.Tensor:
    """bf16-style linear: fp32 products and sums, one rounding to x's dtype.
    ``k_slices > 1`` sums the reduction in that many contiguous slices (each
    an fp32 matmul, added in slice order) - the same arithmetic in another
    fp32 summation order, as a split-K GEMM does it."""
    if k_slices == 1:
        return (x.float() @ w.float().t()).to(x.dtype)
    k = x.shape[-1]
    bounds = [k * i // k_slices for i in range(k_slices + 1)]
    acc = None
    for lo, hi in zip(bounds, bounds[1:]):
        part = x[..., lo:hi].float() @ w[:, lo:hi].float().t()
        acc = part if acc is None else acc + part
    return acc.to(x.dtype)


def forward(cfg: TinyQwen3, w: dict[str, torch.Tensor], token_ids: list[int],
            kv_fp8: tuple[float, float] | None = None,
            logit_rows: list[int] | None = None, k_slices: int = 1) -> torch.Tensor:
    """Full causal forward of one sequence; logits [L, vocab] (storage-dtype values).
    ``kv_fp8=(k_scale, v_scale)`` attends over K/V passed through the FP8 E4M3
    cache layout (quantised, then read back), as an engine with that layout
    does. ``logit_rows`` limits the LM head to those positions (logits
    [len(logit_rows), vocab]). ``k_slices`` sums every linear layer's
    reduction in that many slices (``linear``): the same rounding points in
    another fp32 summation order, which measures how far the bf16 roundings
    alone move the logits."""
    ids = torch.tensor(token_ids, dtype=torch.long)
    length = ids.numel()
    dtype = w["model.embed_tokens.weight"].dtype
    hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    hidden = w["model.embed_tokens.weight"][ids]
    cos, sin = P.rope_tables(torch.arange(length), d, cfg.rope_theta, dtype)
    residual = None
    causal = torch.arange(length)[None, :] <= torch.arange(length)[:, None]
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}"
        if residual is None:
            residual = hidden
            x = P.rms_norm(hidden, w[f"{p}.input_layernorm.weight"], cfg.rms_norm_eps)
        else:
            x, residual = P.add_rms_norm(hidden, residual, w[f"{p}.input_layernorm.weight"],
                                         cfg.rms_norm_eps)
        qkv = linear(x, w[f"{p}.self_attn.qkv_proj.weight"], k_slices)
        q = qkv[:, :hq * d].view(length, hq, d)
        k = qkv[:, hq * d:(hq + hkv) * d].view(length, hkv, d)
        v = qkv[:, (hq + hkv) * d:].view(length, hkv, d)
        q, k = P.qk_norm_rope(q, k, w[f"{p}.self_attn.q_norm.weight"],
                              w[f"{p}.self_attn.k_norm.weight"], cos, sin,
                              cfg.rms_norm_eps, cfg.rms_norm_eps)
        group = hq // hkv
        kf, vf = k.float(), v.float()
        if kv_fp8 is not None:
            kf = KV.fp8_dequantize(KV.fp8_quantize(k, kv_fp8[0]), kv_fp8[0])
            vf = KV.fp8_dequantize(KV.fp8_quantize(v, kv_fp8[1]), kv_fp8[1])
        kf = kf.repeat_interleave(group, 1)
        vf = vf.repeat_interleave(group, 1)
        s = torch.einsum("qhd,khd->hqk", q.float(), kf) * d ** -0.5
        s = s.masked_fill(~causal[None], float("-inf"))
        attn = torch.einsum("hqk,khd->qhd", torch.softmax(s, -1), vf).to(dtype)
        hidden = linear(attn.reshape(length, hq * d), w[f"{p}.self_attn.o_proj.weight"], k_slices)
        x, residual = P.add_rms_norm(hidden, residual,
                                     w[f"{p}.post_attention_layernorm.weight"], cfg.rms_norm_eps)
        gu = linear(x, w[f"{p}.mlp.gate_up_proj.weight"], k_slices)
        hidden = linear(P.silu_and_mul(gu), w[f"{p}.mlp.down_proj.weight"], k_slices)
    if logit_rows is not None:
        rows = torch.tensor(logit_rows, dtype=torch.long)
        hidden, residual = hidden[rows], residual[rows]
    hidden, _ = P.add_rms_norm(hidden, residual, w["model.norm.weight"], cfg.rms_norm_eps)
    head = w.get("lm_head.weight", w["model.embed_tokens.weight"])
    return linear(hidden, head, k_slices).float()  # bf16 logits, as F.linear produces


def greedy_generate(cfg: TinyQwen3, w, prompt: list[int], new_tokens: int) -> list[int]:
    """Greedy continuation by full recomputation (tiny configs only)."""
    seq = list(prompt)
    out = []
    for _ in range(new_tokens):
        logits = forward(cfg, w, seq)
        tok = int(logits[-1].argmax())
        out.append(tok)
        seq.append(tok)
    return out
