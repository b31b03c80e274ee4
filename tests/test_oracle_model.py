"""Pin for oracle/model.py: transformers' Qwen3ForCausalLM with the same
weights, with tied embeddings (the 0.6B route: logits from the embedding
matrix) and with an own ``lm_head`` (the 8B / 32B route)."""
import dataclasses

import pytest
import torch
from transformers import Qwen3Config, Qwen3ForCausalLM

from oracle import model as M

CFG = M.TinyQwen3(vocab_size=97, hidden_size=64, intermediate_size=96,
                  num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                  head_dim=16)


def _hf_model(cfg_o, weights):
    CFG = cfg_o
    cfg = Qwen3Config(vocab_size=CFG.vocab_size, hidden_size=CFG.hidden_size,
                      intermediate_size=CFG.intermediate_size,
                      num_hidden_layers=CFG.num_hidden_layers,
                      num_attention_heads=CFG.num_attention_heads,
                      num_key_value_heads=CFG.num_key_value_heads, head_dim=CFG.head_dim,
                      rope_theta=CFG.rope_theta, rms_norm_eps=CFG.rms_norm_eps,
                      tie_word_embeddings=CFG.tie_word_embeddings, max_position_embeddings=512,
                      attention_bias=False)
    cfg._attn_implementation = "eager"
    model = Qwen3ForCausalLM(cfg).float().eval()
    q = CFG.num_attention_heads * CFG.head_dim
    kv = CFG.num_key_value_heads * CFG.head_dim
    state = {}
    for name, tensor in weights.items():
        if name.endswith("qkv_proj.weight"):
            base = name[: -len("qkv_proj.weight")]
            state[base + "q_proj.weight"] = tensor[:q]
            state[base + "k_proj.weight"] = tensor[q:q + kv]
            state[base + "v_proj.weight"] = tensor[q + kv:]
        elif name.endswith("gate_up_proj.weight"):
            base = name[: -len("gate_up_proj.weight")]
            state[base + "gate_proj.weight"] = tensor[:CFG.intermediate_size]
            state[base + "up_proj.weight"] = tensor[CFG.intermediate_size:]
        else:
            state[name] = tensor
    missing, unexpected = model.load_state_dict(state, strict=False)
    assert not unexpected, unexpected
    if CFG.tie_word_embeddings:
        assert all("lm_head" in m for m in missing), missing
        assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()
    else:
        assert not missing, missing
    return model


@pytest.mark.parametrize("tied", [True, False])
def test_forward_matches_transformers_fp32(tied):
    cfg = dataclasses.replace(CFG, tie_word_embeddings=tied)
    weights = M.random_weights(cfg, seed=0, dtype=torch.float32, std=0.2)
    assert ("lm_head.weight" in weights) == (not tied)
    ids = [5, 17, 3, 96, 40, 40, 2, 11, 0, 63]
    ours = M.forward(cfg, weights, ids)
    with torch.no_grad():
        ref = _hf_model(cfg, weights)(torch.tensor([ids])).logits[0]
    assert torch.allclose(ours, ref, atol=2e-5, rtol=1e-4), (ours - ref).abs().max()
    if not tied:
        # The own head is the one used: the embedding matrix would give
        # other logits.
        other = M.forward(cfg, {**weights, "lm_head.weight": weights["model.embed_tokens.weight"]},
                          ids)
        assert not torch.allclose(other, ref, atol=1e-2)


def test_forward_logit_rows_select_positions():
    cfg = dataclasses.replace(CFG, tie_word_embeddings=False)
    weights = M.random_weights(cfg, seed=1, dtype=torch.float32, std=0.2)
    ids = [5, 17, 3, 96, 40, 40, 2, 11, 0, 63]
    full = M.forward(cfg, weights, ids)
    rows = [9, 3, 4]
    assert torch.allclose(M.forward(cfg, weights, ids, logit_rows=rows), full[rows],
                          rtol=1e-6, atol=1e-6)


def test_linear_k_slices_is_the_same_product_in_another_summation_order():
    """Sliced sums equal the float64 product to fp32 accuracy before the one
    rounding (so the bf16 outputs differ from the unsliced ones by at most a
    rounding flip), and exactly on integer data, where every fp32 sum is
    exact; an uneven split (K not divisible) covers every column once."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(7, 1000, generator=g).to(torch.bfloat16)
    w = (0.02 * torch.randn(33, 1000, generator=g)).to(torch.bfloat16)
    exact = x.double() @ w.double().t()
    for k in (1, 3, 4, 8):
        y = M.linear(x, w, k_slices=k)
        ulp = torch.exp2(torch.floor(torch.log2(exact.abs().clamp_min(1e-30))) - 7)
        assert ((y.double() - exact).abs() <= ulp).all(), k
    xi = torch.randint(-8, 9, (5, 999), generator=g).to(torch.bfloat16)
    wi = torch.randint(-8, 9, (6, 999), generator=g).to(torch.bfloat16)
    ref = (xi.double() @ wi.double().t()).to(torch.bfloat16)
    for k in (1, 2, 7):
        assert torch.equal(M.linear(xi, wi, k_slices=k), ref)


def test_forward_k_slices_changes_only_roundings():
    cfg = dataclasses.replace(CFG, tie_word_embeddings=False)
    weights = M.random_weights(cfg, seed=2, dtype=torch.bfloat16, std=0.2)
    ids = [5, 17, 3, 96, 40, 40, 2, 11, 0, 63]
    a = M.forward(cfg, weights, ids)
    b = M.forward(cfg, weights, ids, k_slices=4)
    assert (a - b).abs().max() < 0.05 * a.abs().max()
