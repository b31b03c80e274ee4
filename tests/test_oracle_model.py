"""Pin for oracle/model.py: transformers' Qwen3ForCausalLM with the same weights."""
import torch
from transformers import Qwen3Config, Qwen3ForCausalLM

from oracle import model as M

CFG = M.TinyQwen3(vocab_size=97, hidden_size=64, intermediate_size=96,
                  num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                  head_dim=16)


def _hf_model(weights):
    cfg = Qwen3Config(vocab_size=CFG.vocab_size, hidden_size=CFG.hidden_size,
                      intermediate_size=CFG.intermediate_size,
                      num_hidden_layers=CFG.num_hidden_layers,
                      num_attention_heads=CFG.num_attention_heads,
                      num_key_value_heads=CFG.num_key_value_heads, head_dim=CFG.head_dim,
                      rope_theta=CFG.rope_theta, rms_norm_eps=CFG.rms_norm_eps,
                      tie_word_embeddings=True, max_position_embeddings=512,
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
    assert not unexpected and all("lm_head" in m for m in missing), (missing, unexpected)
    return model


def test_forward_matches_transformers_fp32():
    weights = M.random_weights(CFG, seed=0, dtype=torch.float32, std=0.2)
    ids = [5, 17, 3, 96, 40, 40, 2, 11, 0, 63]
    ours = M.forward(CFG, weights, ids)
    with torch.no_grad():
        ref = _hf_model(weights)(torch.tensor([ids])).logits[0]
    assert torch.allclose(ours, ref, atol=2e-5, rtol=1e-4), (ours - ref).abs().max()
