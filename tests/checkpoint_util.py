"""Write an oracle weight dict as a HF-style Qwen3 checkpoint directory
(config.json + safetensors shards with separate q/k/v and gate/up tensors)."""
import json

import torch
from safetensors.torch import save_file


def hf_tensors(cfg, weights):
    q = cfg.num_attention_heads * cfg.head_dim
    kv = cfg.num_key_value_heads * cfg.head_dim
    out = {}
    for name, t in weights.items():
        if name.endswith("qkv_proj.weight"):
            base = name[:-len("qkv_proj.weight")]
            out[base + "q_proj.weight"] = t[:q]
            out[base + "k_proj.weight"] = t[q:q + kv]
            out[base + "v_proj.weight"] = t[q + kv:]
        elif name.endswith("gate_up_proj.weight"):
            base = name[:-len("gate_up_proj.weight")]
            out[base + "gate_proj.weight"] = t[:cfg.intermediate_size]
            out[base + "up_proj.weight"] = t[cfg.intermediate_size:]
        else:
            out[name] = t
    return {k: v.contiguous() for k, v in out.items()}


def write_checkpoint(path, cfg, weights, *, shards=1, eos_token_id=None):
    config = dict(model_type="qwen3", vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
                  intermediate_size=cfg.intermediate_size,
                  num_hidden_layers=cfg.num_hidden_layers,
                  num_attention_heads=cfg.num_attention_heads,
                  num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                  max_position_embeddings=cfg.max_position_embeddings,
                  rope_theta=cfg.rope_theta, rms_norm_eps=cfg.rms_norm_eps,
                  tie_word_embeddings=cfg.tie_word_embeddings, torch_dtype="bfloat16",
                  hidden_act="silu")
    if eos_token_id is not None:
        config["eos_token_id"] = eos_token_id
    (path / "config.json").write_text(json.dumps(config))
    tensors = hf_tensors(cfg, weights)
    names = sorted(tensors)
    if shards == 1:
        save_file(tensors, str(path / "model.safetensors"))
        return
    weight_map = {}
    for s in range(shards):
        part = {n: tensors[n] for n in names[s::shards]}
        fname = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        save_file(part, str(path / fname))
        weight_map.update({n: fname for n in part})
    (path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))


__all__ = ["hf_tensors", "write_checkpoint", "torch"]
