"""safetensors loading (reference checkpoint.py:84-143, weight routes
qwen3.py:569-648) on the CPU: HF tensor names are routed into the packed
qkv / gate_up projections bit-exactly, sharded checkpoints follow their
index, and missing / duplicated / unexpected tensors fail loudly."""
import json

import pytest
import torch
from safetensors.torch import save_file

from checkpoint_util import hf_tensors, write_checkpoint
from oracle import model as OM

CFG = OM.TinyQwen3(vocab_size=320, hidden_size=128, intermediate_size=192,
                   num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                   head_dim=32, tie_word_embeddings=False, max_position_embeddings=512)


@pytest.mark.parametrize("shards,tied", [(1, False), (3, False), (2, True)])
def test_checkpoint_round_trip(tmp_path, shards, tied):
    from tinyvllm.models.qwen3 import Qwen3ForCausalLM

    cfg = OM.TinyQwen3(**{**CFG.__dict__, "tie_word_embeddings": tied})
    weights = OM.random_weights(cfg, seed=4, dtype=torch.bfloat16)
    write_checkpoint(tmp_path, cfg, weights, shards=shards, eos_token_id=[7, 9])
    model = Qwen3ForCausalLM.from_pretrained(tmp_path, device="cpu", dtype=torch.bfloat16)
    assert model.config.eos_token_id == (7, 9)
    params = dict(model.named_parameters())
    for name, tensor in weights.items():
        if name == "lm_head.weight" and tied:
            continue
        assert torch.equal(params[name], tensor), name
    assert torch.equal(model.lm_head_weight, weights["lm_head.weight" if not tied
                                                    else "model.embed_tokens.weight"])


def test_checkpoint_errors(tmp_path):
    from tinyvllm.models.qwen3 import Qwen3ForCausalLM

    weights = OM.random_weights(CFG, seed=5, dtype=torch.bfloat16)
    tensors = hf_tensors(CFG, weights)
    write_checkpoint(tmp_path, CFG, weights)
    # missing tensor
    missing = dict(tensors)
    missing.pop("model.layers.1.mlp.up_proj.weight")
    save_file(missing, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match="missing"):
        Qwen3ForCausalLM.from_pretrained(tmp_path, device="cpu", dtype=torch.bfloat16)
    # unexpected name
    extra = dict(tensors)
    extra["model.layers.0.mlp.bogus.weight"] = torch.zeros(2)
    save_file(extra, str(tmp_path / "model.safetensors"))
    with pytest.raises(KeyError, match="unexpected"):
        Qwen3ForCausalLM.from_pretrained(tmp_path, device="cpu", dtype=torch.bfloat16)
    # wrong shape
    bad = dict(tensors)
    bad["model.norm.weight"] = torch.ones(CFG.hidden_size + 1, dtype=torch.bfloat16)
    save_file(bad, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match="shape"):
        Qwen3ForCausalLM.from_pretrained(tmp_path, device="cpu", dtype=torch.bfloat16)
    # the same tensor in two shards
    (tmp_path / "model.safetensors").unlink()
    save_file(tensors, str(tmp_path / "a.safetensors"))
    save_file({"model.norm.weight": tensors["model.norm.weight"]},
              str(tmp_path / "b.safetensors"))
    with pytest.raises(ValueError, match="twice"):
        Qwen3ForCausalLM.from_pretrained(tmp_path, device="cpu", dtype=torch.bfloat16)
    # unsupported configs
    cfg = json.loads((tmp_path / "config.json").read_text())
    for key, value in (("model_type", "llama"), ("hidden_act", "gelu"),
                       ("rope_scaling", {"rope_type": "yarn", "factor": 4.0})):
        (tmp_path / "config.json").write_text(json.dumps({**cfg, key: value}))
        with pytest.raises(ValueError):
            Qwen3ForCausalLM.from_pretrained(tmp_path, device="cpu", dtype=torch.bfloat16)
