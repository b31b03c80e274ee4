"""Head dims other than 128 through the engine (the reference's decode
kernel dispatches head dims 32, 64, 128 and 256, paged_decode.cu:572-666).

Tiny random-init Qwen3 models with head_dim 32, 64 and 256 (and 64 over an
FP8 E4M3 cache) run the whole engine path - chunked prefill, graph-replayed
decode, greedy sampling - on the library's general attention kernel (the
fused and MFMA kernels take head_dim 128 only), with QK-norm + RoPE and the
slot-mapped KV write in their own kernel. Every sampled token is checked
teacher-forced against the CPU oracle model: it must be the oracle's argmax
for the same context, or within one bf16 ulp of it (a tie at bf16
resolution that another summation order may break). Over the FP8 cache the
oracle attends over its own quantisation of its own K/V; a one-ulp bf16
difference in a projection can move an E4M3 value by a whole FP8 step
(~6 %), so there a step also agrees within the 0.05 logit band the FP8
engine test of tests/test_gpu_engine.py uses. The oracle model
(oracle/model.py) is the same for every head dim and is pinned against
transformers' Qwen3 in tests/test_oracle_model.py."""
import math

import pytest
import torch

from oracle import model as OM

pytestmark = pytest.mark.gpu


def _model(cfg, device, seed):
    from tinyvllm.models.qwen3 import Qwen3Config, Qwen3ForCausalLM

    shape = dict(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
                 intermediate_size=cfg.intermediate_size,
                 num_hidden_layers=cfg.num_hidden_layers,
                 num_attention_heads=cfg.num_attention_heads,
                 num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                 max_position_embeddings=cfg.max_position_embeddings,
                 tie_word_embeddings=cfg.tie_word_embeddings)
    model = Qwen3ForCausalLM.random_init(
        Qwen3Config.from_dict(dict(model_type="qwen3", rope_theta=cfg.rope_theta, **shape)),
        device=device, seed=seed, std=0.05)
    return model, {n: p.detach().cpu() for n, p in model.named_parameters()}


@pytest.mark.parametrize("head_dim,heads,kv_heads,fp8", [
    (64, 8, 2, False), (256, 4, 2, False), (32, 6, 3, False), (64, 8, 2, True)])
def test_engine_greedy_at_other_head_dims_matches_oracle(device, head_dim, heads, kv_heads,
                                                         fp8):
    from tinyvllm import SamplingParams
    from tinyvllm.bootstrap import build_engine

    cfg = OM.TinyQwen3(vocab_size=700, hidden_size=256, intermediate_size=512,
                       num_hidden_layers=2, num_attention_heads=heads,
                       num_key_value_heads=kv_heads, head_dim=head_dim,
                       tie_word_embeddings=False, max_position_embeddings=1024)
    model, weights = _model(cfg, device, seed=head_dim + heads)
    scales = (0.25, 0.25) if fp8 else (1.0, 1.0)
    engine = build_engine(model, max_model_len=512, max_num_seqs=4,
                          max_num_batched_tokens=128, num_blocks=128, prefill_chunk_size=64,
                          kv_cache_dtype=torch.float8_e4m3fn if fp8 else None,
                          kv_scales=scales)
    runner = engine.executor.runner
    assert runner.kv_cache.head_dim == head_dim
    assert runner.decode_graphs is not None  # decode steps replay captured graphs
    g = torch.Generator().manual_seed(7)
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist()
               for n in (150, 37, 5, 90)]
    new = 12
    ids = [engine.submit(p, SamplingParams(max_new_tokens=new, ignore_eos=True))
           for p in prompts]
    out = {rid: [] for rid in ids}
    for _ in range(500):
        if not engine.has_unfinished():
            break
        for ev in engine.step().token_events:
            out[ev.request_id].append(ev.token_id)
    assert not engine.has_unfinished()
    engine.close()
    agree = total = 0
    worst = 0.0
    for prompt, rid in zip(prompts, ids):
        ours = out[rid]
        assert len(ours) == new
        rows = [len(prompt) - 1 + i for i in range(new)]
        logits = OM.forward(cfg, weights, prompt + ours, logit_rows=rows,
                            kv_fp8=scales if fp8 else None)
        for i, token in enumerate(ours):
            best = float(logits[i].max())
            ulp = 2.0 ** (math.floor(math.log2(abs(best))) - 7)
            deficit = (best - float(logits[i][token])) / ulp
            worst = max(worst, deficit)
            band = max(1.0, 0.05 / ulp) if fp8 else 1.0
            agree += int(deficit <= band)
            total += 1
    print(f"head_dim {head_dim} ({heads}Q/{kv_heads}KV{', fp8' if fp8 else ''}): "
          f"{agree}/{total} agree, worst deficit {worst:.1f} ulp")
    assert agree / total >= 0.99, (agree, total, worst)
