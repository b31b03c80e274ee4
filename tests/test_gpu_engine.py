"""Engine end to end on the GPU (scheduler + chunked prefill + prefix cache +
graph-replayed decode) vs the CPU oracle model's greedy continuation."""
import pytest
import torch

from oracle import model as OM
from test_gpu_runner import CFG, _our_model

pytestmark = pytest.mark.gpu


def teacher_forced_agreement(weights, prompt, ours, tie=0.05, kv_fp8=None):
    """Steps at which our sampled token is the oracle's greedy choice given
    the same context (one oracle forward over prompt + ours). A step whose
    oracle top-2 logits differ by less than ``tie`` or one bf16 ulp of the
    top logit (|best| * 2^-7 bounds it), whichever is larger, accepts either
    token: GEMM accumulation order may legitimately flip such a near-tie, and
    the sequence then diverges."""
    logits = OM.forward(CFG, weights, list(prompt) + list(ours), kv_fp8=kv_fp8)
    agree = 0
    for i, token in enumerate(ours):
        row = logits[len(prompt) - 1 + i]
        best = row.max()
        slack = max(tie, float(best.abs()) * 2.0 ** -7)
        agree += int(row[token] >= best - slack if row.argmax() != token else True)
    return agree


def _engine(model, **kw):
    from tinyvllm.bootstrap import build_engine

    args = dict(max_model_len=512, max_num_seqs=4, max_num_batched_tokens=256,
                num_blocks=96, prefill_chunk_size=64, prefill_reserve_tokens=32,
                prefill_reserve_requests=1)
    args.update(kw)
    return build_engine(model, **args)


def test_engine_greedy_with_shared_prefixes_matches_oracle(device):
    from tinyvllm import GenerateRequest, SamplingParams

    weights = OM.random_weights(CFG, seed=5, dtype=torch.bfloat16, std=0.2)
    engine = _engine(_our_model(weights, device))
    g = torch.Generator().manual_seed(6)
    shared = torch.randint(0, CFG.vocab_size, (70,), generator=g).tolist()
    prompts = [shared + torch.randint(0, CFG.vocab_size, (n,), generator=g).tolist()
               for n in (3, 40, 1, 90)] + [torch.randint(0, CFG.vocab_size, (150,),
                                                         generator=g).tolist()]
    new = 10
    params = SamplingParams(max_new_tokens=new, ignore_eos=True)
    outs = engine.generate([GenerateRequest(p, params) for p in prompts])
    agree = total = 0
    for prompt, out in zip(prompts, outs):
        agree += teacher_forced_agreement(weights, prompt, out.output_token_ids)
        total += new
    assert agree / total >= 0.99, (agree, total)
    assert engine.scheduler.block_manager.prefix_cache.hits >= 1
    engine.close()


def test_engine_fp8_kv_cache_greedy_matches_fp8_oracle(device):
    """The optional FP8 E4M3 KV layout end to end (chunked prefill, prefix
    cache, graph-replayed decode): greedy tokens agree with the oracle model
    attending over the same FP8-quantised K/V."""
    from tinyvllm import GenerateRequest, SamplingParams

    weights = OM.random_weights(CFG, seed=8, dtype=torch.bfloat16, std=0.2)
    scales = (0.5, 0.25)
    engine = _engine(_our_model(weights, device), kv_cache_dtype=torch.float8_e4m3fn,
                     kv_scales=scales)
    assert engine.executor.runner.kv_cache.key.dtype == torch.float8_e4m3fn
    g = torch.Generator().manual_seed(9)
    shared = torch.randint(0, CFG.vocab_size, (70,), generator=g).tolist()
    prompts = [shared + torch.randint(0, CFG.vocab_size, (n,), generator=g).tolist()
               for n in (5, 33)] + [torch.randint(0, CFG.vocab_size, (120,),
                                                  generator=g).tolist()]
    new = 10
    params = SamplingParams(max_new_tokens=new, ignore_eos=True)
    outs = engine.generate([GenerateRequest(p, params) for p in prompts])
    agree = sum(teacher_forced_agreement(weights, p, o.output_token_ids, kv_fp8=scales)
                for p, o in zip(prompts, outs))
    assert agree / (new * len(prompts)) >= 0.99, agree
    engine.close()


def test_engine_sampling_is_seeded_and_in_vocab(device):
    from tinyvllm import GenerateRequest, SamplingParams

    weights = OM.random_weights(CFG, seed=7, dtype=torch.bfloat16, std=0.2)
    model = _our_model(weights, device)
    params = SamplingParams(max_new_tokens=12, temperature=0.8, top_p=0.9, top_k=50,
                            seed=1234, ignore_eos=True)
    prompts = [[3, 1, 4, 1, 5, 9, 2, 6], [2, 7, 1, 8, 2, 8]]
    runs = []
    for _ in range(2):
        engine = _engine(model, num_blocks=48)
        runs.append([o.output_token_ids for o in
                     engine.generate([GenerateRequest(p, params) for p in prompts])])
        engine.close()
    assert runs[0] == runs[1]
    assert all(0 <= t < CFG.vocab_size for out in runs[0] for t in out)
    assert runs[0][0] != runs[0][1]


def test_llm_from_engine_config_checkpoint(device, tmp_path):
    """The drop-in entry point: EngineConfig(model=<HF checkpoint dir>) ->
    LLM -> greedy token ids, checked against the oracle model."""
    from checkpoint_util import write_checkpoint
    from tinyvllm import SamplingParams
    from tinyvllm.config import EngineConfig
    from tinyvllm.serving.llm import LLM

    weights = OM.random_weights(CFG, seed=9, dtype=torch.bfloat16, std=0.2)
    write_checkpoint(tmp_path, CFG, weights, shards=2)

    class NoText:  # token-id use only; LLM never calls it with ids
        def decode(self, ids):
            return ""

    config = EngineConfig(model=tmp_path, max_model_len=512, max_num_seqs=4,
                          max_num_batched_tokens=256, prefill_chunk_size=64,
                          prefill_reserve_tokens=32, kv_cache_memory_bytes=8 << 20)
    g = torch.Generator().manual_seed(10)
    prompts = [torch.randint(0, CFG.vocab_size, (n,), generator=g).tolist() for n in (9, 130)]
    new = 10
    with LLM(config, tokenizer=NoText()) as llm:
        outs = llm.generate_token_ids(prompts, SamplingParams(max_new_tokens=new,
                                                              ignore_eos=True))
    agree = sum(teacher_forced_agreement(weights, p, o.output_token_ids)
                for p, o in zip(prompts, outs))
    assert agree / (new * len(prompts)) >= 0.99
    assert all(o.finish_reason == "length" and len(o.output_token_ids) == new for o in outs)


def test_engine_pipelined_eos_stops_early_and_frees_blocks(device):
    """Pipelined steps see EOS one step late, with the request's next row
    already launched: outputs must still end at the first EOS, follow the
    oracle, and every block return to the pool."""
    from tinyvllm import GenerateRequest, SamplingParams

    weights = OM.random_weights(CFG, seed=11, dtype=torch.bfloat16, std=0.2)
    model = _our_model(weights, device)
    g = torch.Generator().manual_seed(12)
    prompts = [torch.randint(0, CFG.vocab_size, (n,), generator=g).tolist()
               for n in (20, 45, 7)]
    free = _engine(model)
    ref = free.generate([GenerateRequest(p, SamplingParams(max_new_tokens=12, ignore_eos=True))
                         for p in prompts])
    free.close()
    eos = ref[0].output_token_ids[3]
    serial = _engine(model, eos_token_ids=[eos], pipelined=False)
    expect = serial.generate([GenerateRequest(p, SamplingParams(max_new_tokens=12))
                              for p in prompts])
    serial.close()
    engine = _engine(model, eos_token_ids=[eos])
    assert engine._pipelined
    outs = engine.generate([GenerateRequest(p, SamplingParams(max_new_tokens=12))
                            for p in prompts])
    # Same kernels, same tokens: pipelining changes when ids reach the host,
    # not which ids are sampled (one extra row per stopped request aside).
    assert [o.output_token_ids for o in outs] == [o.output_token_ids for o in expect]
    agree = total = 0
    for prompt, out in zip(prompts, outs):
        toks = list(out.output_token_ids)
        assert eos not in toks[:-1]
        assert toks[-1] == eos or len(toks) == 12
        agree += teacher_forced_agreement(weights, prompt, toks)
        total += len(toks)
    assert len(outs[0].output_token_ids) <= 4 and outs[0].output_token_ids[-1] == eos
    assert agree / total >= 0.99, (agree, total)
    manager = engine.scheduler.block_manager
    assert manager.free_block_count == manager.pool.num_blocks
    assert not engine.scheduler.has_unresolved_steps
    engine.close()
