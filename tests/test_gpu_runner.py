"""End-to-end runner/executor on the GPU vs the CPU oracle model.

A tiny random-init Qwen3 (head_dim 128, two layers) is prefilled in chunks
(MFMA prefill kernel, fused KV write) and then decoded greedily through the
captured hipGraphs; at >= 99% of steps the sampled token must be the CPU
oracle's greedy choice for the same context (teacher-forced)."""
import pytest
import torch

from helpers import ManualBatches
from oracle import model as OM

pytestmark = pytest.mark.gpu

CFG = OM.TinyQwen3(vocab_size=1000, hidden_size=256, intermediate_size=512,
                   num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                   head_dim=128, tie_word_embeddings=False, max_position_embeddings=1024)


def _our_model(weights, device):
    from tinyvllm.models.qwen3 import Qwen3Config, Qwen3ForCausalLM

    cfg = Qwen3Config.from_dict(dict(
        model_type="qwen3", vocab_size=CFG.vocab_size, hidden_size=CFG.hidden_size,
        intermediate_size=CFG.intermediate_size, num_hidden_layers=CFG.num_hidden_layers,
        num_attention_heads=CFG.num_attention_heads,
        num_key_value_heads=CFG.num_key_value_heads, head_dim=CFG.head_dim,
        max_position_embeddings=CFG.max_position_embeddings, rope_theta=CFG.rope_theta,
        tie_word_embeddings=CFG.tie_word_embeddings))
    model = Qwen3ForCausalLM(cfg, device=device, dtype=torch.bfloat16)
    q = CFG.num_attention_heads * CFG.head_dim
    kv = CFG.num_key_value_heads * CFG.head_dim
    for name, tensor in weights.items():
        t = tensor.to(device)
        if name.endswith("qkv_proj.weight"):
            base = name[:-len("qkv_proj.weight")]
            model.load_weight(base + "q_proj.weight", t[:q])
            model.load_weight(base + "k_proj.weight", t[q:q + kv])
            model.load_weight(base + "v_proj.weight", t[q + kv:])
        elif name.endswith("gate_up_proj.weight"):
            base = name[:-len("gate_up_proj.weight")]
            model.load_weight(base + "gate_proj.weight", t[:CFG.intermediate_size])
            model.load_weight(base + "up_proj.weight", t[CFG.intermediate_size:])
        else:
            model.load_weight(name, t)
    return model.eval()


@pytest.mark.parametrize("enforce_eager", [False, True])
def test_greedy_decode_matches_oracle(device, enforce_eager):
    from tinyvllm.executor import Executor

    weights = OM.random_weights(CFG, seed=1, dtype=torch.bfloat16, std=0.2)
    model = _our_model(weights, device)
    g = torch.Generator().manual_seed(3)
    prompts = [torch.randint(0, CFG.vocab_size, (n,), generator=g).tolist()
               for n in (37, 5, 80)]
    executor = Executor(model, block_size=16, num_blocks=48, max_model_len=512,
                        max_num_seqs=4, enforce_eager=enforce_eager)
    mb = ManualBatches(prompts, block_size=16, num_blocks=48)
    # Chunked prefill: seq 0 in chunks of 20 + 17, seq 1 whole, seq 2 as 64 + 16.
    for items in ([(0, 20, False), (1, 5, True)], [(0, 17, True), (2, 64, False)],
                  [(2, 16, True)]):
        res = executor.execute(mb.step(items))
        mb.commit(items, res.sampled_token_ids)
    new = 12
    for _ in range(new - 1):
        items = [(s, 1, True) for s in range(3)]
        res = executor.execute(mb.step(items))
        mb.commit(items, res.sampled_token_ids)
    from test_gpu_engine import teacher_forced_agreement

    for s, prompt in enumerate(prompts):
        ours = mb.tokens[s][len(prompt):]
        assert teacher_forced_agreement(weights, prompt, ours) / new >= 0.99, (s, ours)


def test_logits_match_oracle_at_every_position(device):
    """Prefill logits of the sampled position vs the oracle's, bf16 tolerance."""
    from tinyvllm.executor import Executor

    weights = OM.random_weights(CFG, seed=2, dtype=torch.bfloat16, std=0.2)
    model = _our_model(weights, device)
    prompt = torch.randint(0, CFG.vocab_size, (150,), generator=torch.Generator().manual_seed(4)).tolist()
    executor = Executor(model, block_size=16, num_blocks=16, max_model_len=256,
                        max_num_seqs=2, enforce_eager=True)
    mb = ManualBatches([prompt], block_size=16, num_blocks=16)
    logits = executor.runner.run(mb.step([(0, 150, True)]))
    expect = OM.forward(CFG, weights, prompt)[-1]
    diff = (logits[0].float().cpu() - expect).abs()
    assert diff.max() < 0.15 and diff.mean() / expect.abs().mean() < 2e-2, diff.max()


def _decode_run(model, prompts, *, enforce_eager, pipelined):
    """Prefill seqs 0-2, then 10 decode steps over them; seq 3 joins with a
    whole-prompt prefill in a mixed step. Pipelined: step k+1 is launched
    before step k's tokens reach the host, its decode inputs naming step k's
    sampled rows (input_token_sources)."""
    import dataclasses

    from tinyvllm.executor import Executor

    executor = Executor(model, block_size=16, num_blocks=64, max_model_len=512,
                        max_num_seqs=4, enforce_eager=enforce_eager)
    mb = ManualBatches(prompts, block_size=16, num_blocks=64)
    for items in ([(0, 37, True), (1, 5, True)], [(2, 80, True)]):
        mb.commit(items, executor.execute(mb.step(items)).sampled_token_ids)
    pending = None  # (PendingStep, {seq: (sample row, placeholder index)})
    for step in range(10):
        items = [(s, 1, True) for s in range(3 if step < 4 else 4)]
        if step == 4:
            items[3] = (3, len(prompts[3]), True)
        batch = mb.step(items)
        if pipelined and pending is not None:
            rows = pending[1]
            src = []
            for seq, n, _ in items:
                src += [rows[seq][0] if seq in rows else -1] + [-1] * (n - 1)
            batch = dataclasses.replace(batch, input_token_sources=tuple(src))
        launched = executor.launch(batch)
        if not pipelined:
            mb.commit(items, launched.result().sampled_token_ids)
            continue
        # Placeholders now; the real ids once the step's result arrives.
        mb.commit(items, [0] * len(items))
        rows = {seq: (r, len(mb.tokens[seq]) - 1) for r, (seq, _, _) in enumerate(items)}
        if pending is not None:
            for seq, tok in zip(pending[0].sample_request_ids,
                                pending[0].result().sampled_token_ids):
                mb.tokens[seq][pending[1][seq][1]] = tok
        pending = (launched, rows)
    if pending is not None:
        for seq, tok in zip(pending[0].sample_request_ids, pending[0].result().sampled_token_ids):
            mb.tokens[seq][pending[1][seq][1]] = tok
    return mb.tokens


@pytest.mark.parametrize("enforce_eager", [False, True])
def test_pipelined_launches_match_sequential_steps(device, enforce_eager):
    """Device-side input ids (the previous step's sampled rows) give exactly
    the tokens of steps whose ids went through the host."""
    weights = OM.random_weights(CFG, seed=5, dtype=torch.bfloat16, std=0.2)
    model = _our_model(weights, device)
    g = torch.Generator().manual_seed(6)
    prompts = [torch.randint(0, CFG.vocab_size, (n,), generator=g).tolist()
               for n in (37, 5, 80, 23)]
    seq = _decode_run(model, prompts, enforce_eager=enforce_eager, pipelined=False)
    pipe = _decode_run(model, prompts, enforce_eager=enforce_eager, pipelined=True)
    assert pipe == seq
    assert all(len(t) > len(p) for t, p in zip(seq, prompts))


def test_token_sources_are_validated(device):
    import dataclasses

    from tinyvllm.executor import Executor

    weights = OM.random_weights(CFG, seed=5, dtype=torch.bfloat16, std=0.2)
    executor = Executor(_our_model(weights, device), block_size=16, num_blocks=16,
                        max_model_len=256, max_num_seqs=2, enforce_eager=True)
    mb = ManualBatches([[1, 2, 3]], block_size=16, num_blocks=16)
    batch = mb.step([(0, 3, True)])
    with pytest.raises(ValueError, match="previous step"):  # nothing launched yet
        executor.execute(dataclasses.replace(batch, input_token_sources=(-1, -1, 0)))
    with pytest.raises(ValueError, match="one entry per token"):
        executor.execute(dataclasses.replace(batch, input_token_sources=(-1,)))


@pytest.mark.parametrize("kv_dtype", [None, torch.float8_e4m3fn])
def test_prefill_graphs_match_eager_prefill(device, monkeypatch, kv_dtype):
    """Prefill and mixed steps replayed from the captured bucket graphs
    (padded tokens write no KV, padded items are empty, single-token items
    go through the prefill kernel) give the eager path's logits within bf16
    tolerance and the same greedy tokens; the KV both write then decodes to
    the same tokens."""
    from tinyvllm.executor import Executor
    from tinyvllm.runtime.prefill_graphs import PrefillGraphs

    replays = []
    original = PrefillGraphs.replay

    def counted(self, tokens, items):
        replays.append((tokens, items))
        return original(self, tokens, items)

    monkeypatch.setattr(PrefillGraphs, "replay", counted)
    weights = OM.random_weights(CFG, seed=7, dtype=torch.bfloat16, std=0.2)
    model = _our_model(weights, device)
    g = torch.Generator().manual_seed(8)
    prompts = [torch.randint(0, CFG.vocab_size, (n,), generator=g).tolist()
               for n in (37, 5, 80, 300, 2, 9, 64, 17, 33, 700)]
    steps = ([(0, 37, True), (1, 5, True)], [(2, 40, False), (3, 150, False)],
             [(2, 40, True), (3, 150, True), (4, 2, True), (5, 9, True)],
             [(0, 1, True), (1, 1, True), (6, 64, True), (7, 17, True), (8, 33, True)],
             [(9, 700, True)],
             [(s, 1, True) for s in range(10)])
    results = {}
    forced = None  # the graph run commits the eager run's tokens (teacher forcing)
    for eager in (True, False):
        executor = Executor(model, block_size=16, num_blocks=480, max_model_len=1024,
                            max_num_seqs=12, enforce_eager=eager, kv_cache_dtype=kv_dtype,
                            kv_scales=(0.5, 0.5) if kv_dtype else (1.0, 1.0))
        mb = ManualBatches(prompts, block_size=16, num_blocks=480)
        logits, tokens = [], []
        for step, items in enumerate(steps):
            batch = mb.step(items)
            out = executor.runner.run_and_sample(batch, [0] * batch.num_samples)
            if out is None:
                mb.commit(items, [])
                continue
            logits.append(out[0].float().cpu())
            tokens.append(out[1].cpu().tolist())
            mb.commit(items, tokens[-1] if forced is None else forced[len(tokens) - 1])
        results[eager] = (logits, tokens)
        forced = tokens
        executor.clear()
    assert replays == [(64, 2), (192, 2), (256, 4), (128, 8), (768, 1)]
    # Single-token items run the prefill kernel instead of the split-K
    # decode kernel: a different summation order, whose rounding the next
    # layer carries into the logits: the end-to-end logit bar of these tests.
    for a, b in zip(results[True][0], results[False][0]):
        diff = (a - b).abs()
        assert diff.max() < 0.15 and diff.mean() / a.abs().mean() < 2e-2, diff.max()
    # Greedy tokens agree but for near-ties of the eager logits (within the
    # logit bar above).
    for lg, te, tg in zip(results[True][0], results[True][1], results[False][1]):
        for row, (x, y) in enumerate(zip(te, tg)):
            assert x == y or abs(lg[row, x] - lg[row, y]).item() < 0.15, (row, x, y)


@pytest.mark.parametrize("kv_dtype", [None, torch.float8_e4m3fn])
def test_cache_layouts_give_bit_identical_runs(device, kv_dtype):
    """The kernels address K/V through the cache's slot and head strides and
    do the same arithmetic in either storage order, so a whole run (chunked
    prefill through the prefill graphs, then graph-replayed decode steps)
    gives bit-identical logits and tokens on a token-major and a head-major
    cache."""
    from tinyvllm.executor import Executor

    weights = OM.random_weights(CFG, seed=9, dtype=torch.bfloat16, std=0.2)
    model = _our_model(weights, device)
    g = torch.Generator().manual_seed(10)
    prompts = [torch.randint(0, CFG.vocab_size, (n,), generator=g).tolist()
               for n in (37, 5, 80, 130)]
    steps = ([(0, 37, True), (1, 5, True)], [(2, 80, True), (3, 64, False)],
             [(3, 66, True)]) + tuple([(s, 1, True) for s in range(4)] for _ in range(6))
    runs = {}
    for layout in ("token_major", "head_major"):
        executor = Executor(model, block_size=16, num_blocks=64, max_model_len=512,
                            max_num_seqs=4, kv_cache_dtype=kv_dtype,
                            kv_scales=(0.5, 0.5) if kv_dtype else (1.0, 1.0),
                            kv_cache_layout=layout)
        assert executor.runner.kv_cache.layout == layout
        mb = ManualBatches(prompts, block_size=16, num_blocks=64)
        logits, tokens = [], []
        for items in steps:
            batch = mb.step(items)
            out = executor.runner.run_and_sample(batch, [0] * batch.num_samples)
            if out is None:
                mb.commit(items, [])
                continue
            logits.append(out[0].cpu())
            tokens.append(out[1].cpu().tolist())
            mb.commit(items, tokens[-1])
        runs[layout] = (logits, tokens)
        executor.clear()
    assert runs["token_major"][1] == runs["head_major"][1]
    for a, b in zip(runs["token_major"][0], runs["head_major"][0]):
        assert torch.equal(a, b)


def test_prefill_graphs_exact_fallback_for_v_beyond_fp16(device, monkeypatch):
    """A cache holding V values beyond the fp16 range (layer 0's V rows of
    the packed projection scaled by 4e4): the prefill graphs' replays take
    the exact bf16 fallback launch like eager prefill does, give the eager
    logits and tokens, and leave the graphs' own fallback guard clear."""
    from tinyvllm.executor import Executor
    from tinyvllm.runtime.prefill_graphs import PrefillGraphs

    replays = []
    original = PrefillGraphs.replay

    def counted(self, tokens, items):
        replays.append((tokens, items))
        return original(self, tokens, items)

    monkeypatch.setattr(PrefillGraphs, "replay", counted)
    weights = OM.random_weights(CFG, seed=11, dtype=torch.bfloat16, std=0.2)
    name = "model.layers.0.self_attn.qkv_proj.weight"
    q = CFG.num_attention_heads * CFG.head_dim
    kv = CFG.num_key_value_heads * CFG.head_dim
    w = weights[name].float()
    w[q + kv:] *= 4.0e4
    weights[name] = w.to(torch.bfloat16)
    model = _our_model(weights, device)
    g = torch.Generator().manual_seed(12)
    prompts = [torch.randint(0, CFG.vocab_size, (n,), generator=g).tolist()
               for n in (37, 120, 64)]
    steps = ([(0, 37, True), (1, 60, False)], [(1, 60, True), (2, 64, True)])
    results = {}
    for eager in (True, False):
        executor = Executor(model, block_size=16, num_blocks=64, max_model_len=512,
                            max_num_seqs=4, enforce_eager=eager)
        runner = executor.runner
        assert (runner.prefill_graphs is None) == eager
        mb = ManualBatches(prompts, block_size=16, num_blocks=64)
        logits, tokens = [], []
        for items in steps:
            batch = mb.step(items)
            out = runner.run_and_sample(batch, [0] * batch.num_samples)
            logits.append(out[0].float().cpu())
            tokens.append(out[1].cpu().tolist())
            mb.commit(items, tokens[-1])
        torch.cuda.synchronize()
        v0 = runner.kv_cache.value[0].float()  # slots never written hold NaN
        assert torch.nan_to_num(v0, nan=0.0).abs().max().item() >= 65536.0
        if not eager:
            guard = runner.prefill_graphs.guard
            assert guard is not None and int(guard.count_nonzero()) == 0
        results[eager] = (logits, tokens)
        executor.clear()
    assert len(replays) == len(steps)
    # Padded buckets may run other GEMM tilings than the eager step: the
    # end-to-end logit bar of the graph test above.
    assert results[True][1] == results[False][1]
    for a, b in zip(results[True][0], results[False][0]):
        assert torch.isfinite(b).all()
        diff = (a - b).abs()
        assert diff.max() < 0.15 and diff.mean() / a.abs().mean() < 2e-2, diff.max()
