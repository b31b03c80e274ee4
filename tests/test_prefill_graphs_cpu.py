"""Which steps replay a captured prefill graph, and in which (token, item)
bucket (host logic of tinyvllm/runtime/prefill_graphs.py; no GPU)."""
from helpers import ManualBatches

from tinyvllm.runtime.prefill_graphs import DECODE_CONTEXT_BOUND, PrefillInputs


def _inputs(max_tokens=2048, max_items=16, pitch_pages=64):
    inputs = PrefillInputs.__new__(PrefillInputs)  # bucket logic only: no buffers
    inputs.max_tokens, inputs.max_items = max_tokens, max_items
    inputs.table_capacity = max_items * pitch_pages
    return inputs


def _batch(prompts, items, done=None, num_blocks=1024):
    mb = ManualBatches(prompts, block_size=16, num_blocks=num_blocks)
    if done:
        for seq, n in done.items():
            mb.done[seq] = n
    return mb.step(items)


def test_prefill_buckets_round_up():
    p = [[1] * 700] * 3
    assert _inputs().buckets_for(_batch(p, [(0, 37, True), (1, 5, True)])) == (64, 2)
    assert _inputs().buckets_for(_batch(p, [(0, 600, True)])) == (768, 1)
    assert _inputs().buckets_for(_batch(p, [(0, 2, True), (1, 3, True), (2, 4, True)])) == (32, 4)
    # the bucket ceiling follows max_tokens (the cache's slot count caps it)
    assert _inputs(max_tokens=512).buckets_for(_batch(p, [(0, 600, True)])) is None
    assert _inputs(max_tokens=600).buckets_for(_batch(p, [(0, 500, True)])) == (512, 1)


def test_decode_only_and_long_decode_rows_stay_off_the_prefill_graphs():
    p = [[1] * 2000] * 3
    # every item a single token: a decode step (it has graphs of its own)
    assert _inputs().buckets_for(_batch(p, [(0, 1, True), (1, 1, True)],
                                        done={0: 100, 1: 100})) is None
    # a decode row of short context rides along in the prefill kernel
    short = _batch(p, [(0, 1, True), (1, 64, True)], done={0: DECODE_CONTEXT_BOUND - 1})
    assert _inputs().buckets_for(short) == (128, 2)
    # beyond the bound the split-K decode kernel is faster: eager
    long = _batch(p, [(0, 1, True), (1, 64, True)], done={0: DECODE_CONTEXT_BOUND})
    assert _inputs().buckets_for(long) is None


def test_item_and_table_limits():
    p = [[1] * 40] * 20
    many = _batch(p, [(s, 2, True) for s in range(17)])
    assert _inputs().buckets_for(many) is None            # 17 items > 16
    assert _inputs().buckets_for(_batch(p, [(s, 2, True) for s in range(16)])) == (32, 16)
    assert _inputs(max_items=4).buckets_for(_batch(p, [(s, 2, True) for s in range(5)])) is None
    # block tables beyond the packed capacity
    assert _inputs(max_items=1, pitch_pages=2).buckets_for(_batch(p, [(0, 40, True)])) is None
    assert _inputs(max_items=1, pitch_pages=3).buckets_for(_batch(p, [(0, 40, True)])) == (64, 1)


def test_graph_token_ceiling_follows_the_model_size():
    """Prefill graphs cover steps whose dense GEMMs the host launches would
    otherwise outrun: up to 2048 tokens at 0.6B, 512 at 8B, 128 at 32B."""
    import torch

    from tinyvllm.models.qwen3 import Qwen3Config, Qwen3ForCausalLM
    from tinyvllm.runtime.runner import default_prefill_graph_tokens

    shapes = {  # hidden, intermediate, layers, q heads, kv heads
        2048: (1024, 3072, 28, 16, 8), 512: (4096, 12288, 36, 32, 8),
        128: (5120, 25600, 64, 64, 8)}
    for expected, (hidden, inter, layers, hq, hkv) in shapes.items():
        cfg = Qwen3Config.from_dict(dict(
            model_type="qwen3", vocab_size=151936, hidden_size=hidden,
            intermediate_size=inter, num_hidden_layers=layers, num_attention_heads=hq,
            num_key_value_heads=hkv, head_dim=128, max_position_embeddings=40960,
            rope_theta=1e6, tie_word_embeddings=False))
        model = Qwen3ForCausalLM(cfg, device="meta", dtype=torch.bfloat16)
        assert default_prefill_graph_tokens(model) == expected
