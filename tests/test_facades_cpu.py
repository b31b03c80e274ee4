"""The drop-in facades on the CPU: AsyncEngine (worker thread + asyncio
streams), AsyncLLM, LLM and EngineConfig, over the engine driven by the
slot-simulating fake executor of test_engine_cpu (no GPU)."""
import asyncio

import pytest

from test_engine_cpu import EOS, VOCAB, expected, make_engine
from tinyvllm.async_engine import (
    AsyncEngine, OverloadedError, RequestRejectedError, SlowConsumerError, WorkerError,
)
from tinyvllm.engine import TokenEvent
from tinyvllm.request import CompletionEvent, RequestStatus, SamplingParams


def factory(**kw):
    return lambda: make_engine(**kw)[0]


def slow_factory(delay_s=0.002, **kw):
    """An engine whose simulated executor takes ``delay_s`` per step, so a
    request cannot finish between two submits of the test."""
    import time

    def build():
        engine, ex = make_engine(**kw)
        for name in ("execute", "launch"):
            fn = getattr(ex, name, None)
            if fn is not None:
                def slowed(batch, _fn=fn):
                    time.sleep(delay_s)
                    return _fn(batch)
                setattr(ex, name, slowed)
        return engine
    return build


def run(coro):
    return asyncio.run(asyncio.wait_for(coro, timeout=60))


async def collect(stream):
    tokens, done = [], None
    async for item in stream:
        if isinstance(item, TokenEvent):
            tokens.append(item.token_id)
        else:
            done = item
    return tokens, done


@pytest.mark.parametrize("pipelined", [False, True], ids=["serial", "pipelined"])
def test_async_engine_concurrent_streams_match_the_model(pipelined):
    prompts = [[11 + i] * (3 + 5 * i) for i in range(5)]
    params = SamplingParams(max_new_tokens=9, ignore_eos=True)

    async def main():
        async with AsyncEngine(factory(pipelined=pipelined)) as bridge:
            streams = [await bridge.submit(p, params) for p in prompts]
            return await asyncio.gather(*(collect(s) for s in streams))

    for prompt, (tokens, done) in zip(prompts, run(main())):
        assert isinstance(done, CompletionEvent) and done.status is RequestStatus.FINISHED
        assert tokens == list(done.output_token_ids) == expected(prompt, params, 96)


@pytest.mark.parametrize("pipelined", [False, True], ids=["serial", "pipelined"])
def test_async_engine_cancel_overload_and_rejection(pipelined):
    params = SamplingParams(max_new_tokens=60, ignore_eos=True)

    async def main():
        async with AsyncEngine(slow_factory(pipelined=pipelined), max_requests=2) as bridge:
            a = await bridge.submit([7] * 5, params)
            b = await bridge.submit([8] * 5, params)
            with pytest.raises(OverloadedError):
                await bridge.submit([9] * 5, params)
            first = await a.__anext__()
            assert isinstance(first, TokenEvent)
            await a.aclose()  # cancels the request
            tokens, done = await collect(b)
            assert done.status is RequestStatus.FINISHED and len(tokens) == 60
            with pytest.raises(RequestRejectedError):  # longer than max_model_len
                await bridge.submit([6] * 200, SamplingParams(max_new_tokens=1))
            c = await bridge.submit([10] * 4, SamplingParams(max_new_tokens=3, ignore_eos=True))
            return await collect(c)

    tokens, done = run(main())
    assert done.status is RequestStatus.FINISHED and len(tokens) == 3


def test_async_engine_slow_consumer_is_cancelled():
    async def main():
        async with AsyncEngine(factory(), max_buffered_tokens=2) as bridge:
            s = await bridge.submit([12] * 6, SamplingParams(max_new_tokens=50, ignore_eos=True))
            await asyncio.sleep(0.5)  # let the worker run ahead of the reader
            with pytest.raises(SlowConsumerError):
                async for _ in s:
                    pass

    run(main())


def test_async_engine_worker_failure_ends_every_stream():
    def failing():
        engine, ex = make_engine()
        ex.fail_at = 2
        return engine

    async def main():
        async with AsyncEngine(failing) as bridge:
            s = await bridge.submit([13] * 30, SamplingParams(max_new_tokens=10))
            with pytest.raises(WorkerError):
                async for _ in s:
                    pass
            assert not bridge.is_running
            with pytest.raises(WorkerError):
                await bridge.submit([1], SamplingParams(max_new_tokens=1))

    run(main())


def test_async_engine_factory_error_surfaces_on_enter():
    def broken():
        raise RuntimeError("no device")

    async def main():
        with pytest.raises(WorkerError, match="no device"):
            async with AsyncEngine(broken):
                pass

    run(main())


@pytest.mark.parametrize("pipelined", [False, True], ids=["serial", "pipelined"])
def test_async_llm_streams_deltas_then_output(pipelined):
    from tinyvllm.serving.async_llm import AsyncLLM, TextDelta
    from tinyvllm.serving.llm import TextOutput

    params = SamplingParams(max_new_tokens=5, ignore_eos=True)

    async def main():
        async with AsyncLLM(engine_factory=factory(pipelined=pipelined)) as llm:
            items = [x async for x in llm.stream_token_ids([20, 21, 22], params)]
            out = await llm.generate_token_ids([23, 24], params)
            return items, out

    items, out = run(main())
    assert all(isinstance(x, TextDelta) for x in items[:-1]) and len(items) == 6
    last = items[-1]
    assert isinstance(last, TextOutput) and last.finish_reason == "length"
    assert list(last.output_token_ids) == [d.token_id for d in items[:-1]]
    assert list(last.output_token_ids) == expected([20, 21, 22], params, 96)
    assert list(out.output_token_ids) == expected([23, 24], params, 96)


def test_llm_facade_over_an_engine():
    from tinyvllm.serving.llm import LLM

    engine, _ = make_engine()
    prompts = [[30, 31, 32], [33] * 7]
    stop = SamplingParams(max_new_tokens=40)  # EOS allowed
    with LLM(engine=engine) as llm:
        outs = llm.generate_token_ids(prompts, stop)
        for prompt, out in zip(prompts, outs):
            want = expected(prompt, stop, 96)
            assert list(out.output_token_ids) == want
            assert out.text == ""
            assert out.prompt_token_count == len(prompt)
            assert out.finish_reason == ("stop" if want[-1] == EOS else "length")
        with pytest.raises(RuntimeError, match="tokenizer"):
            llm.generate("hello")
    with pytest.raises(RuntimeError, match="closed"):
        llm.generate_token_ids(prompts)


def test_llm_decodes_text_with_a_tokenizer():
    from tinyvllm.serving.llm import LLM

    class CharTokenizer:  # ids 0..VOCAB-1 <-> characters
        def encode(self, text):
            return [ord(c) % VOCAB for c in text]

        def decode(self, ids):
            return "".join(chr(48 + i % 40) for i in ids)

    engine, _ = make_engine()
    tok = CharTokenizer()
    params = SamplingParams(max_new_tokens=4, ignore_eos=True)
    out = LLM(engine=engine, tokenizer=tok).generate("abc", params)[0]
    want = expected(tok.encode("abc"), params, 96)
    assert list(out.output_token_ids) == want and out.text == tok.decode(want)


def test_engine_config_validation(tmp_path):
    from tinyvllm.config import EngineConfig

    cfg = EngineConfig(model=tmp_path)
    assert cfg.max_num_seqs == 64 and cfg.kv_block_size == 16 and cfg.prefill_chunk_size == 512
    assert EngineConfig(model=tmp_path, attention_backend="cuda").attention_backend == "cuda"
    assert cfg.kv_cache_dtype == "auto" and (cfg.kv_k_scale, cfg.kv_v_scale) == (1.0, 1.0)
    fp8 = EngineConfig(model=tmp_path, kv_cache_dtype="fp8_e4m3", kv_k_scale=0.5)
    assert fp8.kv_cache_dtype == "fp8_e4m3" and fp8.kv_k_scale == 0.5
    assert cfg.kv_cache_layout == "auto" and cfg.prefill_graph_tokens is None
    tuned = EngineConfig(model=tmp_path, kv_cache_layout="head_major", prefill_graph_tokens=0)
    assert tuned.kv_cache_layout == "head_major" and tuned.prefill_graph_tokens == 0
    bad = [dict(model=tmp_path / "missing"), dict(model=tmp_path, dtype="float32"),
           dict(model=tmp_path, attention_backend="triton"),
           dict(model=tmp_path, gpu_memory_utilization=1.0),
           dict(model=tmp_path, prefill_reserve_tokens=0),
           dict(model=tmp_path, prefill_chunk_size=8192),
           dict(model=tmp_path, max_num_seqs=0),
           dict(model=tmp_path, kv_cache_dtype="int8"),
           dict(model=tmp_path, kv_k_scale=2.0),  # scales need the FP8 layout
           dict(model=tmp_path, kv_cache_dtype="fp8_e4m3", kv_v_scale=0.0),
           dict(model=tmp_path, kv_cache_dtype="fp8_e4m3", kv_k_scale=float("inf")),
           dict(model=tmp_path, kv_cache_layout="slot_major"),
           dict(model=tmp_path, prefill_graph_tokens=-1),
           dict(model=tmp_path, prefill_graph_tokens=512.0)]
    for kw in bad:
        with pytest.raises((ValueError, TypeError)):
            EngineConfig(**kw)
    with pytest.raises(TypeError):
        EngineConfig(model=tmp_path, enforce_eager=1)
