"""Async text facade (reference: tinyvllm/serving/async_llm.py:52-214)."""
from __future__ import annotations

from collections.abc import AsyncIterator, Mapping, Sequence
from dataclasses import dataclass

from tinyvllm.async_engine import AsyncEngine
from tinyvllm.config import EngineConfig
from tinyvllm.engine import TokenEvent
from tinyvllm.request import CompletionEvent, SamplingParams
from tinyvllm.serving.llm import TextOutput


@dataclass(frozen=True, slots=True)
class TextDelta:
    request_id: int
    token_id: int
    text: str


class AsyncLLM:
    """One async context; concurrent request streams are supported."""

    def __init__(self, config: EngineConfig | None = None, *, engine_factory=None,
                 tokenizer=None, max_requests: int = 64, max_reserved_tokens: int = 65536,
                 max_buffered_tokens: int = 128) -> None:
        if (config is None) == (engine_factory is None):
            raise ValueError("pass exactly one of config or engine_factory")
        self._config = config
        self._tokenizer = tokenizer
        self._bridge = AsyncEngine(config if config is not None else engine_factory,
                                   max_requests=max_requests,
                                   max_reserved_tokens=max_reserved_tokens,
                                   max_buffered_tokens=max_buffered_tokens)

    @property
    def is_running(self) -> bool:
        return self._bridge.is_running

    async def __aenter__(self) -> "AsyncLLM":
        if self._tokenizer is None and self._config is not None:
            from tinyvllm.serving.tokenizer import Tokenizer

            self._tokenizer = Tokenizer(self._config.model)
        await self._bridge.__aenter__()
        return self

    async def __aexit__(self, exc_type, exc, tb) -> None:
        await self._bridge.__aexit__(exc_type, exc, tb)

    def _decode(self, ids) -> str:
        return self._tokenizer.decode(ids) if self._tokenizer is not None else ""

    async def stream_token_ids(self, prompt_token_ids: Sequence[int],
                               sampling: SamplingParams | None = None
                               ) -> AsyncIterator[TextDelta | TextOutput]:
        sampling = SamplingParams() if sampling is None else sampling
        stream = await self._bridge.submit(prompt_token_ids, sampling)
        async for event in stream:
            if isinstance(event, TokenEvent):
                yield TextDelta(event.request_id, event.token_id, self._decode([event.token_id]))
            elif isinstance(event, CompletionEvent):
                yield TextOutput.from_result(event, self._decode(event.output_token_ids),
                                             sampling, ())

    async def stream(self, prompt: str, sampling: SamplingParams | None = None):
        async for item in self.stream_token_ids(self._tokenizer.encode(prompt), sampling):
            yield item

    async def chat_stream(self, messages: Sequence[Mapping[str, str]],
                          sampling: SamplingParams | None = None, *,
                          enable_thinking: bool = False):
        ids = self._tokenizer.encode_chat(messages, enable_thinking=enable_thinking)
        async for item in self.stream_token_ids(ids, sampling):
            yield item

    async def generate(self, prompt: str, sampling: SamplingParams | None = None) -> TextOutput:
        return await _last(self.stream(prompt, sampling))

    async def generate_token_ids(self, prompt_token_ids: Sequence[int],
                                 sampling: SamplingParams | None = None) -> TextOutput:
        return await _last(self.stream_token_ids(prompt_token_ids, sampling))

    async def chat(self, messages, sampling=None, *, enable_thinking=False) -> TextOutput:
        return await _last(self.chat_stream(messages, sampling,
                                            enable_thinking=enable_thinking))


async def _last(stream):
    result = None
    async for item in stream:
        result = item
    return result
