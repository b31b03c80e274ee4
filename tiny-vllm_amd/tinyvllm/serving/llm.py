"""Synchronous facade (reference: tinyvllm/serving/llm.py:12-146)."""
from __future__ import annotations

from collections.abc import Collection, Mapping, Sequence
from dataclasses import dataclass
from typing import Literal

from tinyvllm.config import EngineConfig
from tinyvllm.engine import Engine, GenerateRequest, RequestOutput
from tinyvllm.request import CompletionEvent, RequestStatus, SamplingParams


@dataclass(frozen=True, slots=True)
class TextOutput:
    request_id: int
    text: str
    output_token_ids: tuple[int, ...]
    prompt_token_count: int
    finish_reason: Literal["stop", "length", "cancelled"]

    @property
    def completion_token_count(self) -> int:
        return len(self.output_token_ids)

    @property
    def total_token_count(self) -> int:
        return self.prompt_token_count + self.completion_token_count

    @classmethod
    def from_result(cls, result: RequestOutput | CompletionEvent, text: str,
                    sampling: SamplingParams, eos_token_ids: Collection[int]) -> "TextOutput":
        tokens = result.output_token_ids
        if result.status is RequestStatus.ABORTED:
            reason = "cancelled"
        elif tokens and not sampling.ignore_eos and tokens[-1] in eos_token_ids:
            reason = "stop"
        else:
            reason = "length"
        return cls(result.request_id, text, tokens, result.prompt_token_count, reason)


class LLM:
    """Text in, text out. Build from an EngineConfig (model directory with
    tokenizer), or wrap an existing Engine (token-id use needs no tokenizer)."""

    def __init__(self, config: EngineConfig | None = None, *, engine: Engine | None = None,
                 tokenizer=None) -> None:
        if (config is None) == (engine is None):
            raise ValueError("pass exactly one of config or engine")
        if config is not None:
            from tinyvllm.serving.tokenizer import Tokenizer

            self.tokenizer = Tokenizer(config.model) if tokenizer is None else tokenizer
            self._engine: Engine | None = Engine.from_config(config)
        else:
            self.tokenizer = tokenizer
            self._engine = engine

    def _get_engine(self) -> Engine:
        if self._engine is None:
            raise RuntimeError("LLM is closed")
        return self._engine

    def generate(self, prompts: str | Sequence[str],
                 sampling: SamplingParams | None = None) -> list[TextOutput]:
        self._get_engine()
        if isinstance(prompts, str):
            prompts = (prompts,)
        if not isinstance(prompts, Sequence) or any(not isinstance(p, str) for p in prompts):
            raise TypeError("prompts must be a string or a sequence of strings")
        if self.tokenizer is None:
            raise RuntimeError("text prompts need a tokenizer")
        return self._generate(tuple(self.tokenizer.encode(p) for p in prompts), sampling)

    def generate_token_ids(self, prompts: Sequence[Sequence[int]],
                           sampling: SamplingParams | None = None) -> list[TextOutput]:
        """Token-id prompts; ``text`` is decoded only when a tokenizer exists."""
        return self._generate(tuple(tuple(p) for p in prompts), sampling)

    def chat(self, messages: Sequence[Mapping[str, str]],
             sampling: SamplingParams | None = None, *,
             enable_thinking: bool = False) -> TextOutput:
        self._get_engine()
        if self.tokenizer is None:
            raise RuntimeError("chat needs a tokenizer")
        ids = self.tokenizer.encode_chat(messages, enable_thinking=enable_thinking)
        return self._generate((ids,), sampling)[0]

    def _generate(self, batches, sampling) -> list[TextOutput]:
        engine = self._get_engine()
        sampling = SamplingParams() if sampling is None else sampling
        if not isinstance(sampling, SamplingParams):
            raise TypeError("sampling must be SamplingParams")
        outputs = engine.generate(tuple(GenerateRequest(t, sampling) for t in batches))
        decode = self.tokenizer.decode if self.tokenizer is not None else (lambda _: "")
        return [TextOutput.from_result(o, decode(o.output_token_ids), sampling,
                                       engine.scheduler.eos_token_ids) for o in outputs]

    def close(self) -> None:
        if self._engine is not None:
            self._engine.close()
            self._engine = None

    def __enter__(self) -> "LLM":
        self._get_engine()
        return self

    def __exit__(self, exc_type, exc, tb) -> None:
        try:
            self.close()
        except BaseException:
            if exc is None:
                raise
